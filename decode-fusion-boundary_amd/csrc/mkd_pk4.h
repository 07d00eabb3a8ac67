// mkd_pk4.h -- persistent decode kernel with a tagged activation exchange.
//
// Workgroup shape as in k_persistent2: one 512-thread workgroup per compute
// unit, waves 0-3 compute (CW), waves 4-7 stream the upcoming tasks' weight
// rows into an LDS ring with global_load_lds (DW).
//
// Cross-workgroup protocol. Every activation a task hands to other workgroups
// is written as 64-bit words whose high half is a tag,
//     tag(layer) = (epoch + 1) * 32 + layer,
// where `epoch` counts the steps completed on this workspace (read once at
// kernel start, advanced by the step's last task). A consumer loads the words
// it needs with device-coherent loads and re-loads the ones whose tag is not
// yet the expected one: the data is its own ready flag. Producers never drain
// their stores or arrive on counters and consumers never read a counter
// before the data, so a hand-off costs the producer's store reaching the
// memory-side cache plus one polling load. A 64-bit aligned store is
// single-copy atomic, so a word is never seen half-written. The schedule's
// wait/signal fields are not used by this kernel: a task's producers are
// exactly the tasks that write the words it reads.
//
// Every dependency points to a task of an earlier stage (the split-KV merge is
// done by the last split of a (row, head), the LM reduction by the last LM
// slot), and every workgroup runs its tasks in stage order, so the step cannot
// deadlock.
//
// DMA waves decode each instruction once and issue fixed-geometry chunks: a
// chunk is 16 KiB of whole rows (8, 4 or 2 rows for K = 1024, 2048, 3072) and
// each DMA wave issues exactly 4 (or 3 for K = 3072) 1-KiB copies per chunk,
// so "chunk c - D has landed" is the constant wait vmcnt(3 * D).
#pragma once

#include "mkd_persistent.h"

namespace mkd {

constexpr int P4_MAX_ROWS = 32;      // rows of one GEMV task held in the result tile
constexpr int P4_SCR_FLAGS = 64;     // int [0] abort, [1] epoch
constexpr int P4_SCR_RED = 128;      // float [4][MAXB] sums / LM (value, index)
constexpr int P4_SCR_STAGE = 512;   // u32 [2 parities][2 owners][MAXB][2] residual words awaiting publication
constexpr int P4_STAGE_WORDS = 2 * MAXB * 2;
constexpr int P4_SCR_RES = 1024;     // float [P4_MAX_ROWS][MAXB] task results
constexpr int P4_SCR_ATTN = 2048;    // attention scratch (3 KiB used)
// Smallest batch bucket whose K = 1024 GEMVs (QKV, gate/up, LM head) run on
// the matrix cores (smaller ones use v_dot2 chains).
#ifndef MKD_MFMA_MIN_B
#define MKD_MFMA_MIN_B 2
#endif
constexpr int MFMA_MIN_B = MKD_MFMA_MIN_B;
// The same for o_proj and down (K = 2048, 3072: 4 and 2 weight rows per chunk,
// so a tile of 16 x 16 keeps less of its work; measured slower at batch 2).
constexpr int MFMA_MIN_B_WIDE = 4;
#ifndef MKD_MFMA_MIN_B_LM
#define MKD_MFMA_MIN_B_LM MKD_MFMA_MIN_B
#endif
template <int B, int OP>
constexpr bool p4_mfma_op() {
  return OP == MKD_OP_OPROJ || OP == MKD_OP_DOWN ? B >= MFMA_MIN_B_WIDE
         : OP == MKD_OP_LMHEAD                  ? B >= MKD_MFMA_MIN_B_LM
                                                : B >= MFMA_MIN_B;
}
// Activation rows of K = 1024 (H) in LDS are padded by 16 bytes (XS_H bf16 per
// row), so that the MFMA GEMV's reads of 8 rows at one offset hit 8 different
// bank groups.
constexpr int XS_H = H + 8;
// Activation rows of K = 2048 and 3072 are not padded (the batch-4 ring would
// lose a slot): 16-byte piece q of row b is stored at piece q ^ (b mod 8).
__device__ __forceinline__ int xs_piece(int b, int q) { return q ^ (b & 7); }
// float partial sums of the MFMA GEMV (batch >= MFMA_MIN_B): [32 rows][B][4 waves]
// at batch 2 (a result's four wave partials are one 16-byte read for the store
// epilogue: batch 2 -3 us, C5 batch 2 -7), [4 waves][32 rows][B] at batch 4-8
// (where the MFMA tile writes 4 batch rows with one 16-byte store: the other
// layout measured +1 us at batch 4, +2 to +3 us at batch 8),
// after the attention scratch (batch 2, 4: 1, 2 KiB) or in the 4 KiB added at batch 8
template <int B>
constexpr bool p4_part_rows_first() { return B == 2; }
// index of entry (row, b, wave) of the partial tile (row < 32, b < B, wave < 4)
template <int B>
__device__ __forceinline__ size_t p4_part_at(int row, int b, int wave) {
  if constexpr (p4_part_rows_first<B>()) return ((size_t)row * B + b) * PK_CW + wave;
  else return ((size_t)wave * 32 + row) * B + b;
}
template <int B>
constexpr int p4_scr_part() { return B >= 8 ? PK_SCRATCH : 5632; }
static_assert(5632 + 4 * 32 * 4 * 4 <= PK_SCRATCH && P4_SCR_ATTN + 3104 <= 5632, "partial tile overlaps");
static_assert(P4_SCR_RES + 4 * P4_MAX_ROWS * MAXB <= P4_SCR_ATTN, "result tile overlaps");

static_assert(P4_SCR_RED + 2 * 4 * PK_CW * MAXB <= P4_SCR_STAGE && P4_SCR_STAGE + 4 * 2 * P4_STAGE_WORDS <= P4_SCR_RES,
              "staging area overlaps");
static_assert(P4_SCR_ATTN + 6144 <= PK_SCRATCH, "attention scratch too large");

constexpr size_t TW_NONE = ~(size_t)0;

// threadIdx.x through an opaque move: values derived from it inside a task body
// are recomputed per task instead of being hoisted out of the task loop, where
// dozens of per-lane addresses would stay live across every task and spill.
__device__ __forceinline__ int p4_tid() {
  int v;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v) : "v"((int)threadIdx.x));
  return v;
}

// XCD (accelerator complex die) of the executing compute unit: HW_REG_XCC_ID bits [3:0].
__device__ __forceinline__ int p4_xcc_id() {
  return __builtin_amdgcn_s_getreg((20) | (0 << 6) | ((4 - 1) << 11));
}
// Store of a tagged word: device-scope, i.e. write-through to the memory-side cache.
__device__ __forceinline__ void st_tw(uint64_t* p, uint64_t v) { st_co(p, v); }
// Words every workgroup reads have one write-through copy per XCD replica.
// (Words with readers on one XCD only are write-through stores as well: plain
// stores kept in that XCD's L2 measured no faster in the decode step.)
// One replica of a word every workgroup reads. Callers spread the replicas of
// a word over lanes: a store instruction costs the same with 1 or 64 active
// lanes, and a wave with more than 63 stores in flight stalls its issue until
// write-through acknowledgements (~2 us) come back.
__device__ __forceinline__ void st_rep(const Ws& ws, size_t word, int rep, uint64_t v) {
  st_tw(ws.tw(word + (size_t)rep * TW_GROUP), v);
}

// Plain load through a global-address-space pointer. A pointer read from
// memory is generic to the compiler, which would emit a flat load: flat loads
// count against the LDS counter too, so every LDS wait after one also waits
// for the global load.
// (T a scalar type: a struct such as uint2 would be copied through a generic reference)
template <typename T>
__device__ __forceinline__ T ldg(const T* p) {
  typedef __attribute__((address_space(1))) const T global_t;
  return *(global_t*)p;
}
__device__ __forceinline__ uint2 ldg2u(const void* p) {
  const uint64_t v = ldg(reinterpret_cast<const uint64_t*>(p));
  return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
}

__device__ __forceinline__ uint32_t p4_tag(uint32_t epoch, int layer) { return (epoch + 1u) * 32u + (uint32_t)layer; }
__device__ __forceinline__ uint64_t tw_make(uint32_t lo, uint32_t tag) { return (uint64_t)lo | ((uint64_t)tag << 32); }
__device__ __forceinline__ uint32_t tw_tag(uint64_t w) { return (uint32_t)(w >> 32); }

// Compute-wave barrier over an LDS counter with relaxed atomics. The LDS
// executes each wave's operations in issue order, so LDS writes a wave made
// before its increment are in place for any wave that has seen the count;
// unlike a release/acquire barrier it imposes no wait on global memory, so the
// tagged stores of the previous task stay in flight. (Each wave adds 1; the
// value its add returns names the barrier generation.)
struct SyncLds {
  uint32_t* ctr;
  mutable uint32_t gen;  // barriers this wave has entered (every compute wave runs the same sequence)
  __device__ __forceinline__ void operator()() const {
    asm volatile("" ::: "memory");
    // the add needs no returned value: barrier k is complete when the counter
    // (4 adds per barrier) reaches 4 k, and the wave's own add, issued before
    // its first read, is seen by it (LDS operations of a wave execute in order)
    const uint32_t target = ++gen * PK_CW;
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) __builtin_amdgcn_s_sleep(0);
    asm volatile("" ::: "memory");
  }
};

// Compute-wave context (all fields in registers or LDS).
struct P4 {
  Ws ws;
  int rep;          // replica of the all-read buffers this workgroup polls: its XCD's
  uint32_t epoch;
  SyncLds sync;
  int* flags;
  float* red;
  float* res;
  uint16_t* xs;
  uint8_t* attn_smem;
  uint32_t* stage;  // [2][P4_STAGE_WORDS] residual words of a task's owners, [owner][b][2]
  int par;          // staging buffer of the current task, alternating over the tasks that
                    // stage (QKV, GATEUP): a task reads its buffer after its last barrier,
                    // and the next task to write that buffer comes after another staging
                    // task, behind that task's barriers.
  uint64_t* trp;    // this task's trace record (debug builds with MKD_TRACE_POLL)
  int task;         // index of the current task in this workgroup's row
  float* part;      // [4 waves][32 rows][B] partial sums of the MFMA GEMV (batch >= MFMA_MIN_B)
};

#if defined(MKD_TRACE_POLL) || defined(MKD_TRACE_BARRIER)
constexpr int P4_TR_STRIDE = 8;  // debug records: slots 4.. hold points inside the prologue
#else
constexpr int P4_TR_STRIDE = 4;
#endif
// Debug: wave-maximum time stamp in slot k of the task's trace record.
__device__ __forceinline__ void p4_trace_at(const P4& c, int k) {
#ifdef MKD_TRACE_POLL
  if (c.trp != nullptr && (threadIdx.x & 63) == 0)
    atomicMax(reinterpret_cast<unsigned long long*>(c.trp + k), (unsigned long long)wall_clock64());
#else
  (void)c; (void)k;
#endif
}
// Debug: time at which the task's first dependency poll completed (trace slot 2).
__device__ __forceinline__ void p4_trace_poll(const P4& c) {
#ifdef MKD_TRACE_POLL
  if (c.trp != nullptr && (threadIdx.x & 63) == 0)  // the last of the four waves
    atomicMax(reinterpret_cast<unsigned long long*>(c.trp + 2), (unsigned long long)wall_clock64());
#else
  (void)c;
#endif
}

// First round of a poll: issue the loads (returned in a[]). Issuing it before
// a task's other loads matters: loads complete in issue order, so a check of
// a[] then waits only for loads issued before it.
// Two adjacent tagged words (16-byte aligned) with one 16-byte buffer load at
// device scope (sc1, as ld_co); each word keeps its own tag, so a pair seen
// half written is polled again.
struct PairAddr {
  __amdgpu_buffer_rsrc_t r;
  uint32_t off;  // bytes
};
__device__ __forceinline__ __amdgpu_buffer_rsrc_t pair_rsrc(const uint64_t* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint64_t*>(base), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void ld_co2(PairAddr pa, uint64_t& lo, uint64_t& hi) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 q = __builtin_amdgcn_raw_buffer_load_b128(pa.r, pa.off, 0, 16 /* sc1 */);
  lo = (uint64_t)q.x | ((uint64_t)q.y << 32);
  hi = (uint64_t)q.z | ((uint64_t)q.w << 32);
}
// One round of N word loads; PAIRS: words 2j and 2j + 1 are adjacent and come
// from one 16-byte load.
template <int N, bool PAIRS, class Addr>
__device__ __forceinline__ void poll_round(Addr addr, uint64_t (&a)[N]) {
  if constexpr (PAIRS) {
    static_assert(N % 2 == 0, "whole pairs");
#pragma unroll
    for (int k = 0; k < N; k += 2) ld_co2(addr(k), a[k], a[k + 1]);
  } else {
#pragma unroll
    for (int k = 0; k < N; k++) a[k] = ld_co(addr(k));
  }
}
template <int N, class Addr>
__device__ __forceinline__ void poll_issue(Addr addr, uint64_t (&a)[N]) {
  poll_round<N, false>(addr, a);
}
// Check the first round and keep polling until every word carries `tag`
// (one round in flight: measured no slower than two, with half the traffic;
// re-polling only one word while the others are missing measured slower).
template <int N, bool PAIRS = false, class Addr>
__device__ __forceinline__ bool poll_finish(Addr addr, uint64_t (&a)[N], uint64_t (&v)[N], uint32_t tag,
                                            const Ws& ws) {
  // The device error word and the clock are read only by a poll that has
  // already spun 62 rounds: the error word is loaded ahead of a round's polls
  // and examined with their results, so no round waits for a load of its own
  // beyond the polls (a poll that succeeds early costs nothing extra).
  uint32_t err = 0u;
  uint64_t t0 = 0;
  for (uint32_t spin = 0;; spin++) {
    // A lane re-polls all of its words until one round finds every tag
    // current (a word once current stays so until this task is done: its
    // next writer depends on this task's outputs). Per-word pending masks
    // cost a branch per word and, inlined at every poll site, put the
    // batch-8 kernel over the instruction cache (batch 8 -29 us, C4 -34 us,
    // measured without them). Every word is examined on every round: a load
    // the compiler sees unconsumed on some path makes it wait for all of the
    // wave's memory operations before that register is next written.
    bool all = true;
#pragma unroll
    for (int k = 0; k < N; k++) all = all && tw_tag(a[k]) == tag;
    if (all) {
#pragma unroll
      for (int k = 0; k < N; k++) v[k] = a[k];
      asm volatile("" ::"v"(err));  // (loaded before the polls just examined)
      return true;
    }
    if ((spin & 63u) == 63u) {
      if (err != 0u) return false;
      const uint64_t now = wall_clock64();
      if (t0 == 0) t0 = now;
      else if (now - t0 > 400000000ull) {  // 4 s at 100 MHz
        st_co(ws.line(CTR_ERR), ERR_TIMEOUT);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(0);  // (longer pauses measured slower at every batch size; 0 vs 1: -1 to -3 us)
    if ((spin & 63u) == 62u) err = ld_co(ws.line(CTR_ERR));
    poll_round<N, PAIRS>(addr, a);
  }
}
// Load N tagged words (addr(k), k < N) and spin until each carries `tag`.
// Returns false on a timeout (which it reports) or when another workgroup
// has reported an error.
template <int N, bool PAIRS = false, class Addr>
__device__ __forceinline__ bool poll_tagged(Addr addr, uint64_t (&v)[N], uint32_t tag, const Ws& ws) {
  uint64_t a[N];
  poll_round<N, PAIRS>(addr, a);
  return poll_finish<N, PAIRS>(addr, a, v, tag, ws);
}

// Compute-wave barrier that also agrees on an abort over the four waves.
// flags[0] holds the index of the first task that failed in any wave (INT_MAX
// while none has): a wave that already runs a later task may record its failure
// before a slower wave reads the flag for this task, and comparing indices keeps
// that later failure from aborting this task in the slow wave only. Every wave
// thus aborts at the same task and all waves run the same sequence of barriers.
__device__ __forceinline__ void p4_fail(const P4& c) {
  __hip_atomic_fetch_min(c.flags, c.task, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ bool p4_agree(const P4& c, bool ok) {
  if (!ok) p4_fail(c);
  c.sync();
  return c.flags[0] > c.task;
}

constexpr int largest_divisor_le8(int n) {
  return n % 8 == 0 ? 8 : (n % 6 == 0 ? 6 : (n % 4 == 0 ? 4 : (n % 2 == 0 ? 2 : 1)));
}

// B rows of a tagged [MAXB][K/2] activation into xs (bf16 [B][K]).
template <int B, int K>
__device__ __forceinline__ bool p4_stage_copy(const P4& c, size_t base, uint32_t tag) {
  constexpr int PER = B * (K / 2) / 256;  // words per thread
  // Words polled as one group (one round in flight per group). Batch 8 polls
  // the most words per hand-over: down input 48 words per thread in two groups
  // of 24, o_proj input 32 in two of 16 (measured against 12 / 8: batch 8
  // -21 us, C4 -24 us; one group of 48 or 32: +150 / +65 us, register bound).
  // Batch 4's down input in two groups of 12 (with the paired loads below:
  // -4.6 us against three of 8); o_proj's in one of 16 measured +19 us and
  // larger groups at batch 2 no faster.
  constexpr int NB = K == 3072 && B >= 4 ? 3 * B : (B >= 8 && K == 2048 ? 16 : largest_divisor_le8(PER));
  static_assert(PER % NB == 0, "whole groups");
  const int t = p4_tid();
  const uint64_t* src = c.ws.tw(base + (size_t)c.rep * TW_GROUP);
  uint32_t* dst = reinterpret_cast<uint32_t*>(c.xs);
  bool ok = true;
  if constexpr (B >= 2) {
    // words polled in pairs: word slot w of this thread is element w % 2 of pair
    // t + 256 (w / 2) of [B][K/2], one 16-byte load per pair (half the load
    // instructions of a round: batch 8 -30 us, C4 -28, C5 batch 8 -34, batch 4
    // -9; batch 1, with 4-6 words per thread, measured +4 us and keeps words)
    constexpr int WPR2 = K / 1024;  // 256-pair blocks per row
#pragma unroll
    for (int k0 = 0; k0 < PER; k0 += NB) {
      uint64_t v[NB];
      const __amdgpu_buffer_rsrc_t rs = pair_rsrc(src);
      ok = ok && poll_tagged<NB, true>(
                     [&](int k) { const int w = k0 + k; return PairAddr{rs, (uint32_t)(16 * (t + 256 * (w >> 1)))}; },
                     v, tag, c.ws);
      if (k0 == 0) p4_trace_poll(c);
#pragma unroll
      for (int k = 0; k < NB; k++) {
        const int w = k0 + k, m = w >> 1, b = m / WPR2, ww = 512 * (m % WPR2) + 2 * t + (w & 1);
        dst[b * (K / 2) + xs_piece(b, ww >> 2) * 4 + (ww & 3)] = (uint32_t)v[k];
      }
    }
  } else {
#pragma unroll
    for (int k0 = 0; k0 < PER; k0 += NB) {
      uint64_t v[NB];
      ok = ok && poll_tagged<NB>([&](int k) { return src + t + 256 * (k0 + k); }, v, tag, c.ws);
      if (k0 == 0) p4_trace_poll(c);
#pragma unroll
      for (int k = 0; k < NB; k++) {
        // word t + 256 m of [B][K/2]: row m / WPR, word 256 (m % WPR) + t of it,
        // its 16-byte piece XOR-swizzled by the row (xs_piece)
        constexpr int WPR = K / 2 / 256;
        const int m = k0 + k, b = m / WPR, ww = 256 * (m % WPR) + t;
        dst[b * (K / 2) + xs_piece(b, ww >> 2) * 4 + (ww & 3)] = (uint32_t)v[k];
      }
    }
  }
  return p4_agree(c, ok);
}

// This thread's 4 features of the residual stream, bf16, per row (words
// pack(f0, f1), pack(f2, f3)): what its last RMSNorm prologue computed. Every
// workgroup computes the whole residual in each RMSNorm prologue, so the next
// one needs only the new hidden rows; the published residual words are polled
// only by the first RMSNorm task of a launch (valid still false).
// Gate/up task word a2 flag (tagged kernel): publish the residual, read by
// the next layer's QKV prologue in the next launch (the last layer of a layer
// segment that is not the step's last, and every layer when each stage is a
// launch of its own).
constexpr int GATEUP_PUBLISH_RES = 1;
// QKV task word a2 flag: publish the residual after the input add, read by the
// same layer's gate/up prologue in a later launch (one launch per stage).
constexpr int QKV_PUBLISH_RES = 1;
template <int B>
struct ResKeep {
  uint32_t w[B][2];
  bool valid;
};

// Residual add + RMSNorm of B rows into xs (rounding as stage_norm in mkd_tasks.h).
// from_embed: the rows are the embedding rows of input_ids (layer 0).
// Otherwise s = hidden + residual: the hidden rows from a tagged [MAXB][H/2]
// buffer, the residual from rk (or, first in a launch, from a tagged buffer).
// Threads res_first .. res_first + res_n - 1 stage their 4 features of bf16(s),
// the next residual, published at the end of the task (p4_residual_word).
template <int B>
__device__ __forceinline__ bool p4_stage_norm(const MkdStepDesc& d, const P4& c, bool from_embed, size_t hid,
                                              size_t resid, uint32_t tag_in, const uint16_t* nw, int res_first,
                                              int res_n, ResKeep<B>& rk) {
  const int t = p4_tid(), wave = t >> 6, lane = t & 63;
  const int k0 = t * 4;  // features k0..k0+3 = words 2t, 2t+1 of each row
  const bool res_owner = res_first <= t && t < res_first + res_n;
  float s[B][4];
  bool ok = true;
  auto load_nw = [&]() {
    return ldg2u(nw + k0);
  };
  uint2 wv;
  if (from_embed) {
    wv = load_nw();
#pragma unroll
    for (int b = 0; b < B; b++) {
      int64_t id = b < d.rows ? d.input_ids[b] : 0;
      if (id < 0 || id >= V) {
        if (t == 0) st_co(c.ws.line(CTR_ERR), ERR_BAD_INPUT);
        id = 0;
      }
      const uint2 e = *reinterpret_cast<const uint2*>(d.embed + (size_t)id * H + k0);
      s[b][0] = bf_lo(e.x); s[b][1] = bf_hi(e.x); s[b][2] = bf_lo(e.y); s[b][3] = bf_hi(e.y);
    }
  } else if (rk.valid) {
    // hidden words only: rows in groups of GH (2 words each)
    constexpr int GH = B < 4 ? B : 4;  // (8 at batch 8: +54 us, measured)
    // this thread's words 2 t, 2 t + 1 of each row: one 16-byte load per row
    // (batch 1 -3 us, batch 4 -7, batch 8 -13, C4 -13, C5 batch 8 -14)
    const __amdgpu_buffer_rsrc_t hrs = pair_rsrc(c.ws.tw(hid + (size_t)c.rep * TW_GROUP));
    auto haddr = [&](int b0) {
      return [=](int k) { return PairAddr{hrs, (uint32_t)(16 * ((b0 + (k >> 1)) * (H / 4) + t))}; };
    };
    constexpr bool PR = true;
    uint64_t first[2 * GH];
    poll_round<2 * GH, PR>(haddr(0), first);  // before any other load of this task
    wv = load_nw();
#pragma unroll
    for (int b0 = 0; b0 < B; b0 += GH) {
      uint64_t v[2 * GH];
      if (b0 == 0) {
        ok = poll_finish<2 * GH, PR>(haddr(0), first, v, tag_in, c.ws);
        p4_trace_poll(c);
      } else {
        ok = ok && poll_tagged<2 * GH, PR>(haddr(b0), v, tag_in, c.ws);
      }
#pragma unroll
      for (int g = 0; g < GH; g++) {
        const int b = b0 + g;
        const uint32_t h0 = (uint32_t)v[2 * g], h1 = (uint32_t)v[2 * g + 1];
        const uint32_t r0 = rk.w[b][0], r1 = rk.w[b][1];
        s[b][0] = bf_lo(h0) + bf_lo(r0); s[b][1] = bf_hi(h0) + bf_hi(r0);
        s[b][2] = bf_lo(h1) + bf_lo(r1); s[b][3] = bf_hi(h1) + bf_hi(r1);
      }
    }
  } else {
    // rows in groups of G (two rows at a time keeps the in-flight poll registers small)
    constexpr int G = B < 2 ? B : 2;
    auto addr = [&](int b0) {
      return [=](int k) {
        return c.ws.tw(((k & 2) ? resid : hid) + (size_t)c.rep * TW_GROUP + (size_t)(b0 + (k >> 2)) * (H / 2) + 2 * t +
                       (k & 1));
      };
    };
    uint64_t first[4 * G];
    poll_issue<4 * G>(addr(0), first);  // before any other load of this task
    wv = load_nw();
#pragma unroll
    for (int b0 = 0; b0 < B; b0 += G) {
      uint64_t v[4 * G];
      if (b0 == 0) {
        ok = poll_finish<4 * G>(addr(0), first, v, tag_in, c.ws);
        p4_trace_poll(c);
      } else {
        ok = ok && poll_tagged<4 * G>(addr(b0), v, tag_in, c.ws);
      }
#pragma unroll
      for (int g = 0; g < G; g++) {
        const int b = b0 + g;
        const uint32_t h0 = (uint32_t)v[4 * g], h1 = (uint32_t)v[4 * g + 1];
        const uint32_t r0 = (uint32_t)v[4 * g + 2], r1 = (uint32_t)v[4 * g + 3];
        s[b][0] = bf_lo(h0) + bf_lo(r0); s[b][1] = bf_hi(h0) + bf_hi(r0);
        s[b][2] = bf_lo(h1) + bf_lo(r1); s[b][3] = bf_hi(h1) + bf_hi(r1);
      }
    }
  }
  // the new residual, for the next RMSNorm prologue of this launch
#pragma unroll
  for (int b = 0; b < B; b++) {
    rk.w[b][0] = pack_bf2(s[b][0], s[b][1]);
    rk.w[b][1] = pack_bf2(s[b][2], s[b][3]);
  }
  rk.valid = true;
  const float w4[4] = {bf_lo(wv.x), bf_hi(wv.x), bf_lo(wv.y), bf_hi(wv.y)};
  // consumed here, before the abort return below: a load left unconsumed on
  // that path would make the compiler wait for all memory operations at the
  // start of every later chunk loop
  asm volatile("" ::"v"(w4[0]), "v"(w4[1]), "v"(w4[2]), "v"(w4[3]));
  // this thread's 4 features of the new residual, when this task owns them:
  // staged in LDS as words [owner][b][2]
  if (res_owner) {
    uint32_t* stage = c.stage + c.par * P4_STAGE_WORDS;
#pragma unroll
    for (int b = 0; b < B; b++) {
      stage[((t - res_first) * B + b) * 2] = rk.w[b][0];
      stage[((t - res_first) * B + b) * 2 + 1] = rk.w[b][1];
    }
  }
  if constexpr (B == 1) {
    const float ss = wave_sum(s[0][0] * s[0][0] + s[0][1] * s[0][1] + s[0][2] * s[0][2] + s[0][3] * s[0][3]);
    if (lane == 0) c.red[wave] = ss;  // [row][wave]
  } else {
    // all rows' sums of squares in one reduction (lane b ends with row b's)
    float sq[B];
#pragma unroll
    for (int b = 0; b < B; b++) sq[b] = s[b][0] * s[b][0] + s[b][1] * s[b][1] + s[b][2] * s[b][2] + s[b][3] * s[b][3];
    const float ss = rows_wave_sum<B>(sq);
    if (lane < B) c.red[lane * PK_CW + wave] = ss;  // [row][wave]
  }
  p4_trace_at(c, 4);
  if (!p4_agree(c, ok)) return false;
  p4_trace_at(c, 5);
  // lane b < B reads row b's four wave sums with one 16-byte LDS read and
  // computes its scale; the rows' scales are then read back lane by lane (a
  // uniform read per row of each wave sum made the compiler chain 4 B LDS
  // round trips, 1.3 us at batch 8)
  const float4 wsum = *reinterpret_cast<const float4*>(c.red + PK_CW * (lane & (B - 1)));
  const float r_lane =
      __builtin_amdgcn_rsqf((((wsum.x + wsum.y) + wsum.z) + wsum.w) * (1.0f / H) + EPS);  // v_rsq_f32 (1 ulp)
#pragma unroll
  for (int b = 0; b < B; b++) {
    const float r = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(r_lane), b));
    // bf16(bf16(s * r) * w), pairwise through the packed conversion
    const uint32_t n01 = pack_bf2(s[b][0] * r, s[b][1] * r), n23 = pack_bf2(s[b][2] * r, s[b][3] * r);
    *reinterpret_cast<uint2*>(c.xs + (size_t)b * XS_H + k0) =
        make_uint2(pack_bf2(bf_lo(n01) * w4[0], bf_hi(n01) * w4[1]), pack_bf2(bf_lo(n23) * w4[2], bf_hi(n23) * w4[3]));
  }
  c.sync();
  return true;
}

// Sums of each 32-lane half of a wave: the DPP butterfly of wave_sum without
// its last (row_bcast31) step; lane 31 ends with lanes 0-31, lane 63 with 32-63.
__device__ __forceinline__ float half_sums(float v) {
  v += dpp_mov<0xB1>(v, 0.f);
  v += dpp_mov<0x4E>(v, 0.f);
  v += dpp_mov<0x141>(v, 0.f);
  v += dpp_mov<0x140>(v, 0.f);
  v += dpp_mov<0x142, 0xA>(v, 0.f);
  return v;
}
__device__ __forceinline__ float lane_value(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// One LDS weight chunk (row-major rows of K bf16) times the B activations in
// xs, over the 4 compute waves with 64 bytes of weights per lane, so that every
// wave's loads, dot products and reductions form one short chain:
//   K = 1024 (8 rows):  wave w -> rows 2w (lanes 0-31) and 2w+1 (lanes 32-63)
//   K = 2048 (4 rows):  wave w -> row w
//   K = 3072 (2 rows):  wave w -> half (w & 1) of row w >> 1; out(2 * row + half)
// out(i, acc) gets the wave-uniform sums acc[B]; only rows < nr are reported.
// The lane's activation operands come from an X source: get(b, c) is operand c
// (8 bf16) of row b in the layout above.
template <int K>
struct GemvShape {
  static constexpr int PARTS = K == 3072 ? 2 : 1;             // waves per row (K > 1024)
  static constexpr int CPL = K == 1024 ? 4 : K / PARTS / 512;  // operands (uint4) per lane
};
// Weight rows in a ring slot: the DMA stores 16-byte piece q of row r of its
// chunk (64 pieces per 1-KiB unit) at position (q - r) mod 64 of its unit, so
// that reads of one piece of up to 8 rows hit different bank groups. Index (in
// pieces) of logical piece q of row r:
__device__ __forceinline__ int wpiece(int r, int q) { return (q & ~63) + (((q & 63) - (r & 7)) & 63); }

typedef __bf16 p4_bf16x8 __attribute__((ext_vector_type(8)));
typedef float p4_f32x4 __attribute__((ext_vector_type(4)));
// One chunk (RPC = 8 / 4 / 2 weight rows of K = 1024 / 2048 / 3072) on the
// matrix cores (p4_mfma_op: batch >= 2, o_proj and down >= 4): wave w multiplies K quarter
// [K w / 4, K (w + 1) / 4) of the chunk's rows with K / 128 v_mfma_f32_16x16x32_bf16
// (A = the B activation rows, M = 16; B = the weight rows, N = 16; rows
// beyond B and RPC repeat real ones and their results are dropped), in two
// accumulator chains. Lane l supplies row / column l % 16 and K elements
// 8 (l / 16) .. + 7 of each 32-wide step; result lane l holds column l % 16,
// rows 4 (l / 16) .. + 3. The wave's partial sums go to entry (row, b, w) of
// the partial tile (p4_part_at; part offset by the chunk's first row); the
// store epilogue adds the four waves' partials in a fixed order.
template <int B, int K>
__device__ __forceinline__ void chunk_mfma(const uint8_t* slot, const uint4* x4, float* part) {
  static_assert(B >= 1 && B <= 8, "MFMA GEMV for batch 1 to 8");
  constexpr int RPC = K == 1024 ? 8 : (K == 2048 ? 4 : 2);
  constexpr int STEPS = K / 128;      // 32-wide K steps per wave
  constexpr int PPW = K / 32;         // 16-byte pieces per wave's K quarter
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, kg = lane >> 4, r = n & (RPC - 1), b = n & (B - 1);
  const uint4* wrow = reinterpret_cast<const uint4*>(slot + (size_t)r * (K * 2));
  const uint4* xrow = x4 + (size_t)b * (K == 1024 ? XS_H / 8 : K / 8);
  p4_f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s0 = 0; s0 < STEPS; s0 += 8) {
    uint4 wv[8], xv[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
      const int q = PPW * wave + 4 * (s0 + s) + kg;  // 8-element piece of K
      wv[s] = wrow[wpiece(r, q)];
      xv[s] = xrow[K == 1024 ? q : xs_piece(b, q)];
    }
#pragma unroll
    for (int s = 0; s < 8; s += 2) {
      a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(p4_bf16x8, xv[s]), __builtin_bit_cast(p4_bf16x8, wv[s]),
                                                   a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(p4_bf16x8, xv[s + 1]),
                                                   __builtin_bit_cast(p4_bf16x8, wv[s + 1]), a1, 0, 0, 0);
    }
  }
  const p4_f32x4 acc = a0 + a1;
  if constexpr (!p4_part_rows_first<B>()) {
    if (n < RPC && 4 * kg < B)
      *reinterpret_cast<float4*>(part + p4_part_at<B>(n, 4 * kg, wave)) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  } else if constexpr (B >= 4) {
    if (n < RPC && 4 * kg < B) {
#pragma unroll
      for (int m = 0; m < 4; m++) part[p4_part_at<B>(n, 4 * kg + m, wave)] = acc[m];
    }
  } else if constexpr (B == 2) {
    if (n < RPC && kg == 0) {
      part[p4_part_at<B>(n, 0, wave)] = acc[0];
      part[p4_part_at<B>(n, 1, wave)] = acc[1];
    }
  } else {
    if (n < RPC && kg == 0) part[p4_part_at<B>(n, 0, wave)] = acc[0];
  }
}
// x[lane] + x[lane ^ 32] and x[lane] + x[lane ^ 16] on every lane (gfx950
// permlane swaps: one VALU op instead of an LDS crossbar round trip).
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// MFMA GEMV of one chunk at batch 4 and 8 on the 4x4x4 block MFMA (16 blocks
// of 4 x 4 x 4 per instruction): a block is an 8-element K piece (two
// instructions, its low and high halves), A its 4 batch rows of x, B its 4
// weight rows, so every operand byte read from LDS is used (the 16x16x32 form
// reads the chunk's few weight rows and the batch rows many times over:
// measured LDS-bound at batch 8). Wave w takes K quarter w in 128-element steps
// (lane 4 blk + i: piece blk of the step, batch row 4 h + i of x, weight row
// 4 g + i), the 16 blocks' sums are added across lanes and written to
// entry (row, b, w) of the partial tile as chunk_mfma does. Rows past the chunk's
// (K = 3072: 2 of a group's 4) repeat its rows and are not written.
template <int B, int K>
__device__ __forceinline__ void chunk_mfma4(const uint8_t* slot, const uint4* x4, float* part) {
  static_assert(B == 4 || B == 8, "4x4x4 GEMV for batch 4 and 8");
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  constexpr int RPC = K == 1024 ? 8 : (K == 2048 ? 4 : 2);
  constexpr int NG = RPC >= 4 ? RPC / 4 : 1;  // groups of 4 weight rows
  constexpr int NH = B / 4;                   // groups of 4 batch rows
  constexpr int STEPS = K / 4 / 128;          // 128-element steps of the wave's K quarter
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int blk = lane >> 2, i = lane & 3;
  p4_f32x4 acc[NG][NH];
#pragma unroll
  for (int g = 0; g < NG; g++)
#pragma unroll
    for (int h = 0; h < NH; h++) acc[g][h] = p4_f32x4{0.f, 0.f, 0.f, 0.f};
  const uint4* wrow[NG];
#pragma unroll
  for (int g = 0; g < NG; g++) wrow[g] = reinterpret_cast<const uint4*>(slot + (size_t)((4 * g + i) & (RPC - 1)) * (K * 2));
#pragma unroll
  for (int s = 0; s < STEPS; s++) {
    const int q = (K / 32) * wave + 16 * s + blk;  // 16-byte piece of the row
    uint4 wv[NG], xv[NH];
#pragma unroll
    for (int g = 0; g < NG; g++) wv[g] = wrow[g][wpiece((4 * g + i) & (RPC - 1), q)];
#pragma unroll
    for (int h = 0; h < NH; h++) {
      const int b = 4 * h + i;
      xv[h] = x4[(size_t)b * (K == 1024 ? XS_H / 8 : K / 8) + (K == 1024 ? q : xs_piece(b, q))];
    }
#pragma unroll
    for (int g = 0; g < NG; g++)
#pragma unroll
      for (int h = 0; h < NH; h++) {
        const uint2 wl = make_uint2(wv[g].x, wv[g].y), wh = make_uint2(wv[g].z, wv[g].w);
        const uint2 xl = make_uint2(xv[h].x, xv[h].y), xh = make_uint2(xv[h].z, xv[h].w);
        acc[g][h] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, xl), __builtin_bit_cast(s16x4, wl),
                                                           acc[g][h], 0, 0, 0);
        acc[g][h] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4, xh), __builtin_bit_cast(s16x4, wh),
                                                           acc[g][h], 0, 0, 0);
      }
  }
  // sum over the 16 blocks (lane bits 2-5) of the NV = 4 NH values of each
  // lane, as a transpose-reduce: lane bits 2 .. 1 + log2 NV each halve the
  // values a lane keeps (it adds its partner's half), the remaining bits are
  // summed whole; lane l then holds value j = (l >> 2) % NV, batch row j, of
  // weight row l % 4 (12 cross-lane moves at batch 8 instead of 32)
  static_assert(NG == 1, "chunk_mfma4 serves K >= 2048: at most 4 rows per chunk");
  constexpr int NV = 4 * NH;
  float v[NV];
#pragma unroll
  for (int h = 0; h < NH; h++)
#pragma unroll
    for (int m = 0; m < 4; m++) v[4 * h + m] = acc[0][h][m];
  {  // lane bit 2: partner lane ^ 4 is lane + 4 (row_shl 4) or lane - 4 (row_shr 4); both
     // moves run with every lane active (the empty asm keeps each out of a branch)
    const bool p = lane & 4;
#pragma unroll
    for (int j = 0; j < NV / 2; j++) {
      const float keep = p ? v[2 * j + 1] : v[2 * j], send = p ? v[2 * j] : v[2 * j + 1];
      float up = dpp_mov<0x104>(send, 0.f), down = dpp_mov<0x114>(send, 0.f);
      asm volatile("" : "+v"(up), "+v"(down));
      v[j] = keep + (p ? down : up);
    }
  }
  {  // lane bit 3: row_ror 8
    const bool p = lane & 8;
#pragma unroll
    for (int j = 0; j < NV / 4; j++) {
      const float keep = p ? v[2 * j + 1] : v[2 * j], send = p ? v[2 * j] : v[2 * j + 1];
      v[j] = keep + dpp_mov<0x128>(send, 0.f);
    }
  }
  float t = v[0];
  if constexpr (NV == 8) {  // lane bit 4 halves once more: the partner's value through the permlane16 swap
    const bool p = lane & 16;
    const float keep = p ? v[1] : v[0], send = p ? v[0] : v[1];
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(send), __float_as_uint(send), false, false);
    t = keep + __uint_as_float(p ? r[0] : r[1]);
  } else {
    t = xor16_sum(t);
  }
  t = xor32_sum(t);
  const int row = lane & 3, j = (lane >> 2) & (NV - 1);
  if (row < RPC && lane < 4 * NV) part[p4_part_at<B>(row, j, wave)] = t;
}
// GEMV chunks on chunk_mfma4: K = 2048 and 3072 (o_proj, down: 4 and 2 rows
// per chunk) at batch 4 and 8. Measured per chunk at batch 8: down 1.06 ->
// 0.86 us, o_proj 0.80 -> 0.65 us; but K = 1024 (8 rows per chunk, where the
// 16x16x32 form wastes less) 0.5 -> 0.9 us, its block sums costing more than
// the operand reads saved. Step: batch 4 693 -> 662 us, C5 batch 4 912 -> 868 us.
template <int B, int K>
constexpr bool p4_mfma4() {
  return B >= 4 && K >= 2048;
}
// Chunk-result sink of the MFMA GEMV (p4_chunks passes it the chunk's rows).
struct PartSink {
  float* part;
};

// LM head on the matrix cores (batch >= MFMA_MIN_B): wave w takes the task's chunks
// j = w, w + 4, ..., each whole (8 vocabulary rows x K = 1024: 32 MFMAs in two
// accumulator chains), so no partial sums cross waves. Lane l (column n = l % 16,
// row n % 8; result rows b = 4 (l / 16) + i) keeps a running greedy argmax of
// its (row, b) logits: bf16-rounded value, then the lowest vocabulary index.
struct LmLane {
  float v[4];
  int i[4];
};
struct LmSink {
  LmLane* best;
  uint16_t* logits;  // optional bf16 logits [batch rows][V]
  int logit_rows;    // batch rows with logits
  int row0, rows;    // first vocabulary row and row count of the task
};
template <int B>
__device__ __forceinline__ void chunk_lm_mfma(const uint8_t* slot, const uint4* x4, int row, bool valid, LmLane& lb,
                                              uint16_t* logits, int logit_rows) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, kg = lane >> 4, r = n & 7;
  const uint4* wrow = reinterpret_cast<const uint4*>(slot + (size_t)r * (H * 2));
  const uint4* xrow = x4 + (size_t)(n & (B - 1)) * (XS_H / 8);
  p4_f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s0 = 0; s0 < 32; s0 += 8) {
    uint4 wv[8], xv[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
      const int q = 4 * (s0 + s) + kg;  // 8-element piece of K
      wv[s] = wrow[wpiece(r, q)];
      xv[s] = xrow[q];
    }
#pragma unroll
    for (int s = 0; s < 8; s += 2) {
      a0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(p4_bf16x8, xv[s]), __builtin_bit_cast(p4_bf16x8, wv[s]),
                                                   a0, 0, 0, 0);
      a1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(p4_bf16x8, xv[s + 1]),
                                                   __builtin_bit_cast(p4_bf16x8, wv[s + 1]), a1, 0, 0, 0);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float acc = a0[i] + a1[i];
    const float v = valid ? round_bf(acc) : -INFINITY;
    const bool better = lm_later_better(v, lb.v[i]);  // (this lane's rows come in increasing order)
    lb.v[i] = better ? v : lb.v[i];
    lb.i[i] = better ? row : lb.i[i];
    const int b = 4 * kg + i;
    if (logits != nullptr && valid && n < 8 && b < B && b < logit_rows) logits[(size_t)b * V + row] = (uint16_t)f2bf(acc);
  }
}

// X source: the activations in LDS (bf16 [B][K]). (Polling them straight into
// registers instead, each wave all of its operands, measured slower: four
// times the polling loads outweigh the staging copy and its barrier.)
template <int K>
struct XLds {
  const uint4* x4;
  __device__ __forceinline__ uint4 get(int b, int c) const {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if constexpr (K == 1024) return x4[b * (XS_H / 8) + c * 32 + (lane & 31)];
    constexpr int CPL = GemvShape<K>::CPL;
    return x4[b * (K / 8) + xs_piece(b, (wave % GemvShape<K>::PARTS) * (CPL * 64) + c * 64 + lane)];
  }
};
template <int B, int K, class X, class Out>
__device__ __forceinline__ void chunk_gemv4(const uint8_t* slot, int nr, const X& xsrc, Out out) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if constexpr (K == 1024) {
    const int half = lane >> 5, l = lane & 31, row = 2 * wave + half;
    const uint4* w4 = reinterpret_cast<const uint4*>(slot + (size_t)row * (K * 2));
    uint4 wv[4];
#pragma unroll
    for (int c = 0; c < 4; c++) wv[c] = w4[wpiece(row, c * 32 + l)];
    float acc[B];
#pragma unroll
    for (int b = 0; b < B; b++) {
      uint4 xv[4];  // all of this row's operand loads before its dot products
#pragma unroll
      for (int c = 0; c < 4; c++) xv[c] = xsrc.get(b, c);
      acc[b] = 0.f;
#pragma unroll
      for (int c = 0; c < 4; c++) acc[b] = dot8(wv[c], xv[c], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = half_sums(acc[b]);
    float lo[B], hi[B];
#pragma unroll
    for (int b = 0; b < B; b++) { lo[b] = lane_value(acc[b], 31); hi[b] = lane_value(acc[b], 63); }
    if (2 * wave < nr) out(2 * wave, lo);
    if (2 * wave + 1 < nr) out(2 * wave + 1, hi);
  } else {
    constexpr int PARTS = K == 2048 ? 1 : 2;      // waves per row
    constexpr int CPL = K / PARTS / 512;          // uint4 per lane: 4 or 3
    const int row = wave / PARTS, part = wave % PARTS;
    const uint4* w4 = reinterpret_cast<const uint4*>(slot + (size_t)row * (K * 2));
    uint4 wv[CPL];
#pragma unroll
    for (int c = 0; c < CPL; c++) wv[c] = w4[wpiece(row, part * (CPL * 64) + c * 64 + lane)];
    float acc[B];
#pragma unroll
    for (int b = 0; b < B; b++) {
      uint4 xv[CPL];
#pragma unroll
      for (int c = 0; c < CPL; c++) xv[c] = xsrc.get(b, c);
      acc[b] = 0.f;
#pragma unroll
      for (int c = 0; c < CPL; c++) acc[b] = dot8(wv[c], xv[c], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = wave_sum(acc[b]);
    if (row < nr) out(PARTS * row + part, acc);
  }
}

// Weight pointer of the layer table through scalar loads.
__device__ __forceinline__ const uint16_t* p4_wptr(const MkdStepDesc& d, int layer, int which) {
  return reinterpret_cast<const uint16_t*>(as_const(d.layer_ptrs)[layer * MKD_LAYER_PTRS + which]);
}

__device__ __forceinline__ int p4_rows(const Inst& w) {
  if (w.op == MKD_OP_GATEUP) return 2 * w.a1;
  if (w.op == MKD_OP_QKV || w.op == MKD_OP_OPROJ || w.op == MKD_OP_DOWN || w.op == MKD_OP_LMHEAD) return w.a1;
  return 0;
}
__device__ __forceinline__ int p4_chunks(const Inst& w) {
  const int rows = p4_rows(w);
  const int rpc = w.op == MKD_OP_OPROJ ? 4 : (w.op == MKD_OP_DOWN ? 2 : 8);
  return (rows + rpc - 1) / rpc;
}

// The new residual is published by the tasks of the stage that computes it,
// each the 4-feature slices of the threads whose index maps into its row range
// (QKV: 16 rows per thread index, GATEUP: 12 channels), so every slice has
// exactly one writer and no task carries the whole vector's stores.
struct ResRange {
  int first, n;  // owner threads first .. first + n - 1
};
template <int F>  // rows (channels) per thread index
__device__ __forceinline__ ResRange p4_res_range(const Inst& w) {
  const int first = (w.a0 + F - 1) / F;
  return ResRange{first, (w.a0 + w.a1 + F - 1) / F - first};
}

template <int B>
__device__ __forceinline__ bool p4_prologue(const MkdStepDesc& d, const P4& c, const Inst& w, ResKeep<B>& rk) {
  const int layer = w.layer;
  const uint32_t tag = p4_tag(c.epoch, layer);
  const int t = p4_tid();
  (void)t;
  if constexpr (B < 4) {
    // batch 1-2: one inlined p4_stage_norm per call site (the code fits the
    // instruction cache; shared, it measured slower at batch 1)
    switch (w.op) {
      case MKD_OP_QKV: {
        const uint16_t* nw = p4_wptr(d, layer, MKD_W_LN_IN);
        const ResRange r = p4_res_range<QKV_N / 256>(w);
        const int rn = (w.a2 & QKV_PUBLISH_RES) ? r.n : 0;
        if (layer == 0) return p4_stage_norm<B>(d, c, true, 0, 0, 0, nw, r.first, rn, rk);
        return p4_stage_norm<B>(d, c, false, TW_DOWN, TW_RES2, p4_tag(c.epoch, layer - 1), nw, r.first, rn, rk);
      }
      case MKD_OP_GATEUP: {
        const ResRange r = p4_res_range<I / 256>(w);
        return p4_stage_norm<B>(d, c, false, TW_O, TW_RES1, tag, p4_wptr(d, layer, MKD_W_LN_POST), r.first,
                                (w.a2 & GATEUP_PUBLISH_RES) ? r.n : 0, rk);
      }
      case MKD_OP_OPROJ: return p4_stage_copy<B, QS>(c, TW_ATTN, tag);
      case MKD_OP_DOWN: return p4_stage_copy<B, I>(c, TW_ACT, tag);
      case MKD_OP_LMHEAD:
        return p4_stage_norm<B>(d, c, false, TW_DOWN, TW_RES2, p4_tag(c.epoch, d.num_layers - 1), d.final_norm, 0, 0, rk);
      default: return true;
    }
  }
  if (w.op == MKD_OP_OPROJ) return p4_stage_copy<B, QS>(c, TW_ATTN, tag);
  if (w.op == MKD_OP_DOWN) return p4_stage_copy<B, I>(c, TW_ACT, tag);
  if (w.op != MKD_OP_QKV && w.op != MKD_OP_GATEUP && w.op != MKD_OP_LMHEAD) return true;
  // batch 4-8: the three RMSNorm prologues share one inlined copy of
  // p4_stage_norm, their operands selected here (a copy per call site would
  // triple its code: the batch-8 kernel was over the instruction cache)
  // (the residual after QKV is consumed by the gate/up prologue of the same
  // layer: published only when that prologue runs in a later launch)
  bool from_embed = false;
  size_t hid = TW_DOWN, resid = TW_RES2;
  uint32_t tag_in = tag;
  const uint16_t* nw;
  int res_first = 0, res_n = 0;
  if (w.op == MKD_OP_QKV) {
    nw = p4_wptr(d, layer, MKD_W_LN_IN);
    const ResRange r = p4_res_range<QKV_N / 256>(w);
    res_first = r.first;
    res_n = (w.a2 & QKV_PUBLISH_RES) ? r.n : 0;
    from_embed = layer == 0;
    tag_in = p4_tag(c.epoch, layer - 1);
  } else if (w.op == MKD_OP_GATEUP) {
    nw = p4_wptr(d, layer, MKD_W_LN_POST);
    const ResRange r = p4_res_range<I / 256>(w);
    res_first = r.first;
    res_n = (w.a2 & GATEUP_PUBLISH_RES) ? r.n : 0;
    hid = TW_O;
    resid = TW_RES1;
  } else {
    nw = d.final_norm;
    tag_in = p4_tag(c.epoch, d.num_layers - 1);
  }
  return p4_stage_norm<B>(d, c, from_embed, hid, resid, tag_in, nw, res_first, res_n, rk);
}

// Chunks are handed from the DMA waves to the compute waves in groups of G
// consecutive chunks (counted over the whole instruction row), one barrier per
// group: the chunks of a layer task are usually one group that landed during
// the task's dependency wait, so the task runs without a per-chunk hand-over.
// 2G <= NS: while the compute waves read group g, the DMA waves can already
// hold group g + 1 in the remaining slots.
template <int NS>
struct P4G {
  // Groups of 2 (measured against min(NS / 2, 4), i.e. 4 at batch 1-4 and 3 at
  // batch 8): a smaller group lets the DMA waves refill sooner, keeping more
  // chunks in flight while the compute waves work (batch 1 499 -> 482 us,
  // batch 8 858 -> 835, C5 batch 8 1161 -> 1105); groups of 1 (a barrier per
  // chunk) were slower at batch 2-8.
  static constexpr int G = 2;
  static_assert(2 * G <= NS, "two groups fit the ring");
};

// The chunk loop of one GEMV task (the op is fixed for the whole loop).
// out(i, j, acc): result i of chunk j (see chunk_gemv4 for i).
template <int B, int K, int NS, class X, class Out>
__device__ __forceinline__ void p4_chunks(uint8_t* ring, int cc, int nch, int rows, bool aborted, uint64_t* tr,
                                          const X& xsrc, Out out, uint64_t* dbg_chunks = nullptr) {
  (void)dbg_chunks;
  constexpr int RPC = K == 1024 ? 8 : (K == 2048 ? 4 : 2);
  uint8_t* slot = ring + (cc % NS) * SLOT_BYTES;
  uint8_t* const ring_end = ring + NS * SLOT_BYTES;
  // (no global store inside the loop: a loop with stores makes the compiler
  // wait for all of the wave's outstanding memory operations before it, the
  // previous task's write-through stores included)
#ifndef MKD_TRACE_POLL
  if (tr != nullptr && threadIdx.x == 0) tr[2] = wall_clock64();
#endif
  for (int j = 0; j < nch; j++) {
#if defined(MKD_TRACE_POLL) || defined(MKD_TRACE_BARRIER)
    if (j == 0 && tr != nullptr && (threadIdx.x & 63) == 0)
      atomicMax(reinterpret_cast<unsigned long long*>(tr + 6), (unsigned long long)wall_clock64());
#endif
    if ((cc + j) % P4G<NS>::G == 0) raw_barrier();  // group of G chunks handed over
#ifdef MKD_TRACE_CHUNKS
    // debug: chunk release and compute-end times after the task trace ([grid][512][2])
    uint64_t* ct = dbg_chunks == nullptr ? nullptr : dbg_chunks + ((size_t)blockIdx.x * 512 + ((cc + j) & 511)) * 2;
    if (ct != nullptr && threadIdx.x == 0) ct[0] = wall_clock64();
#endif
    if constexpr (std::is_same<Out, PartSink>::value) {
      if (!aborted) {
        if constexpr (p4_mfma4<B, K>()) chunk_mfma4<B, K>(slot, xsrc.x4, out.part + p4_part_at<B>(j * RPC, 0, 0));
        else chunk_mfma<B, K>(slot, xsrc.x4, out.part + p4_part_at<B>(j * RPC, 0, 0));
      }
    } else if constexpr (std::is_same<Out, LmSink>::value) {
      // (every wave still takes each hand-over barrier above)
      const int wave = threadIdx.x >> 6, r = (threadIdx.x & 15) & 7;
      if (!aborted && (j & 3) == wave)
        chunk_lm_mfma<B>(slot, xsrc.x4, out.row0 + j * RPC + r, j * RPC + r < out.rows, *out.best, out.logits,
                         out.logit_rows);
    } else {
      if (!aborted) chunk_gemv4<B, K>(slot, min(RPC, rows - j * RPC), xsrc, [&](int i, const float* acc) { out(i, j, acc); });
    }
#if defined(MKD_TRACE_POLL) || defined(MKD_TRACE_BARRIER)
    if (j == 0 && tr != nullptr && (threadIdx.x & 63) == 0)  // debug: first chunk computed
      atomicMax(reinterpret_cast<unsigned long long*>(tr + 7), (unsigned long long)wall_clock64());
#endif
#ifdef MKD_TRACE_CHUNKS
    if (ct != nullptr && threadIdx.x == 0) ct[1] = wall_clock64();
#endif
    slot += SLOT_BYTES;
    if (slot == ring_end) slot = ring;
  }
}

// Running greedy argmax of the LM head, per row, wave-uniform (updated with
// selects, no divergent branches).
template <int B>
struct LmArg {
  float v[B];
  int i[B];
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int b = 0; b < B; b++) { v[b] = -INFINITY; i[b] = 0x7fffffff; }
  }
};

// All chunks of GEMV task w (results into the tile; LM: argmax into best).
template <int B, int NS>
__device__ __forceinline__ void p4_task_chunks(const MkdStepDesc& d, const P4& c, const Inst& w, uint8_t* ring, int cc,
                                               int nch, bool aborted, uint64_t* tr, LmArg<B>& best,
                                               uint64_t* dbg = nullptr) {
  const int lane = threadIdx.x & 63;
  const int rows = p4_rows(w);
  float* res = c.res;
  auto to_res = [&](int rpc, int per_row) {
    return [=](int i, int j, const float* acc) {
      if (lane < B) res[(j * rpc * per_row + i) * MAXB + lane] = pick_lane<B>(acc, lane);
    };
  };
  const uint4* x4 = reinterpret_cast<const uint4*>(c.xs);
  switch (w.op) {
    case MKD_OP_QKV:
    case MKD_OP_GATEUP:
      if constexpr (p4_mfma_op<B, MKD_OP_QKV>()) p4_chunks<B, H, NS>(ring, cc, nch, rows, aborted, tr, XLds<H>{x4}, PartSink{c.part}, dbg);
      else p4_chunks<B, H, NS>(ring, cc, nch, rows, aborted, tr, XLds<H>{x4}, to_res(8, 1), dbg);
      break;
    case MKD_OP_OPROJ:
      if constexpr (p4_mfma_op<B, MKD_OP_OPROJ>()) p4_chunks<B, QS, NS>(ring, cc, nch, rows, aborted, tr, XLds<QS>{x4}, PartSink{c.part}, dbg);
      else p4_chunks<B, QS, NS>(ring, cc, nch, rows, aborted, tr, XLds<QS>{x4}, to_res(4, 1), dbg);
      break;
    // DOWN (v_dot2 chains): two half-row partials per row, result tile entries 2 * row + half
    case MKD_OP_DOWN:
      if constexpr (p4_mfma_op<B, MKD_OP_DOWN>()) p4_chunks<B, I, NS>(ring, cc, nch, rows, aborted, tr, XLds<I>{x4}, PartSink{c.part}, dbg);
      else p4_chunks<B, I, NS>(ring, cc, nch, rows, aborted, tr, XLds<I>{x4}, to_res(2, 2), dbg);
      break;
    case MKD_OP_LMHEAD: {
      uint16_t* logits = d.out_logits;
      const int a0 = w.a0;
      if constexpr (p4_mfma_op<B, MKD_OP_LMHEAD>()) {
        LmLane lb;
#pragma unroll
        for (int i = 0; i < 4; i++) { lb.v[i] = -INFINITY; lb.i[i] = 0x7fffffff; }
        p4_chunks<B, H, NS>(ring, cc, nch, rows, aborted, tr, XLds<H>{x4}, LmSink{&lb, logits, d.rows, a0, rows}, dbg);
        // per batch row b = 4 (l / 16) + i: (max, lowest index) over the 16 lanes
        // of group l / 16, then broadcast from lane 16 (b / 4)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float v = lb.v[i];
          int ix = lb.i[i];
#pragma unroll
          for (int o = 1; o < 16; o <<= 1) {
            const float v2 = __shfl_xor(v, o, 64);
            const int i2 = __shfl_xor(ix, o, 64);
            const bool better = lm_better(v2, i2, v, ix);
            v = better ? v2 : v;
            ix = better ? i2 : ix;
          }
#pragma unroll
          for (int b = i; b < B; b += 4) {
            best.v[b] = lane_value(v, 16 * (b / 4));
            best.i[b] = __builtin_amdgcn_readlane(ix, 16 * (b / 4));
          }
        }
        break;
      }
      p4_chunks<B, H, NS>(ring, cc, nch, rows, aborted, tr, XLds<H>{x4}, [&](int r, int j, const float* acc) {
        const int row = a0 + j * 8 + r;
#pragma unroll
        for (int b = 0; b < B; b++) {
          const float v = round_bf(acc[b]);
          const bool better = lm_later_better(v, best.v[b]);  // (rows in increasing order)
          best.v[b] = better ? v : best.v[b];
          best.i[b] = better ? row : best.i[b];
        }
        if (logits != nullptr && lane < B && lane < d.rows)
          logits[(size_t)lane * V + row] = (uint16_t)f2bf(pick_lane<B>(acc, lane));
      }, dbg);
      break;
    }
    default: break;
  }
}

constexpr int ilog2(int n) { return n <= 1 ? 0 : 1 + ilog2(n / 2); }
// Replicas of the all-read tagged words this batch's kernel writes (the
// workspace holds TW_NREP); workgroups on XCD x read replica x % p4_nrep.
// Measured per batch (us per step with 8 / 4 / 2 / 1 replicas): batch 1 479 /
// 481 / 492 / 516; batch 2 528 / 525 / 530 (C5 647 / 644 / 650); batch 4 610 /
// 603 / 602 / 614; batch 8 758 / 727 / 723 / 723 (C4 867 / 833 / 831 / 828):
// from batch 2 on the replica stores cost more than spreading the reads over
// more copies saves.
template <int B>
constexpr int p4_nrep() {
  return B >= 8 ? 1 : (B >= 4 ? 2 : (B == 2 ? 4 : TW_NREP));
}

// The residual words this task's owner threads staged in its prologue: one
// store per (word, replica), at most one per thread (at most 2 owners x 8 rows
// x 2 words x 8 replicas), spread over the waves. Read from LDS before the
// task's output stores and issued after them: the residual is read two stages
// later, and an LDS read behind the output stores made the compiler wait for
// their write acknowledgements first.
struct ResWord {
  uint64_t* q;  // null: this thread has no residual store
  uint64_t v;
};
template <int B, int F>
__device__ __forceinline__ ResWord p4_residual_word(const P4& c, const Inst& w, size_t base, uint32_t tag) {
  const ResRange r = p4_res_range<F>(w);
  const uint32_t* stage = c.stage + c.par * P4_STAGE_WORDS;
  const int t = p4_tid();
  constexpr int LR = ilog2(p4_nrep<B>()), LB = ilog2(B);
  static_assert(2 * B * 2 * p4_nrep<B>() <= PK_CW * 64, "one residual store per thread");
  const int e = (t & 63) * PK_CW + (t >> 6);
  if (e >= (r.n << (LB + 1 + LR))) return ResWord{nullptr, 0};
  const int k = e >> LR, o = k >> (LB + 1), b = (k >> 1) & (B - 1);
  const size_t word = base + (size_t)b * (H / 2) + 2 * (r.first + o) + (k & 1);
  return ResWord{c.ws.tw(word + (size_t)(e & (p4_nrep<B>() - 1)) * TW_GROUP), tw_make(stage[k], tag)};
}

// Publish one GEMV task's rows as tagged bf16 pairs. Entry e = (pair i, row b,
// replica r) with r in the low bits, then b, then i, so the entries of a task
// are the prefix e < pairs * B * replicas and all index math is shifts: this
// epilogue sits on the step's critical path, where each instruction of a
// single wave costs several cycles.
template <int B, int OP>
__device__ __forceinline__ void p4_store_op(const P4& c, const Inst& w) {
  constexpr int LR = OP == MKD_OP_QKV ? 0 : ilog2(p4_nrep<B>());  // QKV words have one reader XCD
  constexpr int LB = ilog2(B);
  static_assert((1 << LB) == B, "batch bucket is a power of two");
  constexpr uint32_t STRIDE = OP == MKD_OP_QKV ? QKV_N / 2 : (OP == MKD_OP_GATEUP ? I / 2 : H / 2);
  constexpr uint32_t BASE = OP == MKD_OP_QKV ? TW_QKV
                            : OP == MKD_OP_OPROJ ? TW_O
                            : OP == MKD_OP_GATEUP ? TW_ACT : TW_DOWN;
  const uint32_t tag = p4_tag(c.epoch, w.layer);
  const int t = p4_tid();
  // store f goes to wave f % 4: vmcnt also counts stores, so a wave with
  // write-through stores in flight waits for their acknowledgement at its next
  // load; spreading them keeps any one wave from lagging the others
  const int fo = (t & 63) * PK_CW + (t >> 6);
  const int n = (w.a1 >> 1) << (LB + LR);  // (channel or row) pairs x rows x replicas
  uint8_t* const twb = reinterpret_cast<uint8_t*>(c.ws.tw(BASE + (uint32_t)(w.a0 >> 1)));
  ResWord rw{nullptr, 0};
  if (OP == MKD_OP_GATEUP && (w.a2 & GATEUP_PUBLISH_RES)) rw = p4_residual_word<B, I / 256>(c, w, TW_RES2, tag);
  if (OP == MKD_OP_QKV && (w.a2 & QKV_PUBLISH_RES)) rw = p4_residual_word<B, QKV_N / 256>(c, w, TW_RES1, tag);
  for (int e = fo; e < n; e += PK_CW * 64) {
    const int r = e & ((1 << LR) - 1), b = (e >> LR) & (B - 1), i = e >> (LR + LB);
    float v0, v1;
    // result of task row `row`, batch row b: one entry of the tile, or (MFMA
    // GEMV) the four waves' partial sums, added in a fixed order
    auto R = [&](int row) -> float {
      if constexpr (p4_mfma_op<B, OP>()) {
        if constexpr (p4_part_rows_first<B>()) {
          const float4 q = *reinterpret_cast<const float4*>(c.part + p4_part_at<B>(row, b, 0));
          return (q.x + q.y) + (q.z + q.w);  // waves 0-3, one 16-byte read
        } else {
          const float* p = c.part + p4_part_at<B>(row, b, 0);
          return (p[0] + p[32 * B]) + (p[64 * B] + p[96 * B]);
        }
      } else {
        return c.res[row * MAXB + b];
      }
    };
    if (OP == MKD_OP_GATEUP) {
      float h[2];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const float g = round_bf(R(4 * i + 2 * k));
        const float u = round_bf(R(4 * i + 2 * k + 1));
        h[k] = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;  // v_exp_f32, v_rcp_f32 (1 ulp each)
      }
      v0 = h[0]; v1 = h[1];
    } else if (OP == MKD_OP_DOWN && p4_mfma_op<B, MKD_OP_DOWN>()) {
      v0 = R(2 * i);
      v1 = R(2 * i + 1);
    } else if (OP == MKD_OP_DOWN) {  // (v_dot2 chains) rows arrive as two half-row partials
      v0 = c.res[(4 * i) * MAXB + b] + c.res[(4 * i + 1) * MAXB + b];
      v1 = c.res[(4 * i + 2) * MAXB + b] + c.res[(4 * i + 3) * MAXB + b];
    } else {
      v0 = R(2 * i);
      v1 = R(2 * i + 1);
    }
    const uint64_t v = tw_make(pack_bf2(v0, v1), tag);
    const uint32_t off = ((uint32_t)r * (uint32_t)TW_GROUP + (uint32_t)b * STRIDE + (uint32_t)i) * 8u;
    uint64_t* q = reinterpret_cast<uint64_t*>(twb + off);
    st_tw(q, v);
  }
  if (rw.q != nullptr) st_tw(rw.q, rw.v);
}
static_assert(TW_WORDS * 8 < (1ull << 32), "tagged offsets are 32-bit");

template <int B>
__device__ __forceinline__ void p4_store(const P4& c, const Inst& w, uint64_t* dbg_st = nullptr) {
  (void)dbg_st;
#ifdef MKD_TRACE_CHUNKS
  if (dbg_st != nullptr && (threadIdx.x & 63) == 0) dbg_st[threadIdx.x >> 6] = wall_clock64();
#endif
  c.sync();  // the result tile is complete
#ifdef MKD_TRACE_CHUNKS
  if (dbg_st != nullptr && (threadIdx.x & 63) == 0) dbg_st[4 + (threadIdx.x >> 6)] = wall_clock64();
#endif
  switch (w.op) {
    case MKD_OP_QKV: p4_store_op<B, MKD_OP_QKV>(c, w); break;
    case MKD_OP_OPROJ: p4_store_op<B, MKD_OP_OPROJ>(c, w); break;
    case MKD_OP_GATEUP: p4_store_op<B, MKD_OP_GATEUP>(c, w); break;
    case MKD_OP_DOWN: p4_store_op<B, MKD_OP_DOWN>(c, w); break;
    default: break;
  }
}

// LM-head task end: publish this slot's (max, first index) per row; the last
// slot also reduces all slots to the greedy tokens and advances the epoch.
template <int B>
__device__ __forceinline__ bool p4_lm_finish(const MkdStepDesc& d, const P4& c, const Inst& w, const LmArg<B>& best) {
  const int t = p4_tid(), wave = t >> 6, lane = t & 63;
  const uint32_t tag = p4_tag(c.epoch, w.layer);
  float* bv = c.red;
  int* bi = reinterpret_cast<int*>(c.red + PK_CW * MAXB);
  c.sync();  // red is free (earlier users are past a barrier)
  if (lane < B) {
    float v = best.v[0]; int i = best.i[0];
#pragma unroll
    for (int b = 1; b < B; b++) { v = lane == b ? best.v[b] : v; i = lane == b ? best.i[b] : i; }
    bv[wave * MAXB + lane] = v;
    bi[wave * MAXB + lane] = i;
  }
  c.sync();
  const int slot = w.a2;
  if (t < B) {
    float v = bv[t]; int i = bi[t];
    for (int ww = 1; ww < PK_CW; ww++) {
      const float v2 = bv[ww * MAXB + t]; const int i2 = bi[ww * MAXB + t];
      if (lm_better(v2, i2, v, i)) { v = v2; i = i2; }
    }
    uint64_t* o = c.ws.tw(TW_LM + ((size_t)slot * MAXB + t) * 2);
    st_co(o, tw_make(__float_as_uint(v), tag));
    st_co(o + 1, tw_make((uint32_t)i, tag));
  }
  if (slot != d.lm_slots - 1) return true;
  bool ok = true;
  for (int b = wave; b < d.rows; b += PK_CW) {
    float v = -INFINITY; int i = 0x7fffffff;
    // four slots per lane and poll round (slots lane, lane + 64, ...; one round
    // for the usual 256 slots instead of four back to back); past the slot
    // count a lane re-reads its first slot, which changes no (max, first index)
    for (int s0 = lane; s0 < d.lm_slots; s0 += 256) {
      uint64_t e[8];
      ok = ok && poll_tagged<8>(
                     [&](int k) {
                       const int s = s0 + 64 * (k >> 1) < d.lm_slots ? s0 + 64 * (k >> 1) : s0;
                       return c.ws.tw(TW_LM + ((size_t)s * MAXB + b) * 2 + (k & 1));
                     },
                     e, tag, c.ws);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float v2 = __uint_as_float((uint32_t)e[2 * q]); const int i2 = (int)(uint32_t)e[2 * q + 1];
        if (lm_better(v2, i2, v, i)) { v = v2; i = i2; }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float v2 = __shfl_xor(v, o, 64); const int i2 = __shfl_xor(i, o, 64);
      if (lm_better(v2, i2, v, i)) { v = v2; i = i2; }
    }
    if (lane == 0) {
      const int tok = i == 0x7fffffff ? 0 : i;  // (no candidate at all: token 0)
      d.out_tokens[b] = tok;
      if (d.flags & MKD_FLAG_ADVANCE) { d.input_ids[b] = tok; d.cache_seqlens[b] += 1; }
    }
  }
  if (!p4_agree(c, ok)) return false;
  if (t == 0) st_co(c.ws.line(CTR_EPOCH), c.epoch + 1u);
  return true;
}

// Positions of one ATTN task: split `split` of `nsplit` covers [p_begin, p_end)
// of the row's pos + 1 positions (whole KV chunks but the last split's end); the
// cached ones, [p_begin, c_end), come in KV chunks of 32 positions that the DMA
// waves stage in the LDS ring; the token's own position (pos) is not in the
// cache yet and comes from this step's k and v. Computed identically by the
// DMA waves (chunk count) and the compute waves.
constexpr int KV_CHUNK = 32;  // positions per KV chunk: 32 K rows (8 KiB) + 32 V rows (8 KiB)
struct AttnGeo {
  int pos, p_begin, p_end, c_end, nch;
  int ns;     // splits this row uses (<= the schedule's): the last of them merges
  bool live;  // a row of this step with a valid position
};
// Fewest KV chunks per split: the schedule's split count is sized for the
// longest context of the prepared steps or from the block table's width
// (whole pages); a row's context in this step may need fewer. A split past
// the row's count has no positions and does nothing, and split ns - 1 merges
// (batch 2, contexts 1-65 scheduled with 2 splits: 594 -> 552 us per step).
template <int B>
constexpr int p4_split_min_chunks() {
  // batch 2 only (0: none). Batch 1's host rule already fits short contexts
  // (one split below ~170 positions) and batch 4-8 take one split below two
  // pages; there the added code alone measured +4 to +5 us.
  return B == 2 ? 2 : 0;
}
__device__ __forceinline__ AttnGeo attn_geo(int rows, int b, int pos_in, int page_stride, int bs, int split,
                                            int nsplit, int min_chunks) {
  AttnGeo g;
  g.live = b < rows && pos_in >= 0 && pos_in < MKD_MAX_POSITION && pos_in / bs < page_stride;
  g.pos = g.live ? pos_in : 0;
  const int ctx = g.pos + 1;
  g.ns = nsplit;
  if (min_chunks > 0) {
    nsplit = max(1, min(nsplit, ((ctx + KV_CHUNK - 1) / KV_CHUNK + min_chunks - 1) / min_chunks));
    g.ns = nsplit;
    if (split >= nsplit) {  // no positions for this split
      g.p_begin = g.p_end = g.c_end = ctx;
      g.nch = 0;
      return g;
    }
  }
  // the row's KV_CHUNK-position chunks dealt out evenly, the first nck % nsplit
  // splits taking one more (measured against equal spans rounded up to 64
  // positions: C4 batch 8 1057 -> 1029 us, C5 batch 8 1220 -> 1202 us; moving
  // 1-3 chunks off the last split, which also merges, measured no faster)
  const int nck = (ctx + KV_CHUNK - 1) / KV_CHUNK;
  const int q = nck / nsplit, r = nck % nsplit;
  const int c0 = split * q + min(split, r);
  g.p_begin = c0 * KV_CHUNK;
  g.p_end = split == nsplit - 1 ? ctx : min(ctx, (c0 + q + (split < r ? 1 : 0)) * KV_CHUNK);
  g.c_end = min(g.p_end, g.pos);
  g.nch = g.c_end > g.p_begin ? (g.c_end - g.p_begin + KV_CHUNK - 1) / KV_CHUNK : 0;
  return g;
}
// LDS layout of a KV chunk: K row of chunk position p (0..31) at p * 256 bytes,
// its 16-byte piece q at slot ((q + (p & 1)) & 15) (consecutive positions
// shifted by one piece, so the scores' reads, 8 positions x 8 pieces per
// instruction, spread over all banks); V row p at 8192 + p * 256, unswizzled.
__device__ __forceinline__ int kv_kpiece(int p, int q) { return p * 256 + ((q + (p & 1)) & 15) * 16; }
constexpr int KV_V_OFF = KV_CHUNK * 256;

// Sums and maxima over the lanes of a wave that hold one value per group of 8
// lanes (lanes 8p .. 8p + 7 replicate value p): xor 8 within a row of 16 lanes
// (row_ror:8), then xor 16 and xor 32 (permlane swaps).
__device__ __forceinline__ float sum_over_8_groups(float x) {
  x += dpp_mov<0x128>(x, 0.f);
  return xor32_sum(xor16_sum(x));
}
__device__ __forceinline__ float max_over_8_groups(float x) {
  x = fmaxf(x, dpp_mov<0x128>(x, -INFINITY));
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Sum over the 8 lanes 8p .. 8p + 7 (quad swaps, then the other quad by half-row mirror).
__device__ __forceinline__ float sum_within_8(float x) {
  x += dpp_mov<0xB1>(x, 0.f);
  x += dpp_mov<0x4E>(x, 0.f);
  return x + dpp_mov<0x141>(x, 0.f);
}

// The hand-over barriers of a task's nch chunks without using them (a task
// skipped after an abort: the DMA waves issue and hand over its chunks anyway).
template <int NS>
__device__ __forceinline__ void p4_skip_chunks(int cc, int nch) {
  for (int j = 0; j < nch; j++)
    if ((cc + j) % P4G<NS>::G == 0) raw_barrier();
}
// KV chunk count of an ATTN task (as the DMA waves compute it).
template <int B>
__device__ __forceinline__ int p4_attn_chunks(const MkdStepDesc& d, const Inst& w) {
  const int b = (w.a0 & 63) / NKV;  // (a0 = b * 8 + h plus query-head flags from bit 6)
  const int pos_in = b < d.rows ? as_const(d.cache_seqlens)[b] : 0;
  return attn_geo(d.rows, b, pos_in, d.page_stride, d.block_size, w.a1, w.a2, p4_split_min_chunks<B>()).nch;
}

// Softmax in base 2: scores scaled by hd^-0.5 * log2(e), so that every
// exponential is one v_exp_f32 (2^x, 1 ulp); maxima and partial log-sums
// (the split partials included) are in the same base-2 domain.
constexpr float SCALE2 = ATTN_SCALE * 1.4426950408889634f;
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// ATTN task of the tagged kernel: row b, KV head h, split `split` of nsplit of
// the row's positions, and either one query head (task word a0 = b * 8 + h,
// plus ATTN_ONE_HEAD and g * ATTN_QHEAD for head 2h + g) or both (PAIR: a0 =
// b * 8 + h). One-head tasks put the two query heads of a KV head on two
// workgroups of the KV head's XCD, which halves each task's chain of dependent
// instructions (the faster form while the step is latency-bound: short
// contexts, small batches); a PAIR task reads each K/V chunk once for both
// heads, half the cache traffic of the one-head form (the faster form once the
// cache reads bound the step: long contexts at batch 4 and 8). PAIR: wave 3
// polls, normalizes and ropes the second head's q; each chunk's scores and
// P * V are computed for both heads from the same K and V reads.
// The task's cached K/V arrive as KV chunks in the LDS ring (staged by the DMA
// waves like weight rows), so the compute waves issue no cache loads of their
// own: their only global loads before the q/k/v poll are the norm weights and
// the RoPE row, issued first, and the poll's rounds queue behind nothing else.
// After the poll (wave 0: q, wave 1: k, wave 2: v): q/k RMSNorm + RoPE in
// registers, the new token's K/V written to its cache slot (by the g = 0 task,
// split 0, of an active row) straight from registers, then online softmax over
// the chunks, each chunk's 32 positions split over the four waves (wave w:
// positions 8w .. 8w + 7):
//   scores: lane (position p = lane >> 3, dims 16 (lane & 7) ..) dots 16 dims of
//           K with q, summed over the 8 lanes of the position;
//   P * V:  lane (dims 2 lane, 2 lane + 1) over the wave's 8 positions, with the
//           probabilities read from the lanes that hold them.
// The four waves are merged at the end; the token's own K/V (not yet in the
// cache when this task reads it) comes from LDS. The last split folds in the
// other splits' tagged partials. nch returns the task's KV chunk count.
// Last split of an attention task: wave w folds the partials (num, max, sum:
// the same unnormalized base-2 form as its own accumulators, for this lane's
// dims 2 lane, 2 lane + 1) of splits w, w + 4, w + 8, w + 12 into its own, SPR
// splits per poll round.
__device__ __forceinline__ void p4_fold_splits(const Ws ws, size_t pbase, int nsplit, int g, uint32_t tag, float& m0,
                                               float& l0, float& a00, float& a01, bool& ok) {
  const int wave = p4_tid() >> 6, lane = threadIdx.x & 63;
  constexpr int SPW = (MAXS - 1 + PK_CW - 1) / PK_CW;  // splits per wave
  constexpr int SPR = 2;                                // splits per poll round
#pragma unroll
  for (int q0 = 0; q0 < SPW; q0 += SPR) {
    if (wave + PK_CW * q0 >= nsplit - 1) break;
    uint64_t e[4 * SPR];
    // (entries past the last split repeat its words)
    const bool okp = poll_tagged<4 * SPR>(
        [&](int k) {
          const int sp = min(wave + PK_CW * (q0 + (k >> 2)), nsplit - 2), f = k & 3;
          const size_t ps = pbase + (size_t)sp * PART_STRIDE;
          return ws.tw(ps + (f < 2 ? (size_t)(g * HD + 2 * lane + f) : (size_t)(GROUP * HD + (f - 2) * GROUP + g)));
        },
        e, tag, ws);
    ok = ok && okp;
#pragma unroll
    for (int q = 0; q < SPR; q++) {
      if (wave + PK_CW * (q0 + q) >= nsplit - 1) break;
      const float ms = __uint_as_float((uint32_t)e[4 * q + 2]);
      if (ms == -INFINITY) continue;  // an empty split
      const float nm = fmaxf(m0, ms);
      const float sa = m0 == -INFINITY ? 0.f : ex2(m0 - nm), sb = ex2(ms - nm);
      a00 = a00 * sa + __uint_as_float((uint32_t)e[4 * q]) * sb;
      a01 = a01 * sa + __uint_as_float((uint32_t)e[4 * q + 1]) * sb;
      l0 = l0 * sa + __uint_as_float((uint32_t)e[4 * q + 3]) * sb;
      m0 = nm;
    }
  }
}
constexpr int ATTN_QHEAD = 64, ATTN_ONE_HEAD = 128;  // task word a0 flags (b * 8 + h < 64)
constexpr int P4_PAIR_MIN_B = 4;  // smallest batch whose kernel runs tasks of both query heads
template <int B, int NS, bool PAIR>
__device__ __forceinline__ bool p4_attn(const MkdStepDesc& d, const P4& c, int layer, int a0, int split, int nsplit,
                                        uint64_t* tr, uint8_t* ring, int cc, int& nch) {
  const int t = p4_tid(), wave = t >> 6, lane = t & 63;
  const uint32_t tag = p4_tag(c.epoch, layer);
  constexpr int NQH = PAIR ? GROUP : 1;  // query heads of this task
  const int bh = a0 & (ATTN_QHEAD - 1), g = (!PAIR && (a0 & ATTN_QHEAD)) ? 1 : 0;
  const int b = bh / NKV, h = bh % NKV, qh = GROUP * h + g;  // (PAIR: qh and qh + 1)
  const int bs = d.block_size;
  const int pos_in = b < d.rows ? as_const(d.cache_seqlens)[b] : 0;
  const AttnGeo ag = attn_geo(d.rows, b, pos_in, d.page_stride, bs, split, nsplit, p4_split_min_chunks<B>());
  nch = ag.nch;
  if (b < d.rows && !ag.live && t == 0) st_co(c.ws.line(CTR_ERR), ERR_BAD_INPUT);
  if constexpr (p4_split_min_chunks<B>() > 0) {
    if (split >= ag.ns) return true;  // a split this row does not use (wave-uniform: no barrier)
    nsplit = ag.ns;
  }
  const int pos = ag.pos, p_begin = ag.p_begin, p_end = ag.p_end, c_end = ag.c_end;
  const bool active = ag.live && as_const(d.row_active)[b] != 0;
  const bool writes_kv = g == 0 && split == 0 && active;  // one task stores the new token's K/V
  const bool qkv_wave = wave < 3 || PAIR;                  // waves that poll a q, k or v word
  const bool norm_wave = wave < 2 || (PAIR && wave == 3);  // q (waves 0, 3) and k (wave 1): RMSNorm + RoPE
  cint32_t* table = as_const(d.page_table + (size_t)b * d.page_stride);
  const int nblk = d.num_blocks;
  uint8_t* smem = c.attn_smem;
  uint16_t* qb = reinterpret_cast<uint16_t*>(smem);       // [128] roped q (head qh)
  uint16_t* kb = qb + HD;                                 // [128] roped k
  uint16_t* vb = kb + HD;                                 // [128] v
  uint16_t* qb2 = vb + HD;                                // [128] roped q of head qh + 1 (PAIR)
  float* mrg = reinterpret_cast<float*>(smem + 1024);     // [4 waves][NQH heads][128]
  float* mrg_ml = mrg + PK_CW * NQH * HD;                 // [4][NQH] m, then [4][NQH] l
  const size_t layer_off = (size_t)layer * (size_t)d.kv_layer_stride + (size_t)h * HD;

  // static operands of the norm/RoPE step and the new token's cache slot: loaded
  // before the poll (the poll's first check then also covers them)
  uint32_t wnw = 0;
  float c0 = 0.f, c1 = 0.f, s0 = 0.f, s1 = 0.f;
  if (norm_wave) {
    wnw = ldg(reinterpret_cast<const uint32_t*>(p4_wptr(d, layer, wave == 1 ? MKD_W_K_NORM : MKD_W_Q_NORM)) + lane);
    const int j = (2 * lane) & 63;
    const float* cs = d.rope_cos + (size_t)pos * (HD / 2);
    const float* sn = d.rope_sin + (size_t)pos * (HD / 2);
    c0 = cs[j]; c1 = cs[j + 1]; s0 = sn[j]; s1 = sn[j + 1];
  }
  const int blk_new = writes_kv ? table[pos / bs] : 0;
  const int slot_in_blk = pos % bs;  // (integer division, off the poll's path)
  // this step's q (wave 0: head qh; PAIR, wave 3: head qh + 1), k (wave 1), v
  // (wave 2): one word per lane
  size_t src = TW_QKV + (size_t)b * (QKV_N / 2) + lane;
  if (wave == 0) src += (size_t)qh * (HD / 2);
  else if (wave == 1) src += QS / 2 + (size_t)h * (HD / 2);
  else if (wave == 2) src += (QS + KVS) / 2 + (size_t)h * (HD / 2);
  else src += (size_t)(qh + 1) * (HD / 2);
  uint64_t qv[1] = {0};
  bool ok = true;
  if (qkv_wave) ok = poll_tagged<1>([=](int) { return c.ws.tw(src); }, qv, tag, c.ws);
#ifdef MKD_TRACE_POLL
  if (tr != nullptr && lane == 0 && qkv_wave) atomicMax(reinterpret_cast<unsigned long long*>(tr + 1), (unsigned long long)wall_clock64());
#endif
  const uint32_t word = (uint32_t)qv[0];  // dims 2*lane, 2*lane + 1
  uint32_t outw = word;
  if (norm_wave) {
    const float x0 = bf_lo(word), x1 = bf_hi(word);
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = __builtin_amdgcn_rsqf(ss * (1.0f / HD) + EPS);
    const float n0 = round_bf(round_bf(x0 * r) * bf_lo(wnw));
    const float n1 = round_bf(round_bf(x1 * r) * bf_hi(wnw));
    // rotate-half RoPE pairs dims i and i + 64: lane L holds 2L, 2L+1, lane L^32 the partners.
    // permlane32_swap(x, x) returns {[x_lo, x_lo], [x_hi, x_hi]} by 32-lane halves:
    // the value of lane L ^ 32 is the second for L < 32 and the first otherwise
    const auto sw0 = __builtin_amdgcn_permlane32_swap(__float_as_uint(n0), __float_as_uint(n0), false, false);
    const auto sw1 = __builtin_amdgcn_permlane32_swap(__float_as_uint(n1), __float_as_uint(n1), false, false);
    const float p0 = __uint_as_float(lane < 32 ? sw0[1] : sw0[0]);
    const float p1 = __uint_as_float(lane < 32 ? sw1[1] : sw1[0]);
    float o0, o1;
    if (lane < 32) { o0 = n0 * c0 - p0 * s0; o1 = n1 * c1 - p1 * s1; }
    else { o0 = n0 * c0 + p0 * s0; o1 = n1 * c1 + p1 * s1; }
    outw = pack_bf2(o0, o1);
  }
  p4_trace_at(c, 4);
  if (qkv_wave) reinterpret_cast<uint32_t*>(qb + wave * HD)[lane] = outw;  // qb, kb, vb, qb2
  // the new token's K (wave 1) and V (wave 2) go to their cache slot from registers
  if (writes_kv && (wave == 1 || wave == 2)) {
    if (blk_new < 0 || blk_new >= nblk) {
      if (lane == 0) st_co(c.ws.line(CTR_ERR), ERR_BAD_INPUT);
    } else {
      const size_t slotp = (size_t)blk_new * bs + slot_in_blk;
      uint16_t* cache = wave == 1 ? d.k_cache : d.v_cache;
      reinterpret_cast<uint32_t*>(cache + layer_off + slotp * KVS)[lane] = outw;
    }
  }
  // Loads under a lane-dependent condition are consumed on every path: a load
  // the compiler sees unconsumed on some path stays pending in its view, and it
  // then waits for all memory operations (write-through stores included) before
  // that register is next written, in whatever task comes next.
  asm volatile("" ::"v"(blk_new), "v"(wnw), "v"(c0), "v"(c1), "v"(s0), "v"(s1), "v"(slot_in_blk), "v"(word));
  if (!p4_agree(c, ok)) {
    p4_skip_chunks<NS>(cc, nch);  // the DMA waves still hand the chunks over
    return false;
  }
  if (tr != nullptr && t == 0) tr[2] = wall_clock64();

  // scores layout: this lane's 16 dims of q (PAIR: of both query heads)
  const int pl = lane >> 3, part = lane & 7;
  uint4 qa[2], qc[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    qa[i] = reinterpret_cast<const uint4*>(qb + part * 16)[i];
    qc[i] = PAIR ? reinterpret_cast<const uint4*>(qb2 + part * 16)[i] : make_uint4(0, 0, 0, 0);
  }
  // Online softmax with a lazily raised reference maximum m0: the
  // probabilities are 2^(score - m0), and m0 (with the sums and the output
  // accumulators) is rescaled only when a score exceeds it by more than
  // LAZY_LOG2 (so every probability stays below 2^LAZY_LOG2). The sum of
  // probabilities is kept per lane (the lanes with part 0, one per position)
  // and reduced once after the loop. PAIR: the second query head keeps its own
  // m1, sum and accumulators; the two heads share each K/V read from LDS.
  constexpr float LAZY_LOG2 = 8.f;
  float m0 = -INFINITY, ls = 0.f, m1 = -INFINITY, ls1 = 0.f;
  float a00 = 0.f, a01 = 0.f;  // dims 2 lane, 2 lane + 1
  float a10 = 0.f, a11 = 0.f;  // (PAIR: head qh + 1)
  const uint8_t* slot = ring + (cc % NS) * SLOT_BYTES;
  const uint8_t* const ring_end = ring + NS * SLOT_BYTES;
  const int pp = 8 * wave + pl;  // this lane's position within a chunk
  for (int j = 0; j < nch; j++) {
    if ((cc + j) % P4G<NS>::G == 0) raw_barrier();  // group of G chunks handed over
    const uint4 k0 = *reinterpret_cast<const uint4*>(slot + kv_kpiece(pp, 2 * part));
    const uint4 k1 = *reinterpret_cast<const uint4*>(slot + kv_kpiece(pp, 2 * part + 1));
    float sc0 = sum_within_8(dot8(k1, qa[1], dot8(k0, qa[0], 0.f)));
    float sc1 = PAIR ? sum_within_8(dot8(k1, qc[1], dot8(k0, qc[0], 0.f))) : 0.f;
    const bool valid = p_begin + KV_CHUNK * j + pp < c_end;
    sc0 = valid ? sc0 * SCALE2 : -INFINITY;
    sc1 = valid ? sc1 * SCALE2 : -INFINITY;
    // (m0 = -inf: any valid score raises it; invalid scores never do)
    if (__builtin_amdgcn_ballot_w64(sc0 > m0 + LAZY_LOG2) != 0) {
      const float n0 = fmaxf(m0, max_over_8_groups(sc0));
      const float al0 = m0 == -INFINITY ? 0.f : ex2(m0 - n0);
      ls *= al0; a00 *= al0; a01 *= al0;
      m0 = n0;
    }
    if (PAIR && __builtin_amdgcn_ballot_w64(sc1 > m1 + LAZY_LOG2) != 0) {
      const float n1 = fmaxf(m1, max_over_8_groups(sc1));
      const float al1 = m1 == -INFINITY ? 0.f : ex2(m1 - n1);
      ls1 *= al1; a10 *= al1; a11 *= al1;
      m1 = n1;
    }
    // (a wave whose positions are all past c_end keeps m = -inf, sums 0)
    const float e0 = valid ? ex2(sc0 - m0) : 0.f;
    const float e1 = PAIR && valid ? ex2(sc1 - m1) : 0.f;
    ls += part == 0 ? e0 : 0.f;
    ls1 += part == 0 ? e1 : 0.f;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const float w0 = lane_value(e0, 8 * q);
      const uint32_t vw = *reinterpret_cast<const uint32_t*>(slot + KV_V_OFF + (8 * wave + q) * 256 + 4 * lane);
      a00 += w0 * bf_lo(vw); a01 += w0 * bf_hi(vw);
      if constexpr (PAIR) {
        const float w1 = lane_value(e1, 8 * q);
        a10 += w1 * bf_lo(vw); a11 += w1 * bf_hi(vw);
      }
    }
    slot += SLOT_BYTES;
    if (slot == ring_end) slot = ring;
  }
  float l0 = wave_sum(ls);
  float l1 = PAIR ? wave_sum(ls1) : 0.f;
  // the token's own position (wave 3: it has the fewest cached positions in the last chunk)
  if (wave == PK_CW - 1 && p_begin <= pos && pos < p_end) {
    const uint32_t kw = reinterpret_cast<const uint32_t*>(kb)[lane];
    const uint32_t vw = reinterpret_cast<const uint32_t*>(vb)[lane];
    {
      const float t0s = wave_sum(dot2(kw, reinterpret_cast<const uint32_t*>(qb)[lane], 0.f)) * SCALE2;
      const float n0 = fmaxf(m0, t0s);
      const float al0 = ex2(m0 - n0), e0 = ex2(t0s - n0);
      l0 = l0 * al0 + e0;
      m0 = n0;
      a00 = a00 * al0 + e0 * bf_lo(vw); a01 = a01 * al0 + e0 * bf_hi(vw);
    }
    if constexpr (PAIR) {
      const float t1s = wave_sum(dot2(kw, reinterpret_cast<const uint32_t*>(qb2)[lane], 0.f)) * SCALE2;
      const float n1 = fmaxf(m1, t1s);
      const float al1 = ex2(m1 - n1), e1 = ex2(t1s - n1);
      l1 = l1 * al1 + e1;
      m1 = n1;
      a10 = a10 * al1 + e1 * bf_lo(vw); a11 = a11 * al1 + e1 * bf_hi(vw);
    }
  }
  const size_t pbase = TW_APART + (((size_t)b * NKV + h) * MAXS) * PART_STRIDE;  // split partials of (b, h)
  // (batch 2 and 4: inlined at batch 1 and 8, where it never helps a short
  // context, this code slowed the short-context step: 8-15 us, measured)
  constexpr bool FOLD = !PAIR && (B == 2 || B == 4);
  if constexpr (FOLD) {
    if (nsplit > 1 && split == nsplit - 1) {
      // last split: wave w folds the other splits' partials into its own
      // accumulators (p4_fold_splits); the waves' merge below then combines them
      p4_fold_splits(c.ws, pbase, nsplit, g, tag, m0, l0, a00, a01, ok);
    }
  }
  // merge the waves in LDS
  reinterpret_cast<float2*>(mrg + wave * NQH * HD)[lane] = make_float2(a00, a01);
  if (PAIR) reinterpret_cast<float2*>(mrg + wave * NQH * HD + HD)[lane] = make_float2(a10, a11);
  if (lane == 0) {
    mrg_ml[wave * NQH] = m0; mrg_ml[PK_CW * NQH + wave * NQH] = l0;
    if (PAIR) { mrg_ml[wave * NQH + 1] = m1; mrg_ml[PK_CW * NQH + wave * NQH + 1] = l1; }
  }
  c.sync();
  // thread t: dim dd of the head; threads t and t + 128 compute the same value
  // (PAIR: thread t of head qh + (t >> 7), gg = its query head within the group)
  const int dd = t & (HD - 1), half = t >> 7;
  const int hh = PAIR ? half : 0, gg = PAIR ? half : g;
  float M = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < PK_CW; ww++) M = fmaxf(M, mrg_ml[ww * NQH + hh]);
  float num = 0.f, den = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int ww = 0; ww < PK_CW; ww++) {
      const float sc = ex2(mrg_ml[ww * NQH + hh] - M);
      num += mrg[(ww * NQH + hh) * HD + dd] * sc;
      den += mrg_ml[PK_CW * NQH + ww * NQH + hh] * sc;
    }
  }
  if (nsplit > 1 && split != nsplit - 1) {
    // read only by the last split of this (row, query head)
    uint64_t* part = c.ws.tw(pbase + (size_t)split * PART_STRIDE);
    if (PAIR || half == 0) {
      st_tw(part + gg * HD + dd, tw_make(__float_as_uint(num), tag));
      if (dd == 0) {
        st_tw(part + GROUP * HD + gg, tw_make(__float_as_uint(M), tag));
        st_tw(part + GROUP * HD + GROUP + gg, tw_make(__float_as_uint(den), tag));
      }
    }
    c.sync();  // the scratch is reused by this workgroup's next task
    return true;
  }
  if constexpr (B == 1 || PAIR) {
    // batch 1 (and tasks of both query heads): the last split folds the other
    // splits' partials here, up to SPR splits per poll round (all of a round's
    // loads in flight at once: one round trip instead of one per split), in
    // split order
    // (8 partials per round at batch 1 and 4: C5 batch 1 643 -> 614 us, C5 batch
    // 4 834 -> 808 than 3 per round, but batch 8 +14 us; 15 per round spills)
    constexpr int SPR = B == 8 ? 3 : 8;
    for (int sp0 = 0; nsplit > 1 && sp0 < nsplit - 1; sp0 += SPR) {
      uint64_t e[3 * SPR];
      // (entries past the last split repeat its words)
      ok = ok && poll_tagged<3 * SPR>(
                     [&](int k) {
                       const int sp = min(sp0 + k / 3, nsplit - 2), f = k % 3;
                       const size_t ps = pbase + (size_t)sp * PART_STRIDE;
                       return c.ws.tw(ps + (f == 0 ? (size_t)(gg * HD + dd) : (size_t)(GROUP * HD + (f - 1) * GROUP + gg)));
                     },
                     e, tag, c.ws);
#pragma unroll
      for (int q = 0; q < SPR; q++) {
        if (sp0 + q >= nsplit - 1) break;
        const float ns = __uint_as_float((uint32_t)e[3 * q]), ms = __uint_as_float((uint32_t)e[3 * q + 1]);
        const float ls = __uint_as_float((uint32_t)e[3 * q + 2]);
        if (ms == -INFINITY) continue;
        const float nm = fmaxf(M, ms);
        const float sa = M == -INFINITY ? 0.f : ex2(M - nm), sb = ex2(ms - nm);
        num = num * sa + ns * sb;
        den = den * sa + ls * sb;
        M = nm;
      }
    }
  }
  if constexpr (B == 8 && !PAIR) {
    // batch 8: the last split folds the other splits' partials here, one
    // split per round; the two thread halves (the same dims) take the even and
    // the odd splits, then combine (even, odd) in that order
    if (nsplit > 1) {
      float Mh = half == 0 ? M : -INFINITY, nh = half == 0 ? num : 0.f, dh = half == 0 ? den : 0.f;
      for (int sp = half; sp < nsplit - 1; sp += 2) {
        const size_t ps = pbase + (size_t)sp * PART_STRIDE;
        uint64_t e[3];
        ok = ok && poll_tagged<3>(
                       [&](int k) {
                         return c.ws.tw(ps + (k == 0 ? (size_t)(g * HD + dd) : (size_t)(GROUP * HD + (k - 1) * GROUP + g)));
                       },
                       e, tag, c.ws);
        const float ns = __uint_as_float((uint32_t)e[0]), ms = __uint_as_float((uint32_t)e[1]);
        const float ls = __uint_as_float((uint32_t)e[2]);
        if (ms == -INFINITY) continue;
        const float nm = fmaxf(Mh, ms);
        const float sa = Mh == -INFINITY ? 0.f : ex2(Mh - nm), sb = ex2(ms - nm);
        nh = nh * sa + ns * sb;
        dh = dh * sa + ls * sb;
        Mh = nm;
      }
      // through the q/k/v scratch (free after the waves' merge): the odd half's
      // fold, then the combined result
      float* xf = reinterpret_cast<float*>(smem);  // [128] num, then max, sum (odd half), max, sum (combined)
      if (half == 1) {
        xf[dd] = nh;
        if (dd == 0) { xf[HD] = Mh; xf[HD + 1] = dh; }
      }
      c.sync();
      if (half == 0) {
        const float mo = xf[HD], no = xf[dd], lo = xf[HD + 1];
        if (mo != -INFINITY) {
          const float nm = fmaxf(Mh, mo);
          const float sa = Mh == -INFINITY ? 0.f : ex2(Mh - nm), sb = ex2(mo - nm);
          nh = nh * sa + no * sb;
          dh = dh * sa + lo * sb;
          Mh = nm;
        }
      }
      if (half == 0) {
        xf[dd] = nh;  // (this thread's own entry, read above)
        if (dd == 0) { xf[HD + 2] = Mh; xf[HD + 3] = dh; }
      }
      c.sync();
      num = xf[dd]; M = xf[HD + 2]; den = xf[HD + 3];
    }
  }
  const uint32_t mine = f2bf(num / den);
  // the neighbouring dimension's value: a DPP quad swap (every lane active
  // here), not an LDS-crossbar round trip
  const uint32_t nbr = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)mine, 0xB1, 0xF, 0xF, false);
  {
    // the pair (dd, dd + 1) as one word; its p4_nrep replicas are stored by
    // the four threads (dd even / odd, half 0 / 1) that hold it (PAIR: two
    // threads, dd even / odd), spread evenly; a thread past the replica count
    // stores none
    const uint64_t v = tw_make((dd & 1) ? (nbr | (mine << 16)) : (mine | (nbr << 16)), tag);
    constexpr int HOLD = PAIR ? 2 : 4;
    constexpr int NREP = p4_nrep<B>();
    constexpr int NR = NREP / HOLD > 0 ? NREP / HOLD : 1;
    const size_t word = TW_ATTN + (size_t)b * (QS / 2) + ((size_t)(qh + hh) * HD + dd) / 2;
    const int r0 = (PAIR ? (dd & 1) : (dd & 1) * 2 + half) * NR;
#pragma unroll
    for (int r = 0; r < NR; r++)
      if (r0 + r < NREP) st_rep(c.ws, word, r0 + r, v);
  }
  return p4_agree(c, ok);  // also frees the scratch for the next task
}

// ---- DMA waves -------------------------------------------------------------
// A decoded task as one DMA wave sees it (all wave-uniform). A chunk is 16
// 1-KiB units (K = 3072: 12) of whole rows; unit u of a chunk lands at LDS
// offset u * 1 KiB of its slot. In every full chunk this wave's units form an
// arithmetic sequence in both the source and the slot, so a full chunk costs
// a pointer bump and 4 (K = 3072: 3) copies:
//   K = 1024: units dw + 4k   -> rows 2k + (dw >> 1), half (dw & 1) of the row
//             (GATEUP: dw >> 1 picks the gate or up matrix, k the channel)
//   K = 2048: units dw + 4k   -> row k, quarter dw
//   K = 3072: units 3dw + k   -> row dw >> 1, sixth 3 (dw & 1) + k
// A short last chunk (rows not a multiple of the chunk's) takes the general
// path, which repeats the task's last unit to keep the copy count.
//
// ATTN tasks (kind 3) stage their cached K/V: chunk j = positions p0 + 32 j ..
// + 31 (within one cache block, as the block size is a multiple of 32), K in
// units 0-7 and V in units 8-15 (4 positions per unit), this wave's units dw,
// dw + 4 (K) and dw + 8, dw + 12 (V), each lane one 16-byte piece; positions
// at or past the end of the cached ones repeat p0.
struct DmaTask {
  int kind;              // 0: K = 1024, 1: K = 2048, 2: K = 3072, 3: KV chunks of an ATTN task
  int nch;               // chunks (0: no weights)
  int nfull;             // leading full chunks
  int units;             // 1-KiB units of the task's weight rows
  int stride;            // elements between consecutive rows (per channel for GATEUP)
  const uint16_t* b0;    // row 0 (GATEUP: gate rows)
  const uint16_t* b1;    // GATEUP: up rows, else null
  const uint16_t* src;   // this wave's first unit of the next full chunk
  int64_t kstep;         // elements between this wave's units within a chunk
  int64_t cstep;         // elements between chunks
  int lds0, ldsk;        // slot offset of this wave's first unit, and between its units (bytes)
  // ATTN tasks reuse the fields (the struct lives in scalar registers across the
  // DMA loop; more fields would spill it to memory): b0 / b1 = K / V of the layer
  // and head, src = the row's block table, stride = block size, units = cache
  // blocks, nfull = first position p0, lds0 = end of the cached positions.
  __device__ __forceinline__ cint32_t* table() const { return (cint32_t*)(uintptr_t)src; }
};

// Step-descriptor fields the DMA waves need for ATTN tasks, read from the
// kernel arguments through the constant address space (scalar loads).
template <typename T>
__device__ __forceinline__ T karg_field(const uint8_t* karg, size_t off) {
  typedef __attribute__((address_space(4))) const T ct;
  return *reinterpret_cast<ct*>(reinterpret_cast<uintptr_t>(karg) + off);
}
template <int B>
__device__ __forceinline__ void dma_decode_attn(DmaTask& t, const uint8_t* karg, const Inst& w) {
  const int b = (w.a0 & (ATTN_QHEAD - 1)) / NKV, h = w.a0 % NKV;
  const int rows = karg_field<int32_t>(karg, offsetof(MkdStepDesc, rows));
  const int bs = karg_field<int32_t>(karg, offsetof(MkdStepDesc, block_size));
  const int stride = karg_field<int32_t>(karg, offsetof(MkdStepDesc, page_stride));
  const int32_t* seqlens = karg_field<int32_t*>(karg, offsetof(MkdStepDesc, cache_seqlens));
  const int pos_in = b < rows ? as_const(seqlens)[b] : 0;
  const AttnGeo g = attn_geo(rows, b, pos_in, stride, bs, w.a1, w.a2, p4_split_min_chunks<B>());
  t.kind = 3;
  t.nch = g.nch;
  if (g.nch == 0) return;
  const size_t off = (size_t)w.layer * (size_t)karg_field<int64_t>(karg, offsetof(MkdStepDesc, kv_layer_stride)) +
                     (size_t)h * HD;
  t.b0 = karg_field<uint16_t*>(karg, offsetof(MkdStepDesc, k_cache)) + off;
  t.b1 = karg_field<uint16_t*>(karg, offsetof(MkdStepDesc, v_cache)) + off;
  t.src = reinterpret_cast<const uint16_t*>(karg_field<const int32_t*>(karg, offsetof(MkdStepDesc, page_table)) +
                                            (size_t)b * stride);
  t.stride = bs;
  t.units = karg_field<int32_t>(karg, offsetof(MkdStepDesc, num_blocks));
  t.nfull = g.p_begin;
  t.lds0 = g.c_end;
}

// Cache policy of the ring copies (weights and KV cache): non-temporal (the
// gfx950 nt bit). Every byte is read once per step, and with the default policy
// each hand-over's burst of streamed lines competes with the tagged words that
// the whole grid polls at that moment for the memory-side cache. Measured: batch
// 1/2/4/8 -17/-14/-14/-13 us, C5 batch 8 -25 us, C4 batch 8 -14 us. (sc0 or
// sc1 alone: no change.)
constexpr int DMA_NT = 2;

// KV chunk j of ATTN task t into `slot` (this DMA wave's 4 units). A cached
// position's block id outside [0, num_blocks) is reported as ERR_BAD_INPUT and
// clamped, so no copy leaves the cache.
__device__ __forceinline__ void dma_issue_attn(const DmaTask& t, int j, uint8_t* slot, int dw, const uint8_t* karg) {
  const int lane = threadIdx.x & 63;
  const int P0 = t.nfull + KV_CHUNK * j, bs = t.stride;
  const int raw = t.table()[P0 / bs];
  const int blk = min(max(raw, 0), t.units - 1);
  if (raw != blk && lane == 0) {
    const Ws ws{karg_field<uint8_t*>(karg, offsetof(MkdStepDesc, workspace))};
    st_co(ws.line(CTR_ERR), ERR_BAD_INPUT);
  }
  const size_t row0 = (size_t)blk * bs + P0 % bs;
  const int s16 = lane & 15;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int u = dw + 4 * k;                       // k < 2: K units, k >= 2: V units
    const int p = 4 * (u & 7) + (lane >> 4);        // chunk position of this lane
    const int q = k < 2 ? ((s16 - (p & 1)) & 15) : s16;  // source piece (K: unswizzled)
    const int pr = P0 + p < t.lds0 ? p : 0;
    const uint16_t* src = (k < 2 ? t.b0 : t.b1) + (row0 + pr) * KVS + q * 8;
    __builtin_amdgcn_global_load_lds((gbl_void_t*)src, (lds_void_t*)(slot + u * 1024), 16, 0, DMA_NT);
  }
}

template <int B>
__device__ __forceinline__ DmaTask dma_decode(cuint64_t* lp, const uint16_t* emb, const uint8_t* karg, const Inst& w,
                                              int dw) {
  auto W = [&](int which) { return reinterpret_cast<const uint16_t*>(lp[w.layer * MKD_LAYER_PTRS + which]); };
  const int a0 = w.a0, a1 = w.a1;
  DmaTask t{};
  t.b1 = nullptr;
  switch (w.op) {
    case MKD_OP_ATTN:
      dma_decode_attn<B>(t, karg, w);
      return t;
    case MKD_OP_QKV:
      t.b0 = a0 < QS ? W(MKD_W_Q) + (size_t)a0 * H
                     : (a0 < QS + KVS ? W(MKD_W_K) + (size_t)(a0 - QS) * H : W(MKD_W_V) + (size_t)(a0 - QS - KVS) * H);
      t.kind = 0; t.units = 2 * a1; t.stride = H;
      break;
    case MKD_OP_LMHEAD:
      t.b0 = emb + (size_t)a0 * H;
      t.kind = 0; t.units = 2 * a1; t.stride = H;
      break;
    case MKD_OP_GATEUP:
      t.b0 = W(MKD_W_GATE) + (size_t)a0 * H;
      t.b1 = W(MKD_W_UP) + (size_t)a0 * H;
      t.kind = 0; t.units = 4 * a1; t.stride = H;
      break;
    case MKD_OP_OPROJ:
      t.b0 = W(MKD_W_O) + (size_t)a0 * QS;
      t.kind = 1; t.units = 4 * a1; t.stride = QS;
      break;
    case MKD_OP_DOWN:
      t.b0 = W(MKD_W_DOWN) + (size_t)a0 * I;
      t.kind = 2; t.units = 6 * a1; t.stride = I;
      break;
    default:
      t.nch = 0;
      return t;
  }
  const int upc = t.kind == 2 ? 12 : 16;
  t.nch = (t.units + upc - 1) / upc;
  t.nfull = t.units / upc;
  if (t.kind == 0) {
    if (t.b1 != nullptr) {
      t.src = ((dw >> 1) ? t.b1 : t.b0) + (dw & 1) * 512;
      t.kstep = t.stride;
      t.cstep = 4 * (int64_t)t.stride;
    } else {
      t.src = t.b0 + (size_t)(dw >> 1) * t.stride + (dw & 1) * 512;
      t.kstep = 2 * (int64_t)t.stride;
      t.cstep = 8 * (int64_t)t.stride;
    }
    t.lds0 = dw * 1024; t.ldsk = 4096;
  } else if (t.kind == 1) {
    t.src = t.b0 + dw * 512;
    t.kstep = t.stride;
    t.cstep = 4 * (int64_t)t.stride;
    t.lds0 = dw * 1024; t.ldsk = 4096;
  } else {
    t.src = t.b0 + (size_t)(dw >> 1) * t.stride + 3 * (dw & 1) * 512;
    t.kstep = 512;
    t.cstep = 2 * (int64_t)t.stride;
    t.lds0 = 3 * dw * 1024; t.ldsk = 1024;
  }
  return t;
}

// Copy chunk j of task t into `slot` (this DMA wave's share).
template <int K>
__device__ __forceinline__ void dma_issue(DmaTask& t, int j, uint8_t* slot, int dw) {
  constexpr int PR = K / 512;       // 1-KiB units per row
  constexpr int UPC = (16 / PR) * PR;
  constexpr int LPW = UPC / 4;      // copies per DMA wave per chunk
  const int lane = threadIdx.x & 63;
  // lane i of the copy of a 1-KiB unit brings piece (i + r) mod 64 of it, r =
  // the unit's row within the chunk (wpiece): a rotation per row
  if (j < t.nfull) {
#pragma unroll
    for (int k = 0; k < LPW; k++) {
      // (full chunks: this wave's copy k is unit dw + 4k, row 2k + dw / 2 at
      // K = 1024 and row k at 2048; unit 3 dw + k, row dw / 2 at 3072)
      const int r = K == 1024 ? 2 * k + (dw >> 1) : (K == 2048 ? k : dw >> 1);
      const int src_lane = (lane + r) & 63;
      __builtin_amdgcn_global_load_lds((gbl_void_t*)(t.src + k * t.kstep + src_lane * 8),
                                       (lds_void_t*)(slot + t.lds0 + k * t.ldsk), 16, 0, DMA_NT);
    }
    t.src += t.cstep;
    return;
  }
  const int u0 = j * UPC;
#pragma unroll
  for (int k = 0; k < LPW; k++) {
    const int u = min(u0 + dw + 4 * k, t.units - 1);
    const int r = u / PR, p = u - r * PR;
    const uint16_t* row = t.b1 != nullptr ? ((r & 1) ? t.b1 : t.b0) + (size_t)(r >> 1) * t.stride
                                          : t.b0 + (size_t)r * t.stride;
    const int src_lane = (lane + (u - u0) / PR) & 63;
    __builtin_amdgcn_global_load_lds((gbl_void_t*)(row + p * 512 + src_lane * 8), (lds_void_t*)(slot + (u - u0) * 1024),
                                     16, 0, DMA_NT);
  }
}

// s_waitcnt vmcnt(3 * later) for a runtime later in [0, M]: chunk r has landed
// when at most the copies of the `later` chunks issued after it are pending
// (each chunk issues at least 3 copies per DMA wave).
template <int M>
__device__ __forceinline__ void wait_chunk(int later) {
  if (later >= M) { waitcnt_vm<3 * M>(); return; }
  if constexpr (M > 0) wait_chunk<M - 1>(later);
}

// The DMA waves: keep D chunks in flight; for each chunk r, wait until it has
// landed, hand it over (barrier r), then issue chunk r + D. Decoding a new
// task (scalar loads) therefore overlaps the compute waves' work on chunk r
// instead of delaying the hand-over of chunk r + 1. Chunk r + D goes to the
// slot of chunk r - 2, which the compute waves finished before barrier r - 1.
template <int B>
__device__ __noinline__ void p4_dma(const uint64_t* layer_ptrs, const uint16_t* embed, const int32_t* row,
                                    int n_inst_arg, uint8_t* ring_arg, int dw_arg, uint8_t* ws_arg,
                                    const uint8_t* karg_arg) {
  using Cfg = PkCfg<B>;
  cuint64_t* lp = as_const(uniform_ptr(layer_ptrs));
  const uint16_t* emb = uniform_ptr(embed);
  cint32_t* crow = as_const(uniform_ptr(row));
  const int n = __builtin_amdgcn_readfirstlane(n_inst_arg);
  uint8_t* ring = uniform_ptr(ring_arg);
  const int dw = __builtin_amdgcn_readfirstlane(dw_arg);
  const uint8_t* karg = uniform_ptr(karg_arg);
#ifdef MKD_TRACE_CHUNKS
  // debug: chunk arrival/release/issue times after the compute waves' ([grid][512][3])
  uint64_t* dbg = reinterpret_cast<uint64_t*>(uniform_ptr(ws_arg));
#endif
  (void)ws_arg;
  // Task decode is software-pipelined: the instruction words of the task after
  // `nxt` and the weight pointers of `nxt` are requested (scalar loads) while
  // `cur` is being issued, so no chunk hand-over waits on a scalar-cache miss.
  int pf = 0;  // index of the prefetched instruction in `pinst`
  Inst pinst{};
  if (n > 0) pinst = load_inst(crow);
  auto next_weight_task = [&]() {
    while (pf < n) {
      const Inst w = pinst;
      pf++;
      if (pf < n) pinst = load_inst(crow + pf * MKD_INST_WORDS);
      const DmaTask t = dma_decode<B>(lp, emb, karg, w, dw);
      if (t.nch > 0) return t;
    }
    DmaTask none{};
    none.nch = 0;
    return none;
  };
  // make every field of t wave-resident now (waits for its scalar loads here,
  // before newer scalar loads are issued behind them)
  auto settle = [](const DmaTask& t) {
    asm volatile("" ::"s"(t.kind), "s"(t.nch), "s"(t.nfull), "s"(t.units), "s"(t.stride), "s"(t.b0), "s"(t.b1),
                 "s"(t.src), "s"(t.kstep), "s"(t.cstep), "s"(t.lds0), "s"(t.ldsk));
  };
  constexpr int G = P4G<Cfg::NS>::G;
  int tj = 0, issued = 0;
  DmaTask cur = next_weight_task();
  settle(cur);
  DmaTask nxt = next_weight_task();
  auto issue_one = [&]() {
    uint8_t* slot = ring + (issued % Cfg::NS) * SLOT_BYTES;
#ifdef MKD_TRACE_CHUNKS
    if (dbg != nullptr && dw == 0 && (threadIdx.x & 63) == 0)
      dbg[((size_t)blockIdx.x * 512 + (issued & 511)) * 3 + 2] = wall_clock64();
#endif
    if (cur.kind == 0) dma_issue<H>(cur, tj, slot, dw);
    else if (cur.kind == 1) dma_issue<QS>(cur, tj, slot, dw);
    else if (cur.kind == 2) dma_issue<I>(cur, tj, slot, dw);
    else dma_issue_attn(cur, tj, slot, dw, karg);
    issued++;
    if (++tj == cur.nch) {
      tj = 0;
      cur = nxt;
      settle(cur);
      nxt = next_weight_task();
    }
  };
  // before the first hand-over no slot is in use: fill the ring
  while (cur.nch > 0 && issued < Cfg::NS) issue_one();
  // group g = chunks [g G, g G + G): after its hand-over the compute waves are
  // done with group g - 1, so chunks up to g G + NS - 1 may be issued
  for (int g = 0; g * G < issued; g++) {
    const int e = min(g * G + G, issued);   // end of group g (issued >= e: 2G <= NS)
    wait_chunk<Cfg::NS - 1>(issued - e);     // chunk e - 1 (and all before) landed
#ifdef MKD_TRACE_CHUNKS
    if (dbg != nullptr && dw == 0 && (threadIdx.x & 63) == 0) {
      const uint64_t now = wall_clock64();
      for (int k = g * G; k < e; k++) dbg[((size_t)blockIdx.x * 512 + (k & 511)) * 3] = now;
    }
#endif
    raw_barrier();
    while (cur.nch > 0 && issued < g * G + Cfg::NS) issue_one();
  }
}

template <int B>
__global__ __launch_bounds__(PK_THREADS, 1) void k_persistent4(MkdStepDesc d, MkdSchedule s) {
  using Cfg = PkCfg<B>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* ring = lds;
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds + Cfg::NS * SLOT_BYTES);
  uint8_t* scratch = lds + Cfg::NS * SLOT_BYTES + Cfg::XS_BYTES;
  const Ws ws{reinterpret_cast<uint8_t*>(d.workspace)};
  const int n_inst = s.num_inst[blockIdx.x];
  const int32_t* row = s.inst + (size_t)blockIdx.x * s.max_inst * MKD_INST_WORDS;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int* flags = reinterpret_cast<int*>(scratch + P4_SCR_FLAGS);
  if (threadIdx.x == 0) {
    *reinterpret_cast<uint32_t*>(scratch) = 0u;  // SyncCW counter
    flags[0] = 0x7fffffff;  // no task failed
    flags[1] = (int)ld_co(ws.line(CTR_EPOCH));
  }
  __syncthreads();
  if (wave >= PK_CW) {
#ifdef MKD_TRACE_CHUNKS
    uint8_t* dbg_dw = d.trace == nullptr ? nullptr
                                         : reinterpret_cast<uint8_t*>(d.trace + (size_t)s.grid * s.max_inst * 4 + 256 * 512 * 2);
#else
    uint8_t* dbg_dw = nullptr;
#endif
    p4_dma<B>(d.layer_ptrs, d.embed, row, n_inst, ring, wave - PK_CW, dbg_dw,
              reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(__builtin_amdgcn_kernarg_segment_ptr())));
    return;
  }
  P4 c{ws, p4_xcc_id() % p4_nrep<B>(), (uint32_t)flags[1], SyncLds{reinterpret_cast<uint32_t*>(scratch), 0u}, flags,
             reinterpret_cast<float*>(scratch + P4_SCR_RED), reinterpret_cast<float*>(scratch + P4_SCR_RES), xs,
             scratch + P4_SCR_ATTN, reinterpret_cast<uint32_t*>(scratch + P4_SCR_STAGE), 0, nullptr, 0,
             reinterpret_cast<float*>(scratch + p4_scr_part<B>())};
  bool aborted = false;
  int cc = 0;
  ResKeep<B> rk;  // residual stream of this thread's features (after a first RMSNorm task)
  rk.valid = false;
  cint32_t* crow = as_const(row);
  Inst w_next = n_inst > 0 ? load_inst(crow) : Inst{};
  for (int i = 0; i < n_inst; i++) {
    const Inst w = w_next;
    if (i + 1 < n_inst) w_next = load_inst(crow + (i + 1) * MKD_INST_WORDS);  // in flight during this task
    // per-task time stamps (MkdStepDesc::trace, a debugging aid): compiled into
    // builds with MKD_TRACE_TASKS and into the batch-8 kernel; the other
    // kernels leave them out (batch 1/2/4 -3/-6/-4 us; left out at batch 8 the
    // smaller kernel measured 19 us slower)
    uint64_t* tr = nullptr;
#ifndef MKD_TRACE_TASKS
    if constexpr (B >= 8)
#endif
      tr = d.trace != nullptr ? d.trace + ((size_t)blockIdx.x * s.max_inst + i) * P4_TR_STRIDE : nullptr;
    if (tr != nullptr && threadIdx.x == 0) tr[0] = wall_clock64();
    c.trp = tr;
    c.task = i;
    if (w.op == MKD_OP_QKV || w.op == MKD_OP_GATEUP) c.par ^= 1;
    if (w.op == MKD_OP_ATTN) {
      int nkv = 0;
      // ATTN_ONE_HEAD: one query head per task, else both heads of the KV head
      // (compiled from batch P4_PAIR_MIN_B on: at batch 1 the second body alone,
      // never run, slowed the step by 2%, measured)
      const bool pair = !(w.a0 & ATTN_ONE_HEAD);
      if (!aborted && pair && B < P4_PAIR_MIN_B) {
        if (threadIdx.x == 0) st_co(ws.line(CTR_ERR), ERR_BAD_INST);
        aborted = true;
      }
      if (!aborted) {
        if constexpr (B >= P4_PAIR_MIN_B) {
          aborted = pair ? !p4_attn<B, Cfg::NS, true>(d, c, w.layer, w.a0, w.a1, w.a2, tr, ring, cc, nkv)
                         : !p4_attn<B, Cfg::NS, false>(d, c, w.layer, w.a0, w.a1, w.a2, tr, ring, cc, nkv);
        } else {
          aborted = !p4_attn<B, Cfg::NS, false>(d, c, w.layer, w.a0, w.a1, w.a2, tr, ring, cc, nkv);
        }
      } else {
        nkv = p4_attn_chunks<B>(d, w);
        p4_skip_chunks<Cfg::NS>(cc, nkv);
      }
      cc += nkv;
      if (tr != nullptr && threadIdx.x == 0) tr[3] = wall_clock64();
      continue;
    }
    const int nch = p4_chunks(w);
    if (nch == 0) continue;
    if (!aborted && w.op != MKD_OP_LMHEAD && p4_rows(w) * (w.op == MKD_OP_DOWN ? 2 : 1) > P4_MAX_ROWS) {
      if (threadIdx.x == 0) st_co(ws.line(CTR_ERR), ERR_BAD_INST);
      aborted = true;
    }
    if (!aborted) aborted = !p4_prologue<B>(d, c, w, rk);
    if (tr != nullptr && threadIdx.x == 0) tr[1] = wall_clock64();
    LmArg<B> best;
    best.reset();
#ifdef MKD_TRACE_CHUNKS
    uint64_t* dbg = d.trace == nullptr ? nullptr : d.trace + (size_t)s.grid * s.max_inst * 4;
#else
    uint64_t* dbg = nullptr;
#endif
    p4_task_chunks<B, Cfg::NS>(d, c, w, ring, cc, nch, aborted, tr, best, dbg);
    cc += nch;
    if (!aborted) {
      if (w.op == MKD_OP_LMHEAD) aborted = !p4_lm_finish<B>(d, c, w, best);
      else {
#ifdef MKD_TRACE_CHUNKS
        uint64_t* dbg_st = d.trace == nullptr ? nullptr
                                              : d.trace + (size_t)s.grid * s.max_inst * 4 + 256 * 512 * 5 +
                                                    ((size_t)blockIdx.x * s.max_inst + i) * 8;
#else
        uint64_t* dbg_st = nullptr;
#endif
        p4_store<B>(c, w, dbg_st);
      }
    }
    if (tr != nullptr && threadIdx.x == 0) tr[3] = wall_clock64();
  }
}

}  // namespace mkd
