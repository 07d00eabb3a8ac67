// mkd_persistent.h -- the persistent task-graph kernel with LDS-DMA weight streaming.
//
// One 512-thread workgroup per compute unit. Waves 0-3 are compute waves
// (CW): they poll dependency counters, stage activations, run the task math
// and store results. Waves 4-7 are DMA waves (DW): they walk the same
// instruction row D chunks ahead and copy each upcoming task's weight rows
// straight into a ring of 16 KiB LDS slots with global_load_lds_dwordx4
// (no registers involved), so HBM keeps streaming while the compute waves
// wait on the dependency chain. A chunk is a run of whole weight rows; an
// attention task is one chunk without weights.
//
// Synchronisation inside the workgroup:
//  * one s_barrier per chunk pairs the two groups: before it the DMA waves
//    have issued chunk c+D and waited (vmcnt) until chunk c has landed in LDS;
//    after it the compute waves read chunk c. The slot chunk c+D overwrites
//    held chunk c-2, whose compute finished before the previous barrier
//    (NS = D + 2 slots).
//  * the compute waves sync among themselves with an LDS counter (SyncCW),
//    so the DMA waves never block on a compute-only step and never touch
//    LDS themselves (a DMA wave reading LDS would make the compiler wait for
//    all its in-flight copies).
#pragma once

#include "mkd_tasks.h"

namespace mkd {

constexpr int PK_THREADS = 512;
constexpr int PK_CW = 4;
constexpr int SLOT_BYTES = 16384;
constexpr int PK_SCRATCH = 8192;
constexpr int MAX_LDS = 163840;

template <int B>
struct PkCfg {
  static constexpr int XS_BYTES = B * I * 2;
  // (batch 8: 4 KiB more for the tagged kernel's partial-sum tile; the ring
  // keeps its 6 slots)
  static constexpr int SCRATCH = B >= 8 ? PK_SCRATCH + 4096 : PK_SCRATCH;
  static constexpr int NS = (MAX_LDS - XS_BYTES - SCRATCH) / SLOT_BYTES;
  static constexpr int D = NS - 2;
  static constexpr int LDS_BYTES = NS * SLOT_BYTES + XS_BYTES + SCRATCH;
  static_assert(D >= 2, "lookahead too small");
};

// LDS-counter barrier of the four compute waves. Each wave adds 1 per
// barrier; the value a wave's add returns identifies the barrier generation
// (no wave can add for barrier k+1 before all four added for barrier k), so
// the barrier needs no per-wave state.
struct SyncCW {
  uint32_t* ctr;
  __device__ __forceinline__ void operator()() const {
    uint32_t old = 0;
    if ((threadIdx.x & 63) == 0)
      old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __shfl(old, 0, 64);
    const uint32_t target = (old / PK_CW + 1) * PK_CW;
    while (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < target) __builtin_amdgcn_s_sleep(0);
  }
};

// Workgroup-wide s_barrier without the memory fences of __syncthreads (a
// release fence would make the DMA waves wait for their own copies).
__device__ __forceinline__ void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) for a runtime n in [0, 63] (gfx9 encoding, other counters untouched).
template <int N>
__device__ __forceinline__ void waitcnt_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
template <int N = 0>
__device__ __forceinline__ void wait_vmcnt(int n) {
  if constexpr (N < 63) {
    if (n <= N) { waitcnt_vm<N>(); return; }
    wait_vmcnt<N + 1>(n);
  } else {
    waitcnt_vm<63>();
  }
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) const void gbl_void_t;
// Constant-address-space views: loads through them are scalar (s_load,
// counted by lgkmcnt), so the DMA waves can read instruction words and weight
// pointers without waiting for their in-flight copies (vmcnt is in-order).
typedef __attribute__((address_space(4))) const int32_t cint32_t;
typedef __attribute__((address_space(4))) const uint64_t cuint64_t;
__device__ __forceinline__ cint32_t* as_const(const int32_t* p) { return (cint32_t*)(uintptr_t)p; }
// Force a wave-uniform 64-bit value into SGPRs.
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  // readfirstlane returns int: go through uint32_t so the low word is not sign-extended
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | (uint64_t)lo);
}
// One decoded instruction, read once per task with scalar loads and kept in
// registers (re-reading it through a generic pointer after each barrier
// would cost a vector-memory round trip per chunk).
struct Inst {
  int op, layer, a0, a1, a2, wait, wait_cnt, signal;
  __device__ __forceinline__ int operator[](int i) const {
    switch (i) {
      case MKD_I_OP: return op; case MKD_I_LAYER: return layer; case MKD_I_A0: return a0;
      case MKD_I_A1: return a1; case MKD_I_A2: return a2; case MKD_I_WAIT: return wait;
      case MKD_I_WAIT_CNT: return wait_cnt; default: return signal;
    }
  }
};
__device__ __forceinline__ Inst load_inst(cint32_t* w) {
  return Inst{w[MKD_I_OP], w[MKD_I_LAYER], w[MKD_I_A0], w[MKD_I_A1], w[MKD_I_A2], w[MKD_I_WAIT],
              w[MKD_I_WAIT_CNT], w[MKD_I_SIGNAL]};
}
// Weight-table view used by the DMA waves (kept in SGPRs).
struct WeightSrc {
  const uint64_t* layer_ptrs;
  const uint16_t* embed;
};
__device__ __forceinline__ cuint64_t* as_const(const uint64_t* p) { return (cuint64_t*)(uintptr_t)p; }

// ---- chunk geometry ---------------------------------------------------------
__device__ __forceinline__ int op_k(int op) {
  return op == MKD_OP_OPROJ ? QS : (op == MKD_OP_DOWN ? I : H);
}
__device__ __forceinline__ int op_rows_per_chunk(int op) {
  return op == MKD_OP_OPROJ ? 4 : (op == MKD_OP_DOWN ? 2 : 8);
}
// Weight rows of a task (GATEUP: gate and up row of each channel, interleaved).
template <class P>
__device__ __forceinline__ int task_rows(P w) {
  const int op = w[MKD_I_OP];
  if (op == MKD_OP_ATTN || op == MKD_OP_NOP) return 0;
  return op == MKD_OP_GATEUP ? 2 * w[MKD_I_A1] : w[MKD_I_A1];
}
template <class P>
__device__ __forceinline__ int task_chunks(P w) {
  const int r = task_rows(w);
  if (r == 0) return 1;
  const int rpc = op_rows_per_chunk(w[MKD_I_OP]);
  return (r + rpc - 1) / rpc;
}
// Pointer to task-local weight row r.
__device__ __forceinline__ const uint16_t* cwptr(const WeightSrc& d, int layer, int which) {
  return reinterpret_cast<const uint16_t*>(as_const(d.layer_ptrs)[layer * MKD_LAYER_PTRS + which]);
}
template <class P>
__device__ __forceinline__ const uint16_t* task_row_ptr(const WeightSrc& d, P w, int r) {
  const int op = w[MKD_I_OP], layer = w[MKD_I_LAYER], a0 = w[MKD_I_A0];
  switch (op) {
    case MKD_OP_QKV: {
      const int g = a0 + r;
      return g < QS ? cwptr(d, layer, MKD_W_Q) + (size_t)g * H
                    : (g < QS + KVS ? cwptr(d, layer, MKD_W_K) + (size_t)(g - QS) * H
                                    : cwptr(d, layer, MKD_W_V) + (size_t)(g - QS - KVS) * H);
    }
    case MKD_OP_OPROJ: return cwptr(d, layer, MKD_W_O) + (size_t)(a0 + r) * QS;
    case MKD_OP_GATEUP: return cwptr(d, layer, (r & 1) ? MKD_W_UP : MKD_W_GATE) + (size_t)(a0 + (r >> 1)) * H;
    case MKD_OP_DOWN: return cwptr(d, layer, MKD_W_DOWN) + (size_t)(a0 + r) * I;
    default: return d.embed + (size_t)(a0 + r) * H;  // LMHEAD
  }
}

// DMA wave `dw` (0..3) copies its share of chunk `j` of task `w` into `slot`.
// Returns the number of copy instructions it issued (for vmcnt bookkeeping).
// The chunk's source rows are resolved to at most two base pointers once per
// chunk (QKV chunks never straddle the q/k/v matrices; GATEUP rows alternate
// gate/up), keeping the per-copy work to address arithmetic.
__device__ __forceinline__ int dma_chunk(const WeightSrc& d, cint32_t* w, int j, uint8_t* slot, int dw) {
  const int rows = task_rows(w);
  if (rows == 0) return 0;
  const int op = w[MKD_I_OP];
  const int K = op_k(op), rpc = op_rows_per_chunk(op);
  const int r0 = j * rpc, nr = min(rpc, rows - r0);
  const int per_row = K / 512;  // 1 KiB units per row
  const int units = nr * per_row;
  const uint16_t* base0;
  const uint16_t* base1 = nullptr;
  size_t stride;
  if (op == MKD_OP_GATEUP) {
    base0 = task_row_ptr(d, w, r0);      // gate row of channel a0 + r0/2
    base1 = task_row_ptr(d, w, r0 + 1);  // up row of the same channel
    stride = H;                          // per channel
  } else {
    base0 = task_row_ptr(d, w, r0);
    stride = K;
  }
  const int lane = threadIdx.x & 63;
  int n = 0;
  for (int u = dw; u < units; u += 4) {
    const int r = u / per_row, p = u % per_row;
    const uint16_t* row = base1 != nullptr ? ((r & 1) ? base1 : base0) + (size_t)(r >> 1) * stride
                                           : base0 + (size_t)r * stride;
    __builtin_amdgcn_global_load_lds((gbl_void_t*)(row + p * 512 + lane * 8), (lds_void_t*)(slot + u * 1024), 16, 0, 0);
    n++;
  }
  return n;
}

// Rows [0, nr) of an LDS weight chunk (row-major, K) times the B activations in xs.
template <int B, int K, class Out>
__device__ __forceinline__ void chunk_gemv(const uint8_t* slot, int nr, const uint16_t* xs, Out out) {
  constexpr int C = K / 512;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int r = wave; r < nr; r += PK_CW) {
    const uint4* wrow = reinterpret_cast<const uint4*>(slot + (size_t)r * K * 2);
    float acc[B];
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = 0.f;
#pragma unroll
    for (int c = 0; c < C; c++) {
      const uint4 wv = wrow[c * 64 + lane];
#pragma unroll
      for (int b = 0; b < B; b++)
        acc[b] = dot8(wv, *reinterpret_cast<const uint4*>(xs + (size_t)b * K + (c * 64 + lane) * 8), acc[b]);
    }
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = wave_sum(acc[b]);
    out(r, acc);
  }
}

template <int B>
__device__ __forceinline__ bool cw_wait(const Ws& ws, int fanin, uint32_t target, SyncCW sync, int* sh_abort) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const uint64_t t_start = wall_clock64();
    int abort = 0;
    while (true) {
      uint32_t v = lane < FANIN_SUBSLOTS ? ld_co(ws.line(CTR_FANIN_BASE + fanin * FANIN_SUBSLOTS + lane)) : 0u;
#pragma unroll
      for (int o = 1; o < FANIN_SUBSLOTS; o <<= 1) v += __shfl_xor(v, o, 64);
      v = __shfl(v, 0, 64);
      if (v >= target) break;
      if (ld_co(ws.line(CTR_ERR)) != 0u) { abort = 1; break; }
      if (wall_clock64() - t_start > 400000000ull) {
        if (lane == 0) st_co(ws.line(CTR_ERR), 1u);
        abort = 1;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) *sh_abort = abort;
  }
  sync();
  return *sh_abort == 0;
}

// Task prologue of the compute waves: dependency wait + activation staging.
template <int B>
__device__ __forceinline__ bool cw_prologue(const MkdStepDesc& d, const Ws& ws, const Inst& w, uint16_t* xs, float* red,
                            SyncCW sync, int* sh_abort, uint64_t* tr) {
  sync();  // every compute wave is done with the previous task's xs
  const int wait = w[MKD_I_WAIT];
  if (wait >= 0 && !cw_wait<B>(ws, wait, (uint32_t)w[MKD_I_WAIT_CNT], sync, sh_abort)) return false;
  if (tr != nullptr && threadIdx.x == 0) tr[1] = wall_clock64();
  const int op = w[MKD_I_OP], layer = w[MKD_I_LAYER], a0 = w[MKD_I_A0];
  switch (op) {
    case MKD_OP_QKV:
      stage_norm<B, SyncCW>(d, ws, 2 * layer, ws.hid_f(), wptr(d, layer, MKD_W_LN_IN), xs, red, a0 == 0, sync);
      break;
    case MKD_OP_GATEUP:
      stage_norm<B, SyncCW>(d, ws, 2 * layer + 1, ws.hid_a(), wptr(d, layer, MKD_W_LN_POST), xs, red, a0 == 0, sync);
      break;
    case MKD_OP_OPROJ: stage_copy<B, QS, SyncCW>(ws.attn(), QS, xs, sync); break;
    case MKD_OP_DOWN: stage_copy<B, I, SyncCW>(ws.act(), I, xs, sync); break;
    case MKD_OP_LMHEAD:
      stage_norm<B, SyncCW>(d, ws, 2 * d.num_layers, ws.hid_f(), d.final_norm, xs, red, false, sync);
      break;
    default: break;
  }
  if (tr != nullptr && threadIdx.x == 0) tr[2] = wall_clock64();
  return true;
}

struct LmBest {
  float v;
  int i;
};

template <int B>
__device__ __forceinline__ void cw_chunk(const MkdStepDesc& d, const Ws& ws, const Inst& w, int j, const uint8_t* slot,
                         const uint16_t* xs, LmBest& best) {
  const int op = w[MKD_I_OP], a0 = w[MKD_I_A0];
  const int lane = threadIdx.x & 63;
  const int rows = task_rows(w);
  const int rpc = op_rows_per_chunk(op);
  const int r0 = j * rpc, nr = min(rpc, rows - r0);
  switch (op) {
    case MKD_OP_QKV: {
      uint16_t* out = ws.qkv();
      chunk_gemv<B, H>(slot, nr, xs, [&](int r, const float* acc) {
        if (lane < B) st_co(out + (size_t)lane * QKV_N + a0 + r0 + r, (uint16_t)f2bf(pick_lane<B>(acc, lane)));
      });
      break;
    }
    case MKD_OP_OPROJ: {
      uint16_t* out = ws.hid_a();
      chunk_gemv<B, QS>(slot, nr, xs, [&](int r, const float* acc) {
        if (lane < B) st_co(out + (size_t)lane * H + a0 + r0 + r, (uint16_t)f2bf(pick_lane<B>(acc, lane)));
      });
      break;
    }
    case MKD_OP_DOWN: {
      uint16_t* out = ws.hid_f();
      chunk_gemv<B, I>(slot, nr, xs, [&](int r, const float* acc) {
        if (lane < B) st_co(out + (size_t)lane * H + a0 + r0 + r, (uint16_t)f2bf(pick_lane<B>(acc, lane)));
      });
      break;
    }
    case MKD_OP_GATEUP: {
      // chunk rows come in (gate, up) pairs; wave w takes pair w
      uint16_t* out = ws.act();
      const int wave = threadIdx.x >> 6;
      for (int pr = wave; 2 * pr < nr; pr += PK_CW) {
        float g[B], u[B];
        {
          const uint4* grow = reinterpret_cast<const uint4*>(slot + (size_t)(2 * pr) * H * 2);
          const uint4* urow = reinterpret_cast<const uint4*>(slot + (size_t)(2 * pr + 1) * H * 2);
#pragma unroll
          for (int b = 0; b < B; b++) { g[b] = 0.f; u[b] = 0.f; }
#pragma unroll
          for (int c = 0; c < H / 512; c++) {
            const uint4 gw = grow[c * 64 + lane], uw = urow[c * 64 + lane];
#pragma unroll
            for (int b = 0; b < B; b++) {
              const uint4 x = *reinterpret_cast<const uint4*>(xs + (size_t)b * H + (c * 64 + lane) * 8);
              g[b] = dot8(gw, x, g[b]);
              u[b] = dot8(uw, x, u[b]);
            }
          }
#pragma unroll
          for (int b = 0; b < B; b++) { g[b] = wave_sum(g[b]); u[b] = wave_sum(u[b]); }
        }
        if (lane < B) {
          const float gv = round_bf(pick_lane<B>(g, lane)), uv = round_bf(pick_lane<B>(u, lane));
          st_co(out + (size_t)lane * I + a0 + (r0 >> 1) + pr, (uint16_t)f2bf(gv / (1.0f + expf(-gv)) * uv));
        }
      }
      break;
    }
    case MKD_OP_LMHEAD: {
      uint16_t* logits = d.out_logits;
      chunk_gemv<B, H>(slot, nr, xs, [&](int r, const float* acc) {
        const float v = round_bf(pick_lane<B>(acc, lane));
        const int row = a0 + r0 + r;
        if (lane < B) {
          if (lm_better(v, row, best.v, best.i)) { best.v = v; best.i = row; }
          if (logits != nullptr && lane < d.rows) logits[(size_t)lane * V + row] = (uint16_t)f2bf(v);
        }
      });
      break;
    }
    default: break;
  }
}

// LM-head epilogue: per-task partial, ticket, and (last task) the final reduction.
template <int B>
__device__ __forceinline__ void cw_lm_epilogue(const MkdStepDesc& d, const Ws& ws, const Inst& w, LmBest& best, float* red,
                               SyncCW sync) {
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  float* bv = red;
  int* bi = reinterpret_cast<int*>(red + PK_CW * MAXB);
  int* sh = bi + PK_CW * MAXB;
  if (lane < B) { bv[wave * MAXB + lane] = best.v; bi[wave * MAXB + lane] = best.i; }
  sync();
  if (t < B) {
    float v = bv[t]; int i = bi[t];
    for (int ww = 1; ww < PK_CW; ww++) {
      const float v2 = bv[ww * MAXB + t]; const int i2 = bi[ww * MAXB + t];
      if (lm_better(v2, i2, v, i)) { v = v2; i = i2; }
    }
    st_co(reinterpret_cast<uint64_t*>(ws.lmpart(w[MKD_I_A2]) + t),
          (uint64_t)__float_as_uint(v) | ((uint64_t)(uint32_t)i << 32));
  }
  drain();
  sync();
  if (t == 0) {
    const uint32_t old = add_co(ws.line(CTR_LM_TICKET), 1u);
    const bool last = old == (uint32_t)(d.lm_slots - 1);
    if (last) st_co(ws.line(CTR_LM_TICKET), 0u);
    sh[0] = last;
  }
  sync();
  if (!sh[0]) return;
  for (int b = wave; b < d.rows; b += PK_CW) {
    float v = -INFINITY; int i = 0x7fffffff;
    for (int s = lane; s < d.lm_slots; s += 64) {
      const uint64_t e = ld_co(reinterpret_cast<const uint64_t*>(ws.lmpart(s) + b));
      const float v2 = __uint_as_float((uint32_t)e); const int i2 = (int)(e >> 32);
      if (lm_better(v2, i2, v, i)) { v = v2; i = i2; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float v2 = __shfl_xor(v, o, 64); const int i2 = __shfl_xor(i, o, 64);
      if (lm_better(v2, i2, v, i)) { v = v2; i = i2; }
    }
    if (lane == 0) {
      const int tok = i == 0x7fffffff ? 0 : i;
      d.out_tokens[b] = tok;
      if (d.flags & MKD_FLAG_ADVANCE) { d.input_ids[b] = tok; d.cache_seqlens[b] += 1; }
    }
  }
  if (d.flags & MKD_FLAG_ZERO_FANIN)
    for (int f = t; f < d.num_layers * FANIN_PER_LAYER * FANIN_SUBSLOTS; f += PK_CW * 64)
      st_co(ws.line(CTR_FANIN_BASE + f), 0u);
}

// The DMA waves' loop: copy chunk c+D while chunk c is consumed. Kept out of
// line so its register allocation does not inherit the compute paths'
// pressure (a spill reload here would be a vmcnt wait on every copy).
template <int B>
__device__ __noinline__ void dma_waves(const uint64_t* layer_ptrs, const uint16_t* embed, const int32_t* row,
                                       int n_inst_arg, uint8_t* ring_arg, int dw_arg) {
  using Cfg = PkCfg<B>;
  // arguments of a device function arrive in VGPRs; pin them to SGPRs
  const WeightSrc d{uniform_ptr(layer_ptrs), uniform_ptr(embed)};
  cint32_t* crow = as_const(uniform_ptr(row));
  const int cn_inst = __builtin_amdgcn_readfirstlane(n_inst_arg);
  uint8_t* ring = uniform_ptr(ring_arg);
  const int dw = __builtin_amdgcn_readfirstlane(dw_arg);
  int win[Cfg::D + 1];
  int iss_i = 0, iss_j = 0;  // next chunk to copy
  auto issue_next = [&](int slot_idx) -> int {
    if (iss_i >= cn_inst) return 0;
    cint32_t* w = crow + iss_i * MKD_INST_WORDS;
    const int n = dma_chunk(d, w, iss_j, ring + slot_idx * SLOT_BYTES, dw);
    if (++iss_j == task_chunks(w)) { iss_j = 0; iss_i++; }
    return n;
  };
  int c = 0;
#pragma unroll
  for (int k = 0; k < Cfg::D; k++) win[k] = issue_next(k % Cfg::NS);
  for (int i = 0; i < cn_inst; i++) {
    const int nch = task_chunks(crow + i * MKD_INST_WORDS);
    for (int j = 0; j < nch; j++, c++) {
      win[Cfg::D] = issue_next((c + Cfg::D) % Cfg::NS);
      int pending = 0;
#pragma unroll
      for (int k = 1; k <= Cfg::D; k++) pending += win[k];
      wait_vmcnt(pending);
      raw_barrier();
#pragma unroll
      for (int k = 0; k < Cfg::D; k++) win[k] = win[k + 1];
    }
  }
  waitcnt_vm<0>();
}

template <int B>
__global__ __launch_bounds__(PK_THREADS, 1) void k_persistent2(MkdStepDesc d, MkdSchedule s) {
  using Cfg = PkCfg<B>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* ring = lds;
  uint16_t* xs = reinterpret_cast<uint16_t*>(lds + Cfg::NS * SLOT_BYTES);
  uint8_t* scratch = lds + Cfg::NS * SLOT_BYTES + Cfg::XS_BYTES;
  const Ws ws{reinterpret_cast<uint8_t*>(d.workspace)};
  const int n_inst = s.num_inst[blockIdx.x];
  const int32_t* row = s.inst + (size_t)blockIdx.x * s.max_inst * MKD_INST_WORDS;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  uint32_t* sync_ctr = reinterpret_cast<uint32_t*>(scratch);
  if (threadIdx.x == 0) *sync_ctr = 0u;
  raw_barrier();  // the compute-wave counter reads 0 before any wave uses it

  if (wave >= PK_CW) {
    dma_waves<B>(d.layer_ptrs, d.embed, row, n_inst, ring, wave - PK_CW);
    return;
  }

  // ---------------- compute waves ----------------
  int* sh_abort = reinterpret_cast<int*>(scratch + 64);
  float* red = reinterpret_cast<float*>(scratch + 128);
  uint8_t* attn_smem = scratch + 1024;  // 6 KiB for the attention task
  const SyncCW sync{sync_ctr};
  bool aborted = false;
  LmBest best{-INFINITY, 0x7fffffff};
  int c = 0;
  cint32_t* crow = as_const(row);
  for (int i = 0; i < n_inst; i++) {
    const Inst w = load_inst(crow + i * MKD_INST_WORDS);
    const int nch = task_chunks(w);
    const int op = w.op;
    for (int j = 0; j < nch; j++, c++) {
      uint64_t* tr = d.trace != nullptr ? d.trace + ((size_t)blockIdx.x * s.max_inst + i) * 4 : nullptr;
      if (j == 0 && !aborted) {
        if (tr != nullptr && threadIdx.x == 0) tr[0] = wall_clock64();
        aborted = !cw_prologue<B>(d, ws, w, xs, red, sync, sh_abort, tr);
      }
      raw_barrier();
      if (aborted) continue;  // keep pairing barriers with the DMA waves
      const uint8_t* slot = ring + (c % Cfg::NS) * SLOT_BYTES;
      if (op == MKD_OP_ATTN) {
        const bool produced = task_attn<B, SyncCW>(d, ws, w[MKD_I_LAYER], w[MKD_I_A0], w[MKD_I_A1], w[MKD_I_A2],
                                                   attn_smem, sync);
        if (produced && w[MKD_I_SIGNAL] >= 0) {
          drain();
          sync();
          if (threadIdx.x == 0)
            add_co(ws.line(CTR_FANIN_BASE + w[MKD_I_SIGNAL] * FANIN_SUBSLOTS + (blockIdx.x & (FANIN_SUBSLOTS - 1))), 1u);
        }
        if (tr != nullptr && threadIdx.x == 0) tr[3] = wall_clock64();
        continue;
      }
      cw_chunk<B>(d, ws, w, j, slot, xs, best);
      if (j == nch - 1) {
        if (op == MKD_OP_LMHEAD) {
          cw_lm_epilogue<B>(d, ws, w, best, red, sync);
          best = LmBest{-INFINITY, 0x7fffffff};
        } else if (w[MKD_I_SIGNAL] >= 0) {
          drain();
          sync();
          if (threadIdx.x == 0)
            add_co(ws.line(CTR_FANIN_BASE + w[MKD_I_SIGNAL] * FANIN_SUBSLOTS + (blockIdx.x & (FANIN_SUBSLOTS - 1))), 1u);
        }
        if (tr != nullptr && threadIdx.x == 0) tr[3] = wall_clock64();
      }
    }
  }
}

}  // namespace mkd
