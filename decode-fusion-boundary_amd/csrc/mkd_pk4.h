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
constexpr int P4_SCR_RES = 1024;     // float [P4_MAX_ROWS][MAXB] task results
constexpr int P4_SCR_ATTN = 2048;    // attention scratch (6 KiB)
static_assert(P4_SCR_RES + 4 * P4_MAX_ROWS * MAXB <= P4_SCR_ATTN, "result tile overlaps");
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

__device__ __forceinline__ uint32_t p4_tag(uint32_t epoch, int layer) { return (epoch + 1u) * 32u + (uint32_t)layer; }
__device__ __forceinline__ uint64_t tw_make(uint32_t lo, uint32_t tag) { return (uint64_t)lo | ((uint64_t)tag << 32); }
__device__ __forceinline__ uint32_t tw_tag(uint64_t w) { return (uint32_t)(w >> 32); }

// Compute-wave context (all fields in registers or LDS).
struct P4 {
  Ws ws;
  uint32_t epoch;
  SyncCW sync;
  int* flags;
  float* red;
  float* res;
  uint16_t* xs;
  uint8_t* attn_smem;
};

// Load N tagged words (addr(k), k < N) and spin until each carries `tag`.
// Returns false on a timeout (which it reports) or when another workgroup has
// reported an error.
template <int N, class Addr>
__device__ __forceinline__ bool poll_tagged(Addr addr, uint64_t (&v)[N], uint32_t tag, const Ws& ws) {
#pragma unroll
  for (int k = 0; k < N; k++) v[k] = ld_co(addr(k));
  uint64_t t0 = 0;
  for (uint32_t spin = 0;; spin++) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; k++) ok &= tw_tag(v[k]) == tag;
    if (ok) return true;
    if ((spin & 63u) == 0u) {
      const uint64_t now = wall_clock64();
      if (spin == 0) t0 = now;
      if (ld_co(ws.line(CTR_ERR)) != 0u) return false;
      if (now - t0 > 400000000ull) {  // 4 s at 100 MHz
        st_co(ws.line(CTR_ERR), ERR_TIMEOUT);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < N; k++)
      if (tw_tag(v[k]) != tag) v[k] = ld_co(addr(k));
  }
}

// Compute-wave barrier that also ORs an abort flag over the four waves.
__device__ __forceinline__ bool p4_agree(const P4& c, bool ok) {
  if (!ok) c.flags[0] = 1;
  c.sync();
  return c.flags[0] == 0;
}

constexpr int largest_divisor_le8(int n) {
  return n % 8 == 0 ? 8 : (n % 6 == 0 ? 6 : (n % 4 == 0 ? 4 : (n % 2 == 0 ? 2 : 1)));
}

// B rows of a tagged [MAXB][K/2] activation into xs (bf16 [B][K]).
template <int B, int K>
__device__ __forceinline__ bool p4_stage_copy(const P4& c, size_t base, uint32_t tag) {
  constexpr int PER = B * (K / 2) / 256;  // words per thread
  constexpr int NB = largest_divisor_le8(PER);
  const int t = p4_tid();
  const uint64_t* src = c.ws.tw(base);
  uint32_t* dst = reinterpret_cast<uint32_t*>(c.xs);
  bool ok = true;
#pragma unroll
  for (int k0 = 0; k0 < PER; k0 += NB) {
    uint64_t v[NB];
    ok = ok && poll_tagged<NB>([&](int k) { return src + t + 256 * (k0 + k); }, v, tag, c.ws);
#pragma unroll
    for (int k = 0; k < NB; k++) dst[t + 256 * (k0 + k)] = (uint32_t)v[k];
  }
  return p4_agree(c, ok);
}

// Residual add + RMSNorm of B rows into xs (rounding as stage_norm in mkd_tasks.h).
// from_embed: the rows are the embedding rows of input_ids (layer 0).
// Otherwise s = hidden + residual from two tagged [MAXB][H/2] buffers.
// res_out != TW_NONE: this task also publishes bf16(s) as the next residual.
template <int B>
__device__ __forceinline__ bool p4_stage_norm(const MkdStepDesc& d, const P4& c, bool from_embed, size_t hid,
                                              size_t resid, uint32_t tag_in, const uint16_t* nw, size_t res_out,
                                              uint32_t tag_out) {
  const int t = p4_tid(), wave = t >> 6, lane = t & 63;
  const int k0 = t * 4;  // features k0..k0+3 = words 2t, 2t+1 of each row
  float s[B][4];
  bool ok = true;
  if (from_embed) {
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
  } else {
    uint64_t v[4 * B];
    ok = poll_tagged<4 * B>(
        [&](int k) { return c.ws.tw(((k & 2) ? resid : hid) + (size_t)(k >> 2) * (H / 2) + 2 * t + (k & 1)); }, v,
        tag_in, c.ws);
#pragma unroll
    for (int b = 0; b < B; b++) {
      const uint32_t h0 = (uint32_t)v[4 * b], h1 = (uint32_t)v[4 * b + 1];
      const uint32_t r0 = (uint32_t)v[4 * b + 2], r1 = (uint32_t)v[4 * b + 3];
      s[b][0] = bf_lo(h0) + bf_lo(r0); s[b][1] = bf_hi(h0) + bf_hi(r0);
      s[b][2] = bf_lo(h1) + bf_lo(r1); s[b][3] = bf_hi(h1) + bf_hi(r1);
    }
  }
  if (res_out != TW_NONE && ok) {
#pragma unroll
    for (int b = 0; b < B; b++) {
      uint64_t* o = c.ws.tw(res_out + (size_t)b * (H / 2) + 2 * t);
      st_co(o, tw_make(f2bf(s[b][0]) | (f2bf(s[b][1]) << 16), tag_out));
      st_co(o + 1, tw_make(f2bf(s[b][2]) | (f2bf(s[b][3]) << 16), tag_out));
    }
  }
#pragma unroll
  for (int b = 0; b < B; b++) {
    float ss = s[b][0] * s[b][0] + s[b][1] * s[b][1] + s[b][2] * s[b][2] + s[b][3] * s[b][3];
    ss = wave_sum(ss);
    if (lane == 0) c.red[wave * MAXB + b] = ss;
  }
  if (!p4_agree(c, ok)) return false;
  const uint2 wv = *reinterpret_cast<const uint2*>(nw + k0);
  const float w4[4] = {bf_lo(wv.x), bf_hi(wv.x), bf_lo(wv.y), bf_hi(wv.y)};
#pragma unroll
  for (int b = 0; b < B; b++) {
    const float tot = c.red[b] + c.red[MAXB + b] + c.red[2 * MAXB + b] + c.red[3 * MAXB + b];
    const float r = 1.0f / sqrtf(tot * (1.0f / H) + EPS);
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = f2bf(round_bf(s[b][j] * r) * w4[j]);
    *reinterpret_cast<uint2*>(c.xs + (size_t)b * H + k0) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
  }
  c.sync();
  return true;
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

template <int B>
__device__ __forceinline__ bool p4_prologue(const MkdStepDesc& d, const P4& c, const Inst& w) {
  const int layer = w.layer;
  const uint32_t tag = p4_tag(c.epoch, layer);
  switch (w.op) {
    case MKD_OP_QKV: {
      const size_t out = w.a0 == 0 ? TW_RES1 : TW_NONE;
      const uint16_t* nw = wptr(d, layer, MKD_W_LN_IN);
      if (layer == 0) return p4_stage_norm<B>(d, c, true, 0, 0, 0, nw, out, tag);
      return p4_stage_norm<B>(d, c, false, TW_DOWN, TW_RES2, p4_tag(c.epoch, layer - 1), nw, out, tag);
    }
    case MKD_OP_GATEUP:
      return p4_stage_norm<B>(d, c, false, TW_O, TW_RES1, tag, wptr(d, layer, MKD_W_LN_POST),
                              w.a0 == 0 ? TW_RES2 : TW_NONE, tag);
    case MKD_OP_OPROJ: return p4_stage_copy<B, QS>(c, TW_ATTN, tag);
    case MKD_OP_DOWN: return p4_stage_copy<B, I>(c, TW_ACT, tag);
    case MKD_OP_LMHEAD:
      return p4_stage_norm<B>(d, c, false, TW_DOWN, TW_RES2, p4_tag(c.epoch, d.num_layers - 1), d.final_norm,
                              TW_NONE, 0);
    default: return true;
  }
}

// One LDS weight chunk of a GEMV task: rows into the result tile (LM: running argmax).
template <int B>
__device__ __forceinline__ void p4_chunk(const MkdStepDesc& d, const P4& c, const Inst& w, int j, const uint8_t* slot,
                                         LmBest& best) {
  const int lane = threadIdx.x & 63;
  const int rows = p4_rows(w);
  auto to_res = [&](int r0) {
    return [&, r0](int r, const float* acc) {
      if (lane < B) c.res[(r0 + r) * MAXB + lane] = pick_lane<B>(acc, lane);
    };
  };
  switch (w.op) {
    case MKD_OP_QKV:
    case MKD_OP_GATEUP: {
      const int r0 = j * 8;
      chunk_gemv<B, H>(slot, min(8, rows - r0), c.xs, to_res(r0));
      break;
    }
    case MKD_OP_OPROJ: {
      const int r0 = j * 4;
      chunk_gemv<B, QS>(slot, min(4, rows - r0), c.xs, to_res(r0));
      break;
    }
    case MKD_OP_DOWN: {
      const int r0 = j * 2;
      chunk_gemv<B, I>(slot, min(2, rows - r0), c.xs, to_res(r0));
      break;
    }
    case MKD_OP_LMHEAD: {
      const int r0 = j * 8;
      uint16_t* logits = d.out_logits;
      chunk_gemv<B, H>(slot, min(8, rows - r0), c.xs, [&](int r, const float* acc) {
        const float v = round_bf(pick_lane<B>(acc, lane));
        const int row = w.a0 + r0 + r;
        if (lane < B) {
          if (v > best.v || (v == best.v && row < best.i)) { best.v = v; best.i = row; }
          if (logits != nullptr && lane < d.rows) logits[(size_t)lane * V + row] = (uint16_t)f2bf(v);
        }
      });
      break;
    }
    default: break;
  }
}

// Publish a GEMV task's rows (bf16 pairs with the layer tag).
template <int B>
__device__ __forceinline__ void p4_store(const P4& c, const Inst& w) {
  c.sync();  // the result tile is complete
  const uint32_t tag = p4_tag(c.epoch, w.layer);
  const int t = p4_tid();
  const int a0 = w.a0;
  if (w.op == MKD_OP_GATEUP) {
    const int wpb = w.a1 / 2;  // channel pairs
    for (int f = t; f < B * wpb; f += PK_CW * 64) {
      const int b = f / wpb, i = f - b * wpb;
      uint32_t h[2];
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const int ch = 2 * i + e;
        const float g = round_bf(c.res[(2 * ch) * MAXB + b]);
        const float u = round_bf(c.res[(2 * ch + 1) * MAXB + b]);
        h[e] = f2bf(g / (1.0f + expf(-g)) * u);
      }
      st_co(c.ws.tw(TW_ACT + (size_t)b * (I / 2) + a0 / 2 + i), tw_make(h[0] | (h[1] << 16), tag));
    }
    return;
  }
  size_t base, stride;
  if (w.op == MKD_OP_QKV) { base = TW_QKV; stride = QKV_N / 2; }
  else if (w.op == MKD_OP_OPROJ) { base = TW_O; stride = H / 2; }
  else { base = TW_DOWN; stride = H / 2; }
  const int wpb = w.a1 / 2;
  for (int f = t; f < B * wpb; f += PK_CW * 64) {
    const int b = f / wpb, i = f - b * wpb;
    const uint32_t lo = f2bf(c.res[(2 * i) * MAXB + b]), hi = f2bf(c.res[(2 * i + 1) * MAXB + b]);
    st_co(c.ws.tw(base + (size_t)b * stride + a0 / 2 + i), tw_make(lo | (hi << 16), tag));
  }
}

// LM-head task end: publish this slot's (max, first index) per row; the last
// slot also reduces all slots to the greedy tokens and advances the epoch.
template <int B>
__device__ __forceinline__ bool p4_lm_finish(const MkdStepDesc& d, const P4& c, const Inst& w, const LmBest& best) {
  const int t = p4_tid(), wave = t >> 6, lane = t & 63;
  const uint32_t tag = p4_tag(c.epoch, w.layer);
  float* bv = c.red;
  int* bi = reinterpret_cast<int*>(c.red + PK_CW * MAXB);
  c.sync();  // red is free (earlier users are past a barrier)
  if (lane < B) { bv[wave * MAXB + lane] = best.v; bi[wave * MAXB + lane] = best.i; }
  c.sync();
  const int slot = w.a2;
  if (t < B) {
    float v = bv[t]; int i = bi[t];
    for (int ww = 1; ww < PK_CW; ww++) {
      const float v2 = bv[ww * MAXB + t]; const int i2 = bi[ww * MAXB + t];
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
    uint64_t* o = c.ws.tw(TW_LM + ((size_t)slot * MAXB + t) * 2);
    st_co(o, tw_make(__float_as_uint(v), tag));
    st_co(o + 1, tw_make((uint32_t)i, tag));
  }
  if (slot != d.lm_slots - 1) return true;
  bool ok = true;
  for (int b = wave; b < d.rows; b += PK_CW) {
    float v = -INFINITY; int i = 0x7fffffff;
    for (int s = lane; s < d.lm_slots; s += 64) {
      uint64_t e[2];
      ok = ok && poll_tagged<2>([&](int k) { return c.ws.tw(TW_LM + ((size_t)s * MAXB + b) * 2 + k); }, e, tag, c.ws);
      const float v2 = __uint_as_float((uint32_t)e[0]); const int i2 = (int)(uint32_t)e[1];
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float v2 = __shfl_xor(v, o, 64); const int i2 = __shfl_xor(i, o, 64);
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
    if (lane == 0) {
      const int tok = i == 0x7fffffff ? 0 : i;  // all-NaN row: token 0
      d.out_tokens[b] = tok;
      if (d.flags & MKD_FLAG_ADVANCE) { d.input_ids[b] = tok; d.cache_seqlens[b] += 1; }
    }
  }
  if (!p4_agree(c, ok)) return false;
  if (t == 0) st_co(c.ws.line(CTR_EPOCH), c.epoch + 1u);
  return true;
}

// ATTN task (row b, KV head h, split of nsplit): the cached K/V of the split's
// first tile is requested before this step's q/k/v words are polled (it does
// not depend on them); q/k RMSNorm + RoPE, KV write (split 0 of an active
// row), online softmax. The last split merges the others' tagged partials.
template <int B>
__device__ __forceinline__ bool p4_attn(const MkdStepDesc& d, const P4& c, int layer, int bh, int split, int nsplit) {
#ifdef MKD_PROBE_NO_ATTN
  return true;
#endif
  const int t = p4_tid(), wave = t >> 6, lane = t & 63;
  const uint32_t tag = p4_tag(c.epoch, layer);
  const int b = bh / NKV, h = bh % NKV;
  bool live = b < d.rows;
  int pos = live ? d.cache_seqlens[b] : 0;
  const int bs = d.block_size;
  if (live && (pos < 0 || pos >= MKD_MAX_POSITION || pos / bs >= d.page_stride)) {
    if (t == 0) st_co(c.ws.line(CTR_ERR), ERR_BAD_INPUT);
    live = false;
    pos = 0;
  }
  const bool active = live && d.row_active[b] != 0;
  uint8_t* smem = c.attn_smem;
  uint16_t* qb = reinterpret_cast<uint16_t*>(smem);       // [2][128] roped q
  uint16_t* kb = qb + GROUP * HD;                         // [128] roped k
  uint16_t* vb = kb + HD;                                 // [128] v
  float* mrg = reinterpret_cast<float*>(smem + 1024);     // [4][2][128]
  float* mrg_ml = mrg + PK_CW * GROUP * HD;               // [4][2] m, [4][2] l
  int* pages = reinterpret_cast<int*>(mrg_ml + 2 * PK_CW * GROUP) + 4;  // [MAX_PAGES]

  const int n_pages = live ? min(pos / bs + 1, MAX_PAGES) : 0;
  for (int i = t; i < n_pages; i += PK_CW * 64)
    pages[i] = min(max(d.page_table[(size_t)b * d.page_stride + i], 0), d.num_blocks - 1);
  c.sync();

  const int ctx = pos + 1;
  const int chunk = ((ctx + nsplit - 1) / nsplit + 63) & ~63;
  const int p_begin = split * chunk;
  const int p_end = min(ctx, p_begin + chunk);
  const int c_end = min(p_end, pos);  // cached positions of this split
  const int dg = (lane & 15) * 8, sub = lane >> 4;
  const size_t layer_off = (size_t)layer * (size_t)d.kv_layer_stride + (size_t)h * HD;
  const uint16_t* kbase = d.k_cache + layer_off;
  const uint16_t* vbase = d.v_cache + layer_off;
  uint4 kreg[HD / 8], vreg[16];
  auto load_tile = [&](int t0) {
    const int p = t0 + lane;
    const int pc = p < c_end ? p : t0;
    const uint4* krow = reinterpret_cast<const uint4*>(kbase + ((size_t)pages[pc / bs] * bs + pc % bs) * KVS);
#pragma unroll
    for (int i = 0; i < HD / 8; i++) kreg[i] = krow[i];
#pragma unroll
    for (int it = 0; it < 16; it++) {
      int pp = t0 + 4 * it + sub;
      pp = pp < c_end ? pp : t0;
      vreg[it] = *reinterpret_cast<const uint4*>(vbase + ((size_t)pages[pp / bs] * bs + pp % bs) * KVS + dg);
    }
  };
  const int first_t0 = p_begin + wave * 64;
  if (first_t0 < c_end) load_tile(first_t0);

  // this step's q (waves 0, 1: heads 2h, 2h+1), k (wave 2), v (wave 3): one word per lane
  size_t src;
  if (wave < 2) src = TW_QKV + (size_t)b * (QKV_N / 2) + (size_t)(GROUP * h + wave) * (HD / 2) + lane;
  else if (wave == 2) src = TW_QKV + (size_t)b * (QKV_N / 2) + QS / 2 + (size_t)h * (HD / 2) + lane;
  else src = TW_QKV + (size_t)b * (QKV_N / 2) + (QS + KVS) / 2 + (size_t)h * (HD / 2) + lane;
  uint64_t qv[1];
  bool ok = poll_tagged<1>([&](int) { return c.ws.tw(src); }, qv, tag, c.ws);
  const uint32_t word = (uint32_t)qv[0];  // dims 2*lane, 2*lane + 1
  uint32_t outw = word;
  if (wave < 3) {
    const float x0 = bf_lo(word), x1 = bf_hi(word);
    const uint16_t* wn = wptr(d, layer, wave < 2 ? MKD_W_Q_NORM : MKD_W_K_NORM);
    const float ss = wave_sum(x0 * x0 + x1 * x1);
    const float r = 1.0f / sqrtf(ss * (1.0f / HD) + EPS);
    const uint32_t wnw = reinterpret_cast<const uint32_t*>(wn)[lane];
    const float n0 = round_bf(round_bf(x0 * r) * bf_lo(wnw));
    const float n1 = round_bf(round_bf(x1 * r) * bf_hi(wnw));
    // rotate-half RoPE pairs dims i and i + 64: lane L holds 2L, 2L+1, lane L^32 the partners
    const float p0 = __shfl_xor(n0, 32, 64), p1 = __shfl_xor(n1, 32, 64);
    const int j = (2 * lane) & 63;
    const float* cs = d.rope_cos + (size_t)pos * (HD / 2);
    const float* sn = d.rope_sin + (size_t)pos * (HD / 2);
    const float c0 = cs[j], c1 = cs[j + 1], s0 = sn[j], s1 = sn[j + 1];
    float o0, o1;
    if (lane < 32) { o0 = n0 * c0 - p0 * s0; o1 = n1 * c1 - p1 * s1; }
    else { o0 = n0 * c0 + p0 * s0; o1 = n1 * c1 + p1 * s1; }
    outw = f2bf(o0) | (f2bf(o1) << 16);
  }
  uint16_t* dst = wave < 2 ? qb + wave * HD : (wave == 2 ? kb : vb);
  reinterpret_cast<uint32_t*>(dst)[lane] = outw;
  if (!p4_agree(c, ok)) return false;

  if (split == 0 && active && t < 128) {
    const int blk = d.page_table[(size_t)b * d.page_stride + pos / bs];
    if (blk < 0 || blk >= d.num_blocks) {
      if (t == 0) st_co(c.ws.line(CTR_ERR), ERR_BAD_INPUT);
    } else {
      const size_t slotp = (size_t)blk * bs + pos % bs;
      if (t < 64) reinterpret_cast<uint32_t*>(d.k_cache + layer_off + slotp * KVS)[t] = reinterpret_cast<const uint32_t*>(kb)[t];
      else reinterpret_cast<uint32_t*>(d.v_cache + layer_off + slotp * KVS)[t - 64] = reinterpret_cast<const uint32_t*>(vb)[t - 64];
    }
  }

  float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;
  float a0[8], a1[8];
#pragma unroll
  for (int jj = 0; jj < 8; jj++) { a0[jj] = 0.f; a1[jj] = 0.f; }
  const uint4* q0 = reinterpret_cast<const uint4*>(qb);
  const uint4* q1 = reinterpret_cast<const uint4*>(qb + HD);
  for (int t0 = first_t0; t0 < c_end; t0 += PK_CW * 64) {
    asm volatile("" ::: "memory");  // keep the q reads (LDS) inside the tile
    if (t0 != first_t0) load_tile(t0);
    const bool valid = t0 + lane < c_end;
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < HD / 8; i++) {
      s0 = dot8(kreg[i], q0[i], s0);
      s1 = dot8(kreg[i], q1[i], s1);
    }
    s0 = valid ? s0 * ATTN_SCALE : -INFINITY;
    s1 = valid ? s1 * ATTN_SCALE : -INFINITY;
    const float n0 = fmaxf(m0, wave_max(s0)), n1 = fmaxf(m1, wave_max(s1));
    const float al0 = expf(m0 - n0), al1 = expf(m1 - n1);
    const float e0 = expf(s0 - n0), e1 = expf(s1 - n1);
    l0 = l0 * al0 + wave_sum(e0);
    l1 = l1 * al1 + wave_sum(e1);
    m0 = n0; m1 = n1;
#pragma unroll
    for (int jj = 0; jj < 8; jj++) { a0[jj] *= al0; a1[jj] *= al1; }
#pragma unroll
    for (int it = 0; it < 16; it++) {
      const float w0 = __shfl(e0, 4 * it + sub, 64), w1 = __shfl(e1, 4 * it + sub, 64);
      const uint4 v = vreg[it];
      const float vf[8] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w)};
#pragma unroll
      for (int jj = 0; jj < 8; jj++) { a0[jj] += w0 * vf[jj]; a1[jj] += w1 * vf[jj]; }
    }
  }
  if (wave == 0 && p_begin <= pos && pos < p_end) {
    const uint32_t kw = reinterpret_cast<const uint32_t*>(kb)[lane];
    const float s0 = wave_sum(dot2(kw, reinterpret_cast<const uint32_t*>(qb)[lane], 0.f)) * ATTN_SCALE;
    const float s1 = wave_sum(dot2(kw, reinterpret_cast<const uint32_t*>(qb + HD)[lane], 0.f)) * ATTN_SCALE;
    const float n0 = fmaxf(m0, s0), n1 = fmaxf(m1, s1);
    const float al0 = expf(m0 - n0), al1 = expf(m1 - n1);
    const float e0 = expf(s0 - n0), e1 = expf(s1 - n1);
    l0 = l0 * al0 + e0;
    l1 = l1 * al1 + e1;
    m0 = n0; m1 = n1;
    const uint4 v = *reinterpret_cast<const uint4*>(vb + dg);
    const float vf[8] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w)};
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      a0[jj] = a0[jj] * al0 + (sub == 0 ? e0 * vf[jj] : 0.f);
      a1[jj] = a1[jj] * al1 + (sub == 0 ? e1 * vf[jj] : 0.f);
    }
  }
#pragma unroll
  for (int jj = 0; jj < 8; jj++) {
    a0[jj] += __shfl_xor(a0[jj], 16, 64); a0[jj] += __shfl_xor(a0[jj], 32, 64);
    a1[jj] += __shfl_xor(a1[jj], 16, 64); a1[jj] += __shfl_xor(a1[jj], 32, 64);
  }
  if (lane < 16) {
#pragma unroll
    for (int jj = 0; jj < 8; jj++) {
      mrg[(wave * GROUP + 0) * HD + lane * 8 + jj] = a0[jj];
      mrg[(wave * GROUP + 1) * HD + lane * 8 + jj] = a1[jj];
    }
  }
  if (lane == 0) {
    mrg_ml[wave * GROUP + 0] = m0; mrg_ml[wave * GROUP + 1] = m1;
    mrg_ml[PK_CW * GROUP + wave * GROUP + 0] = l0; mrg_ml[PK_CW * GROUP + wave * GROUP + 1] = l1;
  }
  c.sync();
  // thread t = (g, dd): head 2h + g, dim dd
  const int g = t >> 7, dd = t & 127;
  float M = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < PK_CW; ww++) M = fmaxf(M, mrg_ml[ww * GROUP + g]);
  float num = 0.f, den = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int ww = 0; ww < PK_CW; ww++) {
      const float sc = expf(mrg_ml[ww * GROUP + g] - M);
      num += mrg[(ww * GROUP + g) * HD + dd] * sc;
      den += mrg_ml[PK_CW * GROUP + ww * GROUP + g] * sc;
    }
  }
  if (nsplit > 1) {
    const size_t pbase = TW_APART + (((size_t)b * NKV + h) * MAXS) * PART_STRIDE;
    if (split != nsplit - 1) {
      uint64_t* part = c.ws.tw(pbase + (size_t)split * PART_STRIDE);
      st_co(part + g * HD + dd, tw_make(__float_as_uint(num), tag));
      if (dd == 0) {
        st_co(part + GROUP * HD + g, tw_make(__float_as_uint(M), tag));
        st_co(part + GROUP * HD + GROUP + g, tw_make(__float_as_uint(den), tag));
      }
      c.sync();  // the scratch is reused by this workgroup's next task
      return true;
    }
    // last split: fold in the other splits' partials (online, -inf = empty split)
    for (int s = 0; s < nsplit - 1; s++) {
      const size_t ps = pbase + (size_t)s * PART_STRIDE;
      uint64_t e[3];
      ok = ok && poll_tagged<3>(
                     [&](int k) {
                       return c.ws.tw(ps + (k == 0 ? (size_t)(g * HD + dd) : (size_t)(GROUP * HD + (k - 1) * GROUP + g)));
                     },
                     e, tag, c.ws);
      const float ns = __uint_as_float((uint32_t)e[0]), ms = __uint_as_float((uint32_t)e[1]);
      const float ls = __uint_as_float((uint32_t)e[2]);
      if (ms == -INFINITY) continue;
      const float nm = fmaxf(M, ms);
      const float sa = M == -INFINITY ? 0.f : expf(M - nm), sb = expf(ms - nm);
      num = num * sa + ns * sb;
      den = den * sa + ls * sb;
      M = nm;
    }
  }
  const uint32_t mine = f2bf(num / den);
  const uint32_t nbr = __shfl_xor(mine, 1, 64);
  if ((dd & 1) == 0)
    st_co(c.ws.tw(TW_ATTN + (size_t)b * (QS / 2) + ((GROUP * h + g) * HD + dd) / 2), tw_make(mine | (nbr << 16), tag));
  return p4_agree(c, ok);  // also frees the scratch for the next task
}

// ---- DMA waves -------------------------------------------------------------
template <int B, int K>
__device__ __forceinline__ void p4_dma_task(const uint16_t* base0, const uint16_t* base1, size_t stride, int rows,
                                            uint8_t* ring, int dw, int& c) {
  using Cfg = PkCfg<B>;
  constexpr int PR = K / 512;       // 1-KiB units per row
  constexpr int RPC = 16 / PR;      // rows per chunk
  constexpr int UPC = RPC * PR;     // units per chunk
  constexpr int LPW = UPC / 4;      // copies per DMA wave per chunk (4, or 3 for K = 3072)
  const int lane = threadIdx.x & 63;
  const int units = rows * PR;
  for (int u0 = 0; u0 < units; u0 += UPC) {
    uint8_t* slot = ring + (c % Cfg::NS) * SLOT_BYTES;
#pragma unroll
    for (int k = 0; k < LPW; k++) {
      const int u = min(u0 + dw + 4 * k, units - 1);  // a short last chunk repeats its last unit
      const int r = u / PR, p = u - r * PR;
      const uint16_t* row = base1 != nullptr ? ((r & 1) ? base1 : base0) + (size_t)(r >> 1) * stride
                                             : base0 + (size_t)r * stride;
      __builtin_amdgcn_global_load_lds((gbl_void_t*)(row + p * 512 + lane * 8), (lds_void_t*)(slot + (u - u0) * 1024),
                                       16, 0, 0);
    }
    if (c >= Cfg::D) {
      waitcnt_vm<3 * Cfg::D>();  // chunk c - D has landed (every later chunk issued >= 3 copies)
      raw_barrier();             // ... and is handed to the compute waves
    }
    c++;
  }
}

template <int M>
__device__ __forceinline__ void p4_dma_tail(int c) {
  // chunks c-1-M .. c-1 are still to be handed over; chunk c-1-M has M later chunks
  if constexpr (M >= 0) {
    if (M < c) {
      waitcnt_vm<3 * M>();
      raw_barrier();
    }
    p4_dma_tail<M - 1>(c);
  }
}

template <int B>
__device__ __noinline__ void p4_dma(const uint64_t* layer_ptrs, const uint16_t* embed, const int32_t* row,
                                    int n_inst_arg, uint8_t* ring_arg, int dw_arg) {
  using Cfg = PkCfg<B>;
  cuint64_t* lp = as_const(uniform_ptr(layer_ptrs));
  const uint16_t* emb = uniform_ptr(embed);
  cint32_t* crow = as_const(uniform_ptr(row));
  const int n = __builtin_amdgcn_readfirstlane(n_inst_arg);
  uint8_t* ring = uniform_ptr(ring_arg);
  const int dw = __builtin_amdgcn_readfirstlane(dw_arg);
  int c = 0;
  for (int i = 0; i < n; i++) {
    const Inst w = load_inst(crow + i * MKD_INST_WORDS);
    const int a0 = w.a0, a1 = w.a1;
    auto W = [&](int which) { return reinterpret_cast<const uint16_t*>(lp[w.layer * MKD_LAYER_PTRS + which]); };
    switch (w.op) {
      case MKD_OP_QKV: {
        const uint16_t* base = a0 < QS ? W(MKD_W_Q) + (size_t)a0 * H
                                       : (a0 < QS + KVS ? W(MKD_W_K) + (size_t)(a0 - QS) * H
                                                        : W(MKD_W_V) + (size_t)(a0 - QS - KVS) * H);
        p4_dma_task<B, H>(base, nullptr, H, a1, ring, dw, c);
        break;
      }
      case MKD_OP_OPROJ: p4_dma_task<B, QS>(W(MKD_W_O) + (size_t)a0 * QS, nullptr, QS, a1, ring, dw, c); break;
      case MKD_OP_GATEUP:
        p4_dma_task<B, H>(W(MKD_W_GATE) + (size_t)a0 * H, W(MKD_W_UP) + (size_t)a0 * H, H, 2 * a1, ring, dw, c);
        break;
      case MKD_OP_DOWN: p4_dma_task<B, I>(W(MKD_W_DOWN) + (size_t)a0 * I, nullptr, I, a1, ring, dw, c); break;
      case MKD_OP_LMHEAD: p4_dma_task<B, H>(emb + (size_t)a0 * H, nullptr, H, a1, ring, dw, c); break;
      default: break;
    }
  }
  p4_dma_tail<Cfg::D - 1>(c);
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
    flags[0] = 0;
    flags[1] = (int)ld_co(ws.line(CTR_EPOCH));
  }
  __syncthreads();
  if (wave >= PK_CW) {
    p4_dma<B>(d.layer_ptrs, d.embed, row, n_inst, ring, wave - PK_CW);
    return;
  }
  const P4 c{ws, (uint32_t)flags[1], SyncCW{reinterpret_cast<uint32_t*>(scratch)}, flags,
             reinterpret_cast<float*>(scratch + P4_SCR_RED), reinterpret_cast<float*>(scratch + P4_SCR_RES), xs,
             scratch + P4_SCR_ATTN};
  bool aborted = false;
  int cc = 0;
  cint32_t* crow = as_const(row);
  for (int i = 0; i < n_inst; i++) {
    const Inst w = load_inst(crow + i * MKD_INST_WORDS);
    uint64_t* tr = d.trace != nullptr ? d.trace + ((size_t)blockIdx.x * s.max_inst + i) * 4 : nullptr;
    if (tr != nullptr && threadIdx.x == 0) tr[0] = wall_clock64();
    if (w.op == MKD_OP_ATTN) {
      if (!aborted) aborted = !p4_attn<B>(d, c, w.layer, w.a0, w.a1, w.a2);
      if (tr != nullptr && threadIdx.x == 0) { tr[1] = tr[0]; tr[2] = tr[0]; tr[3] = wall_clock64(); }
      continue;
    }
    const int nch = p4_chunks(w);
    if (nch == 0) continue;
    if (!aborted && p4_rows(w) > P4_MAX_ROWS && w.op != MKD_OP_LMHEAD) {
      if (threadIdx.x == 0) st_co(ws.line(CTR_ERR), ERR_BAD_INST);
      aborted = true;
    }
    if (!aborted) aborted = !p4_prologue<B>(d, c, w);
    if (tr != nullptr && threadIdx.x == 0) { tr[1] = wall_clock64(); tr[2] = tr[1]; }
    LmBest best{-INFINITY, 0x7fffffff};
    for (int j = 0; j < nch; j++, cc++) {
      raw_barrier();
      if (aborted) continue;  // keep pairing barriers with the DMA waves
      p4_chunk<B>(d, c, w, j, ring + (cc % Cfg::NS) * SLOT_BYTES, best);
    }
    if (!aborted) {
      if (w.op == MKD_OP_LMHEAD) aborted = !p4_lm_finish<B>(d, c, w, best);
      else p4_store<B>(c, w);
    }
    if (tr != nullptr && threadIdx.x == 0) tr[3] = wall_clock64();
  }
}

}  // namespace mkd
