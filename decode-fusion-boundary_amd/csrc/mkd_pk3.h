// mkd_pk3.h -- persistent task-graph kernel, register-streaming variant.
//
// One 512-thread workgroup per compute unit:
//  * wave 0 is the I/O wave: it polls the dependency counters, loads and
//    normalises the activations into LDS, stores the task's results, drains
//    and arrives on the task's counter. It is the only wave that touches
//    activations in global memory.
//  * waves 1-7 hold the weights: each round of a GEMV task gives every one of
//    them a fixed 8 x 16-byte loads per lane (rows of the task's weight
//    slice; short slices re-load a valid address). The next round's loads are
//    issued before this round's dependency wait, into the other register
//    buffer, so HBM streams while wave 0 waits and stages. Their only global
//    memory operations are those weight loads, which keeps each wave's
//    in-order vmcnt queue exact (a wait for round r never waits on an
//    activation load or a store).
// Two s_barriers per round pair the waves: after wave 0 has staged the inputs,
// and after the weight waves have written their row results to LDS.
#pragma once

#include "mkd_persistent.h"

namespace mkd {

constexpr int P3_THREADS = 512;
constexpr int P3_WW = 7;    // weight waves (1..7)
constexpr int P3_UPW = 8;   // 16-byte loads per weight-wave lane per round
constexpr int P3_MAX_ROWS = P3_WW * 4;  // rows per round at most
constexpr int P3_ATTN_SMEM = 12 * 1024;

// Per-op round geometry: K, 1 KiB units per row, rows per weight wave.
template <int OP>
struct G3;
template <> struct G3<MKD_OP_QKV> { static constexpr int K = H, PER = 2, RPW = 4; };
template <> struct G3<MKD_OP_GATEUP> { static constexpr int K = H, PER = 2, RPW = 4; };
template <> struct G3<MKD_OP_LMHEAD> { static constexpr int K = H, PER = 2, RPW = 4; };
template <> struct G3<MKD_OP_OPROJ> { static constexpr int K = QS, PER = 4, RPW = 2; };
template <> struct G3<MKD_OP_DOWN> { static constexpr int K = I, PER = 6, RPW = 1; };

__device__ __forceinline__ int rows_per_round(int op) {
  return P3_WW * (op == MKD_OP_OPROJ ? 2 : (op == MKD_OP_DOWN ? 1 : 4));
}
__device__ __forceinline__ int task_rounds3(const Inst& w) {
  const int rows = task_rows(w);
  if (rows == 0) return 0;
  const int R = rows_per_round(w.op);
  return (rows + R - 1) / R;
}

// Weight wave `ww` (0..6) loads its rows of round k of task w into buf.
template <int OP>
__device__ __forceinline__ void issue_t(const WeightSrc& src, const Inst& w, int k, int ww, uint4 (&buf)[P3_UPW]) {
  using G = G3<OP>;
  const int rows = task_rows(w);
  const int row0 = k * P3_WW * G::RPW + ww * G::RPW;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < P3_UPW; i++) {
    int r = row0 + i / G::PER;
    int p = i % G::PER;
    if (i >= G::RPW * G::PER || r >= rows) {  // padding load: a valid address of this task
      r = min(row0, rows - 1);
      p = 0;
    }
    const uint16_t* rp = task_row_ptr(src, w, r);
    buf[i] = *reinterpret_cast<const uint4*>(rp + p * 512 + lane * 8);
  }
}
__device__ __forceinline__ void issue_round(const WeightSrc& src, const Inst& w, int k, int ww, uint4 (&buf)[P3_UPW]) {
  switch (w.op) {
    case MKD_OP_QKV: issue_t<MKD_OP_QKV>(src, w, k, ww, buf); break;
    case MKD_OP_GATEUP: issue_t<MKD_OP_GATEUP>(src, w, k, ww, buf); break;
    case MKD_OP_OPROJ: issue_t<MKD_OP_OPROJ>(src, w, k, ww, buf); break;
    case MKD_OP_DOWN: issue_t<MKD_OP_DOWN>(src, w, k, ww, buf); break;
    default: issue_t<MKD_OP_LMHEAD>(src, w, k, ww, buf); break;
  }
}

// Weight wave `ww` computes its rows of round k: results to res[row_in_round][b]
// (LDS), or, for the LM head, the running (max, first index) per batch row.
template <int B, int OP>
__device__ __forceinline__ void compute_t(const Inst& w, int k, int ww, const uint4 (&buf)[P3_UPW],
                                          const uint16_t* xs, float* res, LmBest& best) {
  using G = G3<OP>;
  const int rows = task_rows(w);
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int rr = 0; rr < G::RPW; rr++) {
    const int rin = ww * G::RPW + rr;              // row within the round
    const int r = k * P3_WW * G::RPW + rin;        // task-local row
    if (r >= rows) break;
    float acc[B];
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = 0.f;
#pragma unroll
    for (int p = 0; p < G::PER; p++) {
#pragma unroll
      for (int b = 0; b < B; b++)
        acc[b] = dot8(buf[rr * G::PER + p], *reinterpret_cast<const uint4*>(xs + (size_t)b * G::K + p * 512 + lane * 8), acc[b]);
    }
#pragma unroll
    for (int b = 0; b < B; b++) acc[b] = wave_sum(acc[b]);
    if constexpr (OP == MKD_OP_LMHEAD) {
      const float v = round_bf(pick_lane<B>(acc, lane));
      const int row = w.a0 + r;
      if (lane < B && (v > best.v || (v == best.v && row < best.i))) { best.v = v; best.i = row; }
    } else {
      if (lane < B) res[rin * MAXB + lane] = pick_lane<B>(acc, lane);
    }
  }
}
template <int B>
__device__ __forceinline__ void compute_round(const Inst& w, int k, int ww, const uint4 (&buf)[P3_UPW],
                                              const uint16_t* xs, float* res, LmBest& best) {
  switch (w.op) {
    case MKD_OP_QKV: compute_t<B, MKD_OP_QKV>(w, k, ww, buf, xs, res, best); break;
    case MKD_OP_GATEUP: compute_t<B, MKD_OP_GATEUP>(w, k, ww, buf, xs, res, best); break;
    case MKD_OP_OPROJ: compute_t<B, MKD_OP_OPROJ>(w, k, ww, buf, xs, res, best); break;
    case MKD_OP_DOWN: compute_t<B, MKD_OP_DOWN>(w, k, ww, buf, xs, res, best); break;
    default: compute_t<B, MKD_OP_LMHEAD>(w, k, ww, buf, xs, res, best); break;
  }
}

// Attention task of the persistent kernel, out of line so its registers are
// allocated apart from the weight buffers that stay live across it. The
// descriptor is re-read through the constant address space (scalar loads)
// from the kernel-argument address; the LDS it needs is its own.
// Copies a kernel-argument struct through the constant address space so the
// compiler fetches it with scalar loads (a generic-pointer read would be a
// per-lane vector load).
template <typename T>
__device__ __forceinline__ T load_const(uint64_t addr) {
  static_assert(sizeof(T) % 4 == 0, "dword-sized struct");
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)addr);
  typedef __attribute__((address_space(4))) const uint32_t cu32_t;
  cu32_t* p = reinterpret_cast<cu32_t*>(((uint64_t)hi << 32) | lo);
  union { T t; uint32_t w[sizeof(T) / 4]; } u;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); i++) u.w[i] = p[i];
  return u.t;
}
template <int B>
__device__ __noinline__ int attn_task_call(uint64_t desc_addr, int layer, int bh, int split, int nsplit) {
  __shared__ __attribute__((aligned(16))) uint8_t attn_smem[P3_ATTN_SMEM];
  const MkdStepDesc d = load_const<MkdStepDesc>(desc_addr);
  const Ws ws{reinterpret_cast<uint8_t*>(d.workspace)};
  const bool produced = task_attn<B, SyncAll, P3_THREADS / 64>(d, ws, layer, bh, split, nsplit, attn_smem);
  drain();
  return produced ? 1 : 0;
}

// ---- wave-0 helpers ------------------------------------------------------------
// Dependency wait by wave 0 alone. Returns false on timeout / device error.
__device__ __forceinline__ bool w0_wait(const Ws& ws, int fanin, uint32_t target) {
  const int lane = threadIdx.x & 63;
  const uint64_t t_start = wall_clock64();
  while (true) {
    uint32_t v = lane < FANIN_SUBSLOTS ? ld_co(ws.line(CTR_FANIN_BASE + fanin * FANIN_SUBSLOTS + lane)) : 0u;
#pragma unroll
    for (int o = 1; o < FANIN_SUBSLOTS; o <<= 1) v += __shfl_xor(v, o, 64);
    if (__shfl(v, 0, 64) >= target) return true;
    if (ld_co(ws.line(CTR_ERR)) != 0u) return false;
    if (wall_clock64() - t_start > 400000000ull) {
      if (lane == 0) st_co(ws.line(CTR_ERR), ERR_TIMEOUT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Residual add + RMSNorm of B rows by wave 0 (16 features per lane), into xs.
template <int B, int B0 = 0, int NB = B>
__device__ __forceinline__ void w0_norm_rows(const MkdStepDesc& d, const Ws& ws, int norm_idx, const uint16_t* hidden,
                                             const uint16_t* wln, uint16_t* xs, bool write_resid) {
  const int lane = threadIdx.x & 63;
  const int k0 = lane * 16;
  uint32_t hv[NB][8], rv[NB][8];
#pragma unroll
  for (int bb = 0; bb < NB; bb++) {
    const int b = B0 + bb;
    if (norm_idx == 0) {
      int64_t id = b < d.rows ? d.input_ids[b] : 0;
      if (id < 0 || id >= V) {
        if (lane == 0) st_co(ws.line(CTR_ERR), ERR_BAD_INPUT);
        id = 0;
      }
      const uint4* e = reinterpret_cast<const uint4*>(d.embed + (size_t)id * H + k0);
      const uint4 e0 = e[0], e1 = e[1];
      hv[bb][0] = e0.x; hv[bb][1] = e0.y; hv[bb][2] = e0.z; hv[bb][3] = e0.w;
      hv[bb][4] = e1.x; hv[bb][5] = e1.y; hv[bb][6] = e1.z; hv[bb][7] = e1.w;
#pragma unroll
      for (int j = 0; j < 8; j++) rv[bb][j] = 0u;
    } else {
      const uint64_t* hp = reinterpret_cast<const uint64_t*>(hidden + (size_t)b * H + k0);
      const uint64_t* rp = reinterpret_cast<const uint64_t*>(ws.resid(norm_idx) + (size_t)b * H + k0);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint64_t a = ld_co(hp + j), c = ld_co(rp + j);
        hv[bb][2 * j] = (uint32_t)a; hv[bb][2 * j + 1] = (uint32_t)(a >> 32);
        rv[bb][2 * j] = (uint32_t)c; rv[bb][2 * j + 1] = (uint32_t)(c >> 32);
      }
    }
  }
  uint32_t wv[8];
  {
    const uint4* wp = reinterpret_cast<const uint4*>(wln + k0);
    const uint4 w0 = wp[0], w1 = wp[1];
    wv[0] = w0.x; wv[1] = w0.y; wv[2] = w0.z; wv[3] = w0.w; wv[4] = w1.x; wv[5] = w1.y; wv[6] = w1.z; wv[7] = w1.w;
  }
  uint16_t* rout = ws.resid(norm_idx + 1);
#pragma unroll
  for (int bb = 0; bb < NB; bb++) {
    const int b = B0 + bb;
    float s[16];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      s[2 * j] = bf_lo(hv[bb][j]) + bf_lo(rv[bb][j]);
      s[2 * j + 1] = bf_hi(hv[bb][j]) + bf_hi(rv[bb][j]);
      ss += s[2 * j] * s[2 * j] + s[2 * j + 1] * s[2 * j + 1];
    }
    if (write_resid) {
      uint64_t* op = reinterpret_cast<uint64_t*>(rout + (size_t)b * H + k0);
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t lo = f2bf(s[4 * j]) | (f2bf(s[4 * j + 1]) << 16);
        const uint32_t hi = f2bf(s[4 * j + 2]) | (f2bf(s[4 * j + 3]) << 16);
        st_co(op + j, (uint64_t)lo | ((uint64_t)hi << 32));
      }
    }
    const float r = 1.0f / sqrtf(wave_sum(ss) * (1.0f / H) + EPS);
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t a = f2bf(round_bf(s[2 * j] * r) * bf_lo(wv[j]));
      const uint32_t c = f2bf(round_bf(s[2 * j + 1] * r) * bf_hi(wv[j]));
      o[j] = a | (c << 16);
    }
    uint4* xp = reinterpret_cast<uint4*>(xs + (size_t)b * H + k0);
    xp[0] = make_uint4(o[0], o[1], o[2], o[3]);
    xp[1] = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

template <int B>
__device__ __forceinline__ void w0_norm(const MkdStepDesc& d, const Ws& ws, int norm_idx, const uint16_t* hidden,
                                        const uint16_t* wln, uint16_t* xs, bool write_resid) {
  if constexpr (B <= 4) {
    w0_norm_rows<B>(d, ws, norm_idx, hidden, wln, xs, write_resid);
  } else {
    w0_norm_rows<B, 0, B / 2>(d, ws, norm_idx, hidden, wln, xs, write_resid);
    w0_norm_rows<B, B / 2, B / 2>(d, ws, norm_idx, hidden, wln, xs, write_resid);
  }
}

// Copy B rows of a bf16 activation [B][K] into xs by wave 0 (64-bit coherent loads).
template <int B, int K>
__device__ __forceinline__ void w0_copy(const uint16_t* src, uint16_t* xs) {
  constexpr int PER_LANE = K / 4 / 64;  // 64-bit words per lane per row
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int b = 0; b < B; b++) {
    uint64_t v[PER_LANE];
    const uint64_t* sp = reinterpret_cast<const uint64_t*>(src + (size_t)b * K);
#pragma unroll
    for (int j = 0; j < PER_LANE; j++) v[j] = ld_co(sp + j * 64 + lane);
    uint64_t* dp = reinterpret_cast<uint64_t*>(xs + (size_t)b * K);
#pragma unroll
    for (int j = 0; j < PER_LANE; j++) dp[j * 64 + lane] = v[j];
  }
}

template <int B>
__device__ __forceinline__ bool w0_prologue(const MkdStepDesc& d, const Ws& ws, const Inst& w, uint16_t* xs,
                                            uint64_t* tr) {
  if (w.wait >= 0 && !w0_wait(ws, w.wait, (uint32_t)w.wait_cnt)) return false;
  if (tr != nullptr && (threadIdx.x & 63) == 0) tr[1] = wall_clock64();
  switch (w.op) {
    case MKD_OP_QKV:
      w0_norm<B>(d, ws, 2 * w.layer, ws.hid_f(), wptr(d, w.layer, MKD_W_LN_IN), xs, w.a0 == 0);
      break;
    case MKD_OP_GATEUP:
      w0_norm<B>(d, ws, 2 * w.layer + 1, ws.hid_a(), wptr(d, w.layer, MKD_W_LN_POST), xs, w.a0 == 0);
      break;
    case MKD_OP_OPROJ: w0_copy<B, QS>(ws.attn(), xs); break;
    case MKD_OP_DOWN: w0_copy<B, I>(ws.act(), xs); break;
    case MKD_OP_LMHEAD: w0_norm<B>(d, ws, 2 * d.num_layers, ws.hid_f(), d.final_norm, xs, false); break;
    default: break;
  }
  if (tr != nullptr && (threadIdx.x & 63) == 0) tr[2] = wall_clock64();
  return true;
}

// Wave 0 stores round k's results (bf16) from res.
template <int B>
__device__ __forceinline__ void w0_store_round(const Ws& ws, const Inst& w, int k, const float* res) {
  const int lane = threadIdx.x & 63;
  const int R = rows_per_round(w.op);
  const int rows = task_rows(w);
  const int nr = min(R, rows - k * R);
  if (w.op == MKD_OP_GATEUP) {
    const int np = nr / 2;
    const int c0 = w.a0 + (k * R) / 2;
    for (int e = lane; e < np * B; e += 64) {
      const int pr = e / B, b = e % B;
      const float g = round_bf(res[(2 * pr) * MAXB + b]), u = round_bf(res[(2 * pr + 1) * MAXB + b]);
      st_co(ws.act() + (size_t)b * I + c0 + pr, (uint16_t)f2bf(g / (1.0f + expf(-g)) * u));
    }
    return;
  }
  uint16_t* out;
  int ld;
  switch (w.op) {
    case MKD_OP_QKV: out = ws.qkv(); ld = QKV_N; break;
    case MKD_OP_OPROJ: out = ws.hid_a(); ld = H; break;
    default: out = ws.hid_f(); ld = H; break;  // DOWN
  }
  const int r0 = w.a0 + k * R;
  for (int e = lane; e < nr * B; e += 64) {
    const int rr = e / B, b = e % B;
    st_co(out + (size_t)b * ld + r0 + rr, (uint16_t)f2bf(res[rr * MAXB + b]));
  }
}

__device__ __forceinline__ void w0_signal(const Ws& ws, int signal) {
  drain();
  if ((threadIdx.x & 63) == 0 && signal >= 0)
    add_co(ws.line(CTR_FANIN_BASE + signal * FANIN_SUBSLOTS + (blockIdx.x & (FANIN_SUBSLOTS - 1))), 1u);
}

// LM-head finish by wave 0: combine the weight waves' (max, first index), write
// this task's partial, take the ticket; the last task reduces all partials.
template <int B>
__device__ __forceinline__ void w0_lm_finish(const MkdStepDesc& d, const Ws& ws, const Inst& w, const float* lm_v,
                                             const int* lm_i) {
  const int lane = threadIdx.x & 63;
  if (lane < B) {
    float v = lm_v[lane]; int i = lm_i[lane];
    for (int ww = 1; ww < P3_WW; ww++) {
      const float v2 = lm_v[ww * MAXB + lane]; const int i2 = lm_i[ww * MAXB + lane];
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
    st_co(reinterpret_cast<uint64_t*>(ws.lmpart(w.a2) + lane), (uint64_t)__float_as_uint(v) | ((uint64_t)(uint32_t)i << 32));
  }
  drain();
  uint32_t old = 0;
  if (lane == 0) old = add_co(ws.line(CTR_LM_TICKET), 1u);
  old = __shfl(old, 0, 64);
  if (old != (uint32_t)(d.lm_slots - 1)) return;
  if (lane == 0) st_co(ws.line(CTR_LM_TICKET), 0u);
  for (int b = 0; b < d.rows; b++) {
    float v = -INFINITY; int i = 0x7fffffff;
    for (int s = lane; s < d.lm_slots; s += 64) {
      const uint64_t e = ld_co(reinterpret_cast<const uint64_t*>(ws.lmpart(s) + b));
      const float v2 = __uint_as_float((uint32_t)e); const int i2 = (int)(e >> 32);
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float v2 = __shfl_xor(v, o, 64); const int i2 = __shfl_xor(i, o, 64);
      if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
    }
    if (lane == 0) {
      const int tok = i == 0x7fffffff ? 0 : i;
      d.out_tokens[b] = tok;
      if (d.flags & MKD_FLAG_ADVANCE) { d.input_ids[b] = tok; d.cache_seqlens[b] += 1; }
    }
  }
  if (d.flags & MKD_FLAG_ZERO_FANIN)
    for (int f = lane; f < d.num_layers * FANIN_PER_LAYER * FANIN_SUBSLOTS; f += 64)
      st_co(ws.line(CTR_FANIN_BASE + f), 0u);
}

// LDS shared by the two role loops (namespace scope so both functions see it).
__shared__ __attribute__((aligned(16))) uint16_t p3_xs[MAXB * I];
__shared__ float p3_res[P3_MAX_ROWS * MAXB];
__shared__ float p3_lm_v[P3_WW * MAXB];
__shared__ int p3_lm_i[P3_WW * MAXB];
__shared__ int p3_abort;

// Wave 0: dependency waits, staging, result stores, arrivals.
template <int B>
__device__ __noinline__ void p3_io_wave(uint64_t desc_addr, uint64_t sched_addr) {
  const MkdStepDesc d = load_const<MkdStepDesc>(desc_addr);
  const MkdSchedule s = load_const<MkdSchedule>(sched_addr);
  const Ws ws{reinterpret_cast<uint8_t*>(d.workspace)};
  cint32_t* crow = as_const(s.inst) + (size_t)blockIdx.x * s.max_inst * MKD_INST_WORDS;
  const int n = as_const(s.num_inst)[blockIdx.x];
  const int lane = threadIdx.x & 63;
  for (int i = 0; i < n; i++) {
    const Inst w = load_inst(crow + i * MKD_INST_WORDS);
    uint64_t* tr = d.trace != nullptr ? d.trace + ((size_t)blockIdx.x * s.max_inst + i) * 4 : nullptr;
    if (tr != nullptr && lane == 0) tr[0] = wall_clock64();
    if (w.op == MKD_OP_ATTN) {
      const bool ok = w.wait < 0 || w0_wait(ws, w.wait, (uint32_t)w.wait_cnt);
      if (!ok && lane == 0) p3_abort = 1;
      __syncthreads();
      if (p3_abort) return;
      if (tr != nullptr && lane == 0) { tr[1] = wall_clock64(); tr[2] = tr[1]; }
      const bool produced = attn_task_call<B>(desc_addr, w.layer, w.a0, w.a1, w.a2) != 0;
      __syncthreads();
      if (produced) w0_signal(ws, w.signal);
      if (tr != nullptr && lane == 0) tr[3] = wall_clock64();
      continue;
    }
    const int rounds = task_rounds3(w);
    for (int k = 0; k < rounds; k++) {
      const bool last = k == rounds - 1;
      if (k == 0 && !w0_prologue<B>(d, ws, w, p3_xs, tr) && lane == 0) p3_abort = 1;
      raw_barrier();  // #1: inputs staged
      if (p3_abort) return;
      raw_barrier();  // #2: weight waves' results in LDS
      if (w.op == MKD_OP_LMHEAD) {
        if (last) w0_lm_finish<B>(d, ws, w, p3_lm_v, p3_lm_i);
      } else {
        w0_store_round<B>(ws, w, k, p3_res);
        if (last) w0_signal(ws, w.signal);
      }
      if (last && tr != nullptr && lane == 0) tr[3] = wall_clock64();
    }
  }
}

// Waves 1-7: weight streaming (double-buffered registers) and the dot products.
template <int B>
__device__ __noinline__ void p3_weight_wave(uint64_t desc_addr, uint64_t sched_addr, int ww_arg) {
  const MkdStepDesc d = load_const<MkdStepDesc>(desc_addr);
  const MkdSchedule s = load_const<MkdSchedule>(sched_addr);
  const int ww = __builtin_amdgcn_readfirstlane(ww_arg);
  const WeightSrc src{d.layer_ptrs, d.embed};
  cint32_t* crow = as_const(s.inst) + (size_t)blockIdx.x * s.max_inst * MKD_INST_WORDS;
  const int n = as_const(s.num_inst)[blockIdx.x];
  const int lane = threadIdx.x & 63;
  int pi = 0, pk = 0;  // next GEMV round to load
  auto skip_to_gemv = [&]() {
    while (pi < n && task_rounds3(load_inst(crow + pi * MKD_INST_WORDS)) == 0) pi++;
  };
  auto issue_next = [&](uint4 (&buf)[P3_UPW]) {
    if (pi >= n) return;
    const Inst w = load_inst(crow + pi * MKD_INST_WORDS);
    issue_round(src, w, pk, ww, buf);
    if (++pk == task_rounds3(w)) { pk = 0; pi++; skip_to_gemv(); }
  };
  uint4 bufA[P3_UPW], bufB[P3_UPW];
  skip_to_gemv();
  issue_next(bufA);
  LmBest best{-INFINITY, 0x7fffffff};
  int g = 0;
  for (int i = 0; i < n; i++) {
    const Inst w = load_inst(crow + i * MKD_INST_WORDS);
    if (w.op == MKD_OP_ATTN) {
      __syncthreads();
      if (p3_abort) return;
      attn_task_call<B>(desc_addr, w.layer, w.a0, w.a1, w.a2);
      __syncthreads();
      continue;
    }
    const int rounds = task_rounds3(w);
    for (int k = 0; k < rounds; k++, g++) {
      const bool last = k == rounds - 1;
      if (g & 1) issue_next(bufA); else issue_next(bufB);
      raw_barrier();  // #1
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      if (p3_abort) return;
      if (g & 1) compute_round<B>(w, k, ww, bufB, p3_xs, p3_res, best);
      else compute_round<B>(w, k, ww, bufA, p3_xs, p3_res, best);
      if (w.op == MKD_OP_LMHEAD && last) {
        if (lane < B) { p3_lm_v[ww * MAXB + lane] = best.v; p3_lm_i[ww * MAXB + lane] = best.i; }
        best = LmBest{-INFINITY, 0x7fffffff};
      }
      raw_barrier();  // #2
    }
  }
}

// The role loops read the kernel arguments from the kernarg segment itself.
// Taking `&d` of a by-value kernel parameter would instead give the address of
// a private (scratch) copy, which constant-address-space loads cannot reach.
constexpr size_t P3_SCHED_ARG_OFF =
    (sizeof(MkdStepDesc) + alignof(MkdSchedule) - 1) / alignof(MkdSchedule) * alignof(MkdSchedule);

template <int B>
__global__ __launch_bounds__(P3_THREADS, 1) void k_persistent3(MkdStepDesc d, MkdSchedule s) {
  (void)d;
  (void)s;
  if (threadIdx.x == 0) p3_abort = 0;
  __syncthreads();
  const uint64_t karg = reinterpret_cast<uint64_t>(__builtin_amdgcn_kernarg_segment_ptr());
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave == 0) p3_io_wave<B>(karg, karg + P3_SCHED_ARG_OFF);
  else p3_weight_wave<B>(karg, karg + P3_SCHED_ARG_OFF, wave - 1);
}

}  // namespace mkd
