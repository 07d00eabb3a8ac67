// mkd_tasks.h -- the decode-step task bodies shared by the persistent kernel and
// the per-op kernels. One workgroup (256 threads, 4 wave64) runs one task.
//
// Rounding points follow the reference torch path (models/qwen3.py:147-160,
// layers/layernorm.py:16-40, rotary_embedding.py:6-14, activation.py:6-11,
// embed_head.py:56-66, sampler.py:5-16): bf16 between ops, fp32 inside norms,
// RoPE and softmax, fp32 accumulation of bf16 products, bf16 logits, greedy
// argmax = first maximal index.
#pragma once

#include "mkd_common.h"

namespace mkd {

constexpr int SMEM_BYTES = MAXB * I * 2 + 4096;  // activation tile + reduction scratch

// Workgroup-wide barrier (per-op kernels: every thread runs the task).
struct SyncAll {
  __device__ __forceinline__ void operator()() const { __syncthreads(); }
};
constexpr float ATTN_SCALE = 0.08838834764831845f;  // 128 ** -0.5
constexpr int MAX_PAGES = 64;  // block-table entries staged per attention task (>= 2048 / block_size)

__device__ __forceinline__ const uint16_t* wptr(const MkdStepDesc& d, int layer, int which) {
  return reinterpret_cast<const uint16_t*>(d.layer_ptrs[layer * MKD_LAYER_PTRS + which]);
}

// ---------------------------------------------------------------------------
// Residual add + RMSNorm of B rows into LDS (bf16 [B][H]).
//   norm_idx 2l: input norm of layer l (l == 0 reads the embedding rows),
//   2l+1: post-attention norm, 2*num_layers: final norm.
// s = hidden + residual in fp32; xs = bf16(bf16(s * rsqrt(mean(s^2)+eps)) * w);
// when write_resid, the new residual bf16(s) goes to resid(norm_idx + 1).
// ---------------------------------------------------------------------------
template <int B, class Sync = SyncAll>
__device__ void stage_norm(const MkdStepDesc& d, const Ws& ws, int norm_idx,
                           const uint16_t* hidden, const uint16_t* w, uint16_t* xs,
                           float* red, bool write_resid, Sync sync = Sync()) {
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int k0 = t * 4;  // 4 consecutive features per thread
  float s[B][4];
  if (norm_idx == 0) {
#pragma unroll
    for (int b = 0; b < B; b++) {
      int64_t id = b < d.rows ? d.input_ids[b] : 0;
      if (id < 0 || id >= V) {
        if (threadIdx.x == 0) st_co(ws.line(CTR_ERR), ERR_BAD_INPUT);
        id = 0;
      }
      const uint2 e = *reinterpret_cast<const uint2*>(d.embed + (size_t)id * H + k0);
      s[b][0] = bf_lo(e.x); s[b][1] = bf_hi(e.x); s[b][2] = bf_lo(e.y); s[b][3] = bf_hi(e.y);
    }
  } else {
    const uint16_t* res = ws.resid(norm_idx);
#pragma unroll
    for (int b = 0; b < B; b++) {
      const uint64_t hv = ld_co(reinterpret_cast<const uint64_t*>(hidden + (size_t)b * H + k0));
      const uint64_t rv = ld_co(reinterpret_cast<const uint64_t*>(res + (size_t)b * H + k0));
      const uint32_t h0 = (uint32_t)hv, h1 = (uint32_t)(hv >> 32);
      const uint32_t r0 = (uint32_t)rv, r1 = (uint32_t)(rv >> 32);
      s[b][0] = bf_lo(h0) + bf_lo(r0); s[b][1] = bf_hi(h0) + bf_hi(r0);
      s[b][2] = bf_lo(h1) + bf_lo(r1); s[b][3] = bf_hi(h1) + bf_hi(r1);
    }
  }
  if (write_resid) {
    uint16_t* out = ws.resid(norm_idx + 1);
#pragma unroll
    for (int b = 0; b < B; b++) {
      const uint64_t v = (uint64_t)(f2bf(s[b][0]) | (f2bf(s[b][1]) << 16)) |
                         ((uint64_t)(f2bf(s[b][2]) | (f2bf(s[b][3]) << 16)) << 32);
      st_co(reinterpret_cast<uint64_t*>(out + (size_t)b * H + k0), v);
    }
  }
#pragma unroll
  for (int b = 0; b < B; b++) {
    float ss = s[b][0] * s[b][0] + s[b][1] * s[b][1] + s[b][2] * s[b][2] + s[b][3] * s[b][3];
    ss = wave_sum(ss);
    if (lane == 0) red[wave * MAXB + b] = ss;
  }
  sync();
  const uint2 wv = *reinterpret_cast<const uint2*>(w + k0);
  const float w4[4] = {bf_lo(wv.x), bf_hi(wv.x), bf_lo(wv.y), bf_hi(wv.y)};
#pragma unroll
  for (int b = 0; b < B; b++) {
    const float tot = red[b] + red[MAXB + b] + red[2 * MAXB + b] + red[3 * MAXB + b];
    const float r = 1.0f / sqrtf(tot * (1.0f / H) + EPS);
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = f2bf(round_bf(s[b][j] * r) * w4[j]);
    *reinterpret_cast<uint2*>(xs + (size_t)b * H + k0) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
  }
  sync();
}

// Copy B rows of a bf16 activation [B][K] (row stride ld) from global into LDS.
template <int B, int K, class Sync = SyncAll>
__device__ void stage_copy(const uint16_t* src, int ld, uint16_t* xs, Sync sync = Sync()) {
  constexpr int PER_ROW = K / 4;  // 64-bit words per row
  for (int i = threadIdx.x; i < B * PER_ROW; i += NT) {
    const int b = i / PER_ROW, c = i % PER_ROW;
    reinterpret_cast<uint64_t*>(xs + (size_t)b * K)[c] =
        ld_co(reinterpret_cast<const uint64_t*>(src + (size_t)b * ld) + c);
  }
  sync();
}

// ---------------------------------------------------------------------------
// Row-block GEMV: y[b][r] = sum_k W[r][k] * x[b][k] for rows r in [r0, r0+nr).
// Each wave takes RU consecutive rows at a time; a wave64 covers 1 KiB of a
// row per load (16 B per lane, fully coalesced) and keeps RU*K/512 loads in
// flight per lane. x is read from LDS as 16-byte vectors (conflict-free).
// `out(row, acc)` receives the wave-reduced sums acc[B] (every lane holds them).
// ---------------------------------------------------------------------------
template <int B, int K, int RU, class RowPtr, class Out>
__device__ __forceinline__ void gemv(RowPtr rowptr, int r0, int nr, const uint16_t* xs, Out out) {
  constexpr int C = K / 512;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int base = wave * RU; base < nr; base += NWAVE * RU) {
    uint4 w[RU][C];
#pragma unroll
    for (int u = 0; u < RU; u++) {
      const int r = base + u < nr ? base + u : nr - 1;
      const uint4* p = reinterpret_cast<const uint4*>(rowptr(r0 + r));
#pragma unroll
      for (int c = 0; c < C; c++) w[u][c] = p[c * 64 + lane];
    }
    float acc[RU][B];
#pragma unroll
    for (int u = 0; u < RU; u++)
#pragma unroll
      for (int b = 0; b < B; b++) acc[u][b] = 0.f;
#pragma unroll
    for (int c = 0; c < C; c++) {
#pragma unroll
      for (int b = 0; b < B; b++) {
        const uint4 x = *reinterpret_cast<const uint4*>(xs + (size_t)b * K + (c * 64 + lane) * 8);
#pragma unroll
        for (int u = 0; u < RU; u++) acc[u][b] = dot8(w[u][c], x, acc[u][b]);
      }
    }
#pragma unroll
    for (int u = 0; u < RU; u++) {
#pragma unroll
      for (int b = 0; b < B; b++) acc[u][b] = wave_sum(acc[u][b]);
      if (base + u < nr) out(r0 + base + u, acc[u]);
    }
  }
}

// Value of acc[b] for b == lane (lanes >= B get acc[0]); avoids dynamic indexing.
template <int B>
__device__ __forceinline__ float pick_lane(const float* acc, int lane) {
  float v = acc[0];
#pragma unroll
  for (int b = 1; b < B; b++) v = lane == b ? acc[b] : v;
  return v;
}

// ---------------------------------------------------------------------------
// QKV: norm (residual add) + rows [r0, r0+nr) of [Wq; Wk; Wv] -> qkv bf16.
// ---------------------------------------------------------------------------
template <int B>
__device__ void task_qkv(const MkdStepDesc& d, const Ws& ws, int layer, int r0, int nr, uint8_t* smem) {
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* red = reinterpret_cast<float*>(smem + MAXB * I * 2);
  stage_norm<B>(d, ws, 2 * layer, ws.hid_f(), wptr(d, layer, MKD_W_LN_IN), xs, red, r0 == 0);
  const uint16_t* wq = wptr(d, layer, MKD_W_Q);
  const uint16_t* wk = wptr(d, layer, MKD_W_K);
  const uint16_t* wv = wptr(d, layer, MKD_W_V);
  uint16_t* out = ws.qkv();
  const int lane = threadIdx.x & 63;
  auto rowptr = [&](int r) -> const uint16_t* {
    return r < QS ? wq + (size_t)r * H : (r < QS + KVS ? wk + (size_t)(r - QS) * H : wv + (size_t)(r - QS - KVS) * H);
  };
  gemv<B, H, 4>(rowptr, r0, nr, xs, [&](int r, const float* acc) {
    if (lane < B) st_co(out + (size_t)lane * QKV_N + r, (uint16_t)f2bf(pick_lane<B>(acc, lane)));
  });
}

// Plain projection rows: OPROJ (K = 2048, input attn) and DOWN (K = 3072, input act).
template <int B, int K>
__device__ void task_proj(const uint16_t* W, const uint16_t* in, uint16_t* out, int r0, int nr, uint8_t* smem) {
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  stage_copy<B, K>(in, K, xs);
  const int lane = threadIdx.x & 63;
  auto rowptr = [&](int r) -> const uint16_t* { return W + (size_t)r * K; };
  gemv<B, K, 1>(rowptr, r0, nr, xs, [&](int r, const float* acc) {
    if (lane < B) st_co(out + (size_t)lane * H + r, (uint16_t)f2bf(pick_lane<B>(acc, lane)));
  });
}

// GATEUP: norm (post-attention) + channels [c0, c0+nc) of gate and up + SiLU*mul.
template <int B>
__device__ void task_gateup(const MkdStepDesc& d, const Ws& ws, int layer, int c0, int nc, uint8_t* smem) {
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* red = reinterpret_cast<float*>(smem + MAXB * I * 2);
  stage_norm<B>(d, ws, 2 * layer + 1, ws.hid_a(), wptr(d, layer, MKD_W_LN_POST), xs, red, c0 == 0);
  const uint16_t* wg = wptr(d, layer, MKD_W_GATE);
  const uint16_t* wu = wptr(d, layer, MKD_W_UP);
  uint16_t* out = ws.act();
  const int lane = threadIdx.x & 63;
  // Row 2j is gate channel j, row 2j+1 is up channel j: each wave owns whole pairs.
  auto rowptr = [&](int r) -> const uint16_t* { return ((r & 1) ? wu : wg) + (size_t)(r >> 1) * H; };
  float gate_keep[B];
  gemv<B, H, 2>(rowptr, 2 * c0, 2 * nc, xs, [&](int r, const float* acc) {
    if ((r & 1) == 0) {
#pragma unroll
      for (int b = 0; b < B; b++) gate_keep[b] = acc[b];
    } else if (lane < B) {
      const float g = round_bf(pick_lane<B>(gate_keep, lane));
      const float u = round_bf(pick_lane<B>(acc, lane));
      const float a = g / (1.0f + expf(-g)) * u;
      st_co(out + (size_t)lane * I + (r >> 1), (uint16_t)f2bf(a));
    }
  });
}

// ---------------------------------------------------------------------------
// ATTN: one (row, kv head, split). q/k RMSNorm + RoPE of the new token, KV
// write (split 0 of an active row), online-softmax attention over the split's
// positions; splits are merged by the last arriving split (ticket counter).
// Returns true when this workgroup produced the final attention output.
// ---------------------------------------------------------------------------
template <int B, class Sync = SyncAll, int NW = NWAVE>
__device__ __forceinline__ bool task_attn(const MkdStepDesc& d, const Ws& ws, int layer, int bh, int split, int nsplit,
                          uint8_t* smem, Sync sync = Sync()) {
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const int b = bh / NKV, h = bh % NKV;
  bool live = b < d.rows;
  int pos = live ? d.cache_seqlens[b] : 0;
  const int bs = d.block_size;
  if (live && (pos < 0 || pos >= MKD_MAX_POSITION || pos / bs >= d.page_stride)) {
    // Out-of-range position: record it, and run the row as an inactive
    // position-0 row so no address leaves the cache, table or RoPE rows.
    if (threadIdx.x == 0) st_co(ws.line(CTR_ERR), ERR_BAD_INPUT);
    live = false;
    pos = 0;
  }
  const bool active = live && d.row_active[b] != 0;
  const int nblk = d.num_blocks;

  uint16_t* qb = reinterpret_cast<uint16_t*>(smem);          // [2][128] roped q (bf16)
  uint16_t* kb = qb + GROUP * HD;                            // [128] roped k
  uint16_t* vb = kb + HD;                                    // [128] v
  float* mrg = reinterpret_cast<float*>(smem + 1024);        // [4 waves][2][128] + m/l
  float* mrg_ml = mrg + NW * GROUP * HD;                     // [NW][2] m, [NW][2] l
  int* sh = reinterpret_cast<int*>(mrg_ml + 2 * NW * GROUP);
  int* pages = sh + 4;                                       // [MAX_PAGES] this row's physical blocks

  // -- the row's block table (clamped to the cache) into LDS; q/k norm + RoPE
  //    (waves 0,1: q heads 2h, 2h+1; wave 2: k; wave 3: v copy)
  {
    const int n_pages = live ? min(pos / d.block_size + 1, MAX_PAGES) : 0;
    for (int i = t; i < n_pages; i += NW * 64) {
      // a block id outside the cache is reported and clamped (no access leaves the cache)
      const int raw = d.page_table[(size_t)b * d.page_stride + i];
      const int blk = min(max(raw, 0), d.num_blocks - 1);
      if (raw != blk) st_co(ws.line(CTR_ERR), ERR_BAD_INPUT);
      pages[i] = blk;
    }
    const uint16_t* row = ws.qkv() + (size_t)b * QKV_N;
    if (wave < 4) {
    const uint16_t* src = wave < 2 ? row + (GROUP * h + wave) * HD : (wave == 2 ? row + QS + h * HD : row + QS + KVS + h * HD);
    const float x0 = bf2f(ld_co(src + lane)), x1 = bf2f(ld_co(src + lane + 64));
    uint16_t* dst = wave < 2 ? qb + wave * HD : (wave == 2 ? kb : vb);
    if (wave < 3) {
      const uint16_t* wn = wptr(d, layer, wave < 2 ? MKD_W_Q_NORM : MKD_W_K_NORM);
      const float ss = wave_sum(x0 * x0 + x1 * x1);
      const float r = 1.0f / sqrtf(ss * (1.0f / HD) + EPS);
      const float n0 = round_bf(round_bf(x0 * r) * bf2f(wn[lane]));
      const float n1 = round_bf(round_bf(x1 * r) * bf2f(wn[lane + 64]));
      const float c = d.rope_cos[pos * (HD / 2) + lane], s = d.rope_sin[pos * (HD / 2) + lane];
      dst[lane] = (uint16_t)f2bf(n0 * c - n1 * s);
      dst[lane + 64] = (uint16_t)f2bf(n1 * c + n0 * s);
    } else {
      dst[lane] = (uint16_t)f2bf(x0);
      dst[lane + 64] = (uint16_t)f2bf(x1);
    }
    }
  }
  sync();
  const int32_t* table = d.page_table + (size_t)b * d.page_stride;
  const size_t layer_off = (size_t)layer * (size_t)d.kv_layer_stride + (size_t)h * HD;
  if (split == 0 && active && t < 128) {
    const int blk = table[pos / bs];
    if (blk < 0 || blk >= nblk) {
      if (t == 0) st_co(ws.line(CTR_ERR), ERR_BAD_INPUT);
    } else {
    const size_t slot = (size_t)blk * bs + pos % bs;
    if (t < 64) reinterpret_cast<uint32_t*>(d.k_cache + layer_off + slot * KVS)[t] = reinterpret_cast<const uint32_t*>(kb)[t];
    else reinterpret_cast<uint32_t*>(d.v_cache + layer_off + slot * KVS)[t - 64] = reinterpret_cast<const uint32_t*>(vb)[t - 64];
    }
  }

  // -- this split's positions
  const int ctx = pos + 1;
  const int chunk = ((ctx + nsplit - 1) / nsplit + 63) & ~63;
  const int p_begin = split * chunk;
  const int p_end = min(ctx, p_begin + chunk);

  float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;
  float a0[8], a1[8];
#pragma unroll
  for (int j = 0; j < 8; j++) { a0[j] = 0.f; a1[j] = 0.f; }
  const uint4* q0 = reinterpret_cast<const uint4*>(qb);
  const uint4* q1 = reinterpret_cast<const uint4*>(qb + HD);

  // Cached positions [p_begin, c_end): everything before this token's own
  // position. The token itself (pos) is attended from LDS below, so the
  // loop never depends on this step's cache write. Per 64-position tile a
  // lane loads one K row (scores: one position per lane) and, for P*V, the
  // 16 V slices of positions t0 + 4*it + sub (dims dg..dg+8); all 32 loads
  // are issued before any math so the tile costs one memory round trip.
  const int c_end = min(p_end, pos);
  const int dg = (lane & 15) * 8, sub = lane >> 4;
  const uint16_t* kbase = d.k_cache + layer_off;
  const uint16_t* vbase = d.v_cache + layer_off;
  for (int t0 = p_begin + wave * 64; t0 < c_end; t0 += NW * 64) {
    asm volatile("" ::: "memory");  // keep the q reads (LDS) inside the tile: hoisting them costs 128 VGPRs
    const int p = t0 + lane;
    const bool valid = p < c_end;
    const int pc = valid ? p : t0;
    const uint4* krow = reinterpret_cast<const uint4*>(kbase + ((size_t)pages[pc / bs] * bs + pc % bs) * KVS);
    uint4 kreg[HD / 8], vreg[16];
#pragma unroll
    for (int i = 0; i < HD / 8; i++) kreg[i] = krow[i];
#pragma unroll
    for (int it = 0; it < 16; it++) {
      int pp = t0 + 4 * it + sub;
      pp = pp < c_end ? pp : t0;
      vreg[it] = *reinterpret_cast<const uint4*>(vbase + ((size_t)pages[pp / bs] * bs + pp % bs) * KVS + dg);
    }
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
    const float p0 = expf(s0 - n0), p1 = expf(s1 - n1);
    l0 = l0 * al0 + wave_sum(p0);
    l1 = l1 * al1 + wave_sum(p1);
    m0 = n0; m1 = n1;
#pragma unroll
    for (int j = 0; j < 8; j++) { a0[j] *= al0; a1[j] *= al1; }
#pragma unroll
    for (int it = 0; it < 16; it++) {
      const float w0 = __shfl(p0, 4 * it + sub, 64), w1 = __shfl(p1, 4 * it + sub, 64);  // 0 past c_end
      const uint4 v = vreg[it];
      const float vf[8] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w)};
#pragma unroll
      for (int j = 0; j < 8; j++) { a0[j] += w0 * vf[j]; a1[j] += w1 * vf[j]; }
    }
  }
  // The token's own K/V (position pos) belongs to the split whose range holds it.
  if (wave == 0 && p_begin <= pos && pos < p_end) {
    const uint32_t kw = reinterpret_cast<const uint32_t*>(kb)[lane];
    const float s0 = wave_sum(dot2(kw, reinterpret_cast<const uint32_t*>(qb)[lane], 0.f)) * ATTN_SCALE;
    const float s1 = wave_sum(dot2(kw, reinterpret_cast<const uint32_t*>(qb + HD)[lane], 0.f)) * ATTN_SCALE;
    const float n0 = fmaxf(m0, s0), n1 = fmaxf(m1, s1);
    const float al0 = expf(m0 - n0), al1 = expf(m1 - n1);
    const float p0 = expf(s0 - n0), p1 = expf(s1 - n1);
    l0 = l0 * al0 + p0;
    l1 = l1 * al1 + p1;
    m0 = n0; m1 = n1;
    const uint4 v = *reinterpret_cast<const uint4*>(vb + dg);
    const float vf[8] = {bf_lo(v.x), bf_hi(v.x), bf_lo(v.y), bf_hi(v.y), bf_lo(v.z), bf_hi(v.z), bf_lo(v.w), bf_hi(v.w)};
#pragma unroll
    for (int j = 0; j < 8; j++) {
      a0[j] = a0[j] * al0 + (sub == 0 ? p0 * vf[j] : 0.f);
      a1[j] = a1[j] * al1 + (sub == 0 ? p1 * vf[j] : 0.f);
    }
  }
  // reduce the 4 position sub-groups of the wave, then merge waves through LDS
#pragma unroll
  for (int j = 0; j < 8; j++) {
    a0[j] += __shfl_xor(a0[j], 16, 64); a0[j] += __shfl_xor(a0[j], 32, 64);
    a1[j] += __shfl_xor(a1[j], 16, 64); a1[j] += __shfl_xor(a1[j], 32, 64);
  }
  if (lane < 16) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      mrg[(wave * GROUP + 0) * HD + lane * 8 + j] = a0[j];
      mrg[(wave * GROUP + 1) * HD + lane * 8 + j] = a1[j];
    }
  }
  if (lane == 0) {
    mrg_ml[wave * GROUP + 0] = m0; mrg_ml[wave * GROUP + 1] = m1;
    mrg_ml[NW * GROUP + wave * GROUP + 0] = l0; mrg_ml[NW * GROUP + wave * GROUP + 1] = l1;
  }
  sync();
  // threads 0..255 = 2 heads x 128 dims finish the merge; with NW > 4 the
  // other threads only take part in the barriers
  const int g = (t >> 7) & 1, dd = t & 127;
  const bool merger = t < GROUP * HD;
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; w++) M = fmaxf(M, mrg_ml[w * GROUP + g]);
  float num = 0.f, den = 0.f;
  if (M != -INFINITY) {
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float sc = expf(mrg_ml[w * GROUP + g] - M);
      num += mrg[(w * GROUP + g) * HD + dd] * sc;
      den += mrg_ml[NW * GROUP + w * GROUP + g] * sc;
    }
  }
  uint16_t* out = ws.attn() + (size_t)b * QS + (GROUP * h + g) * HD + dd;
  if (nsplit == 1) {
    if (merger) st_co(out, (uint16_t)f2bf(num / den));
    return true;
  }
  float* part = ws.apart(b, h, split);
  if (merger) {
    st_co(part + g * HD + dd, num);
    if (dd == 0) { st_co(part + GROUP * HD + g, M); st_co(part + GROUP * HD + GROUP + g, den); }
  }
  drain();
  sync();
  if (t == 0) {
    uint32_t* ticket = ws.line(CTR_COMB_BASE + (layer * MAXB + b) * NKV + h);
    const uint32_t old = add_co(ticket, 1u);
    const bool last = old == (uint32_t)(nsplit - 1);
    if (last) st_co(ticket, 0u);
    sh[0] = last;
  }
  sync();
  if (!sh[0]) return false;
  if (!merger) return true;
  float Ms = -INFINITY;
  for (int s = 0; s < nsplit; s++) Ms = fmaxf(Ms, ld_co(ws.apart(b, h, s) + GROUP * HD + g));
  num = 0.f; den = 0.f;
  for (int s = 0; s < nsplit; s++) {
    const float* ps = ws.apart(b, h, s);
    const float ms = ld_co(ps + GROUP * HD + g);
    if (ms == -INFINITY) continue;
    const float sc = expf(ms - Ms);
    num += ld_co(ps + g * HD + dd) * sc;
    den += ld_co(ps + GROUP * HD + GROUP + g) * sc;
  }
  st_co(out, (uint16_t)f2bf(num / den));
  return true;
}

// ---------------------------------------------------------------------------
// LMHEAD: final norm + rows [r0, r0+nr) of the tied embedding, bf16 logits,
// per-row (max, first index) partial in `slot`; the last slot to arrive
// reduces all partials to the greedy tokens and finishes the step.
// ---------------------------------------------------------------------------
template <int B>
__device__ void task_lmhead(const MkdStepDesc& d, const Ws& ws, int r0, int nr, int slot, uint8_t* smem) {
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* red = reinterpret_cast<float*>(smem + MAXB * I * 2);
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  stage_norm<B>(d, ws, 2 * d.num_layers, ws.hid_f(), d.final_norm, xs, red, false);
  float best = -INFINITY;
  int best_i = 0x7fffffff;
  uint16_t* logits = d.out_logits;
  auto rowptr = [&](int r) -> const uint16_t* { return d.embed + (size_t)r * H; };
  gemv<B, H, 4>(rowptr, r0, nr, xs, [&](int r, const float* acc) {
    const float v = round_bf(pick_lane<B>(acc, lane));
    if (lane < B) {
      if (lm_better(v, r, best, best_i)) { best = v; best_i = r; }
      if (logits != nullptr && lane < d.rows) logits[(size_t)lane * V + r] = (uint16_t)f2bf(v);
    }
  });
  float* bv = red;                                    // [4][MAXB]
  int* bi = reinterpret_cast<int*>(red + NWAVE * MAXB);  // [4][MAXB]
  int* sh = bi + NWAVE * MAXB;
  __syncthreads();
  if (lane < B) { bv[wave * MAXB + lane] = best; bi[wave * MAXB + lane] = best_i; }
  __syncthreads();
  if (t < B) {
    float v = bv[t]; int i = bi[t];
    for (int w = 1; w < NWAVE; w++) {
      const float v2 = bv[w * MAXB + t]; const int i2 = bi[w * MAXB + t];
      if (lm_better(v2, i2, v, i)) { v = v2; i = i2; }
    }
    st_co(reinterpret_cast<uint64_t*>(ws.lmpart(slot) + t), (uint64_t)__float_as_uint(v) | ((uint64_t)(uint32_t)i << 32));
  }
  drain();
  __syncthreads();
  if (t == 0) {
    const uint32_t old = add_co(ws.line(CTR_LM_TICKET), 1u);
    const bool last = old == (uint32_t)(d.lm_slots - 1);
    if (last) st_co(ws.line(CTR_LM_TICKET), 0u);
    sh[0] = last;
  }
  __syncthreads();
  if (!sh[0]) return;
  // Final reduction: wave b reduces row b over all slots (rows > 4 loop).
  for (int b = wave; b < d.rows; b += NWAVE) {
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
      const int tok = i == 0x7fffffff ? 0 : i;  // (no candidate at all: token 0)
      d.out_tokens[b] = tok;
      if (d.flags & MKD_FLAG_ADVANCE) {
        d.input_ids[b] = tok;
        d.cache_seqlens[b] += 1;
      }
    }
  }
  if (d.flags & MKD_FLAG_ZERO_FANIN) {
    for (int f = t; f < d.num_layers * FANIN_PER_LAYER * FANIN_SUBSLOTS; f += NT)
      st_co(ws.line(CTR_FANIN_BASE + f), 0u);
  }
}

}  // namespace mkd
