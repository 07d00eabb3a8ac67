// mkd_common.h -- constants and device helpers of the MI355X decode-step kernels.
//
// Coherence protocol used by every task (measured on MI355X, 8 XCDs with
// private L2s): activations exchanged between workgroups inside one launch are
// written and read with relaxed agent-scope atomic accesses, which the
// compiler emits as sc1 global loads/stores (coherent across XCDs without any
// L2 writeback/invalidate). A producer drains its stores with s_waitcnt before
// it arrives on a counter; a consumer issues its loads only after it has seen
// the counter. Agent-scope fences are avoided on purpose: each one costs an L2
// writeback or invalidate (~1.7 us measured).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mkd_abi.h"

namespace mkd {

constexpr int H = MKD_HIDDEN;
constexpr int I = MKD_INTERMEDIATE;
constexpr int NQ = MKD_NUM_Q_HEADS;
constexpr int NKV = MKD_NUM_KV_HEADS;
constexpr int HD = MKD_HEAD_DIM;
constexpr int QS = NQ * HD;            // 2048
constexpr int KVS = NKV * HD;          // 1024
constexpr int QKV_N = QS + 2 * KVS;    // 4096
constexpr int V = MKD_VOCAB;
constexpr int MAXB = MKD_MAX_BATCH;
constexpr int MAXS = MKD_MAX_SPLITS;
constexpr int GROUP = NQ / NKV;        // 2 query heads per KV head
constexpr int NT = 256;                // threads per workgroup (4 waves)
constexpr int NWAVE = NT / 64;
constexpr float EPS = 1e-6f;
constexpr int PART_STRIDE = GROUP * HD + 2 * GROUP;  // floats per attention partial

// ---- workspace layout (byte offsets) -------------------------------------
constexpr size_t OFF_RESID = 0;                                   // bf16 [2][MAXB][H]
constexpr size_t OFF_HID_A = OFF_RESID + 2ull * MAXB * H * 2;     // bf16 [MAXB][H]  o_proj out
constexpr size_t OFF_HID_F = OFF_HID_A + 1ull * MAXB * H * 2;     // bf16 [MAXB][H]  down out
constexpr size_t OFF_QKV = OFF_HID_F + 1ull * MAXB * H * 2;       // bf16 [MAXB][QKV_N]
constexpr size_t OFF_ATTN = OFF_QKV + 1ull * MAXB * QKV_N * 2;    // bf16 [MAXB][QS]
constexpr size_t OFF_ACT = OFF_ATTN + 1ull * MAXB * QS * 2;       // bf16 [MAXB][I]
constexpr size_t OFF_APART = OFF_ACT + 1ull * MAXB * I * 2;       // f32 [MAXB][NKV][MAXS][PART_STRIDE]
constexpr size_t OFF_LMPART = OFF_APART + 4ull * MAXB * NKV * MAXS * PART_STRIDE;  // {f32,i32} [slots][MAXB]
constexpr size_t OFF_CTR = OFF_LMPART + 8ull * MKD_MAX_LM_SLOTS * MAXB;
// Counters: one 128-byte line each. Line 0 = error word. Fan-in counters own 8
// consecutive lines (one per XCD-spread sub-slot); ticket counters own one.
constexpr int CTR_LINE_U32 = 32;
constexpr int CTR_ERR = 0;
constexpr int CTR_LM_TICKET = 1;
constexpr int CTR_EPOCH = 2;                                       // step counter of the tagged exchange
constexpr int CTR_COMB_BASE = 3;                                   // [layers][MAXB][NKV] tickets
constexpr int CTR_FANIN_BASE = CTR_COMB_BASE + MKD_NUM_LAYERS * MAXB * NKV;
constexpr int FANIN_PER_LAYER = NKV + 4;                           // qkv[h], attn, oproj, gateup, down
constexpr int FANIN_SUBSLOTS = 8;
constexpr int NUM_FANIN = MKD_NUM_LAYERS * FANIN_PER_LAYER;
constexpr int NUM_CTR_LINES = CTR_FANIN_BASE + NUM_FANIN * FANIN_SUBSLOTS;
// Tagged exchange region (persistent kernel): 64-bit words, low half = two bf16
// values (or one fp32), high half = tag (epoch + 1) * 32 + layer. Offsets in words.
// The buffers every workgroup reads come in TW_NREP replicas (one per XCD, so
// each is polled by one XCD's workgroups); the QKV words, split partials and LM
// partials have a single copy.
constexpr size_t OFF_TAGGED = (OFF_CTR + 128ull * NUM_CTR_LINES + 255) & ~255ull;
constexpr size_t TW_RES1 = 0;                                        // [MAXB][H/2]   residual after QKV-stage add
constexpr size_t TW_RES2 = TW_RES1 + (size_t)MAXB * H / 2;           // [MAXB][H/2]   residual after GATEUP-stage add
constexpr size_t TW_ATTN = TW_RES2 + (size_t)MAXB * H / 2;           // [MAXB][QS/2]
constexpr size_t TW_O = TW_ATTN + (size_t)MAXB * QS / 2;             // [MAXB][H/2]
constexpr size_t TW_ACT = TW_O + (size_t)MAXB * H / 2;               // [MAXB][I/2]
constexpr size_t TW_DOWN = TW_ACT + (size_t)MAXB * I / 2;            // [MAXB][H/2]
constexpr size_t TW_GROUP = TW_DOWN + (size_t)MAXB * H / 2;          // words of one replica
constexpr int TW_NREP = 8;
constexpr size_t TW_QKV = TW_GROUP * TW_NREP;                        // [MAXB][QKV_N/2]
constexpr size_t TW_APART = TW_QKV + (size_t)MAXB * QKV_N / 2;       // [MAXB][NKV][MAXS][PART_STRIDE] fp32
constexpr size_t TW_LM = TW_APART + (size_t)MAXB * NKV * MAXS * PART_STRIDE;  // [MAX_LM_SLOTS][MAXB][2]
constexpr size_t TW_WORDS = TW_LM + (size_t)MKD_MAX_LM_SLOTS * MAXB * 2;
constexpr size_t WORKSPACE_BYTES = OFF_TAGGED + 8 * TW_WORDS;

// Error codes written to the error word.
constexpr uint32_t ERR_TIMEOUT = 1;
constexpr uint32_t ERR_BAD_INST = 2;
constexpr uint32_t ERR_BAD_INPUT = 3;  // position / block id / token id out of range

// ---- bf16 --------------------------------------------------------------------
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

__device__ __forceinline__ float bf2f(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even fp32 -> bf16 (torch's rounding), NaN kept quiet.
// Written as a select (no branch): a wave-uniform value would otherwise turn
// the NaN test into scalar branches inside hot loops.
// fp32 -> bf16, round to nearest even (NaN stays NaN): gfx950's v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef float f32x2v_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v_t){lo, hi}, bf16x2v_t));
}
__device__ __forceinline__ uint32_t f2bf(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ float round_bf(float f) { return bf2f(f2bf(f)); }

// Greedy-argmax order of torch.argmax: a NaN ranks above every number (the
// first NaN wins), otherwise the larger value, and on equal values the lower
// index. True when candidate (v, i) ranks above the current best (bv, bi).
__device__ __forceinline__ bool lm_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  return vn ? (!bn || i < bi) : (!bn && (v > bv || (v == bv && i < bi)));
}
// The same rule for a running argmax that visits rows in increasing order: a
// later row never wins a tie, so only a larger value or a first NaN replaces
// the best (an all -inf run keeps the "no candidate" index, which the final
// merge turns into token 0, as torch.argmax of all -inf gives).
__device__ __forceinline__ bool lm_later_better(float v, float bv) {
  return v != v ? bv == bv : v > bv;
}

// a.lo*b.lo + a.hi*b.hi + c in fp32 (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}
__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float c) {
  c = dot2(a.x, b.x, c);
  c = dot2(a.y, b.y, c);
  c = dot2(a.z, b.z, c);
  return dot2(a.w, b.w, c);
}

// ---- coherent (cross-XCD) accesses ------------------------------------------
template <typename T>
__device__ __forceinline__ T ld_co(const T* p) {
  return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void st_co(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t add_co(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this wave's outstanding memory operations have completed.
__device__ __forceinline__ void drain() { __builtin_amdgcn_s_waitcnt(0); }

// ---- wave reductions (wave64) --------------------------------------------------
// DPP butterfly: quad swaps, row half-mirror and mirror give every lane its
// 16-lane row total; row_bcast15 / row_bcast31 fold the four rows into lane
// 63, which is read back as a uniform value. Six VALU DPP ops instead of six
// LDS-crossbar (ds_bpermute) round trips.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_mov(float v, float old) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_mov<0xB1>(v, 0.f);         // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v, 0.f);         // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v, 0.f);        // row_half_mirror
  v += dpp_mov<0x140>(v, 0.f);        // row_mirror
  v += dpp_mov<0x142, 0xA>(v, 0.f);   // row_bcast15 -> rows 1, 3
  v += dpp_mov<0x143, 0xC>(v, 0.f);   // row_bcast31 -> rows 2, 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// Wave totals of B (2, 4 or 8) per-lane values at once: lane l returns the
// total of value l % B. A reduce-scatter over lane bits 0 .. log2 B - 1 (each
// step keeps half of the values and adds the partner's other half: quad swaps,
// then row_shl / row_shr by 4), then an all-reduce over the remaining bits
// (row_ror 8, the gfx950 permlane16 / permlane32 swaps): 11 cross-lane moves
// at B = 8 where B separate wave_sum chains take 6 B and B lane reads.
template <int B>
__device__ __forceinline__ float rows_wave_sum(const float (&x)[B]) {
  static_assert(B == 2 || B == 4 || B == 8, "2, 4 or 8 values");
  const int l = threadIdx.x & 63;
  float v[B];
#pragma unroll
  for (int j = 0; j < B; j++) v[j] = x[j];
  {  // lane bit 0: keep values of index bit 0 = the lane's bit 0
    const bool p = l & 1;
#pragma unroll
    for (int j = 0; j < B / 2; j++) {
      const float keep = p ? v[2 * j + 1] : v[2 * j], send = p ? v[2 * j] : v[2 * j + 1];
      v[j] = keep + dpp_mov<0xB1>(send, 0.f);  // quad_perm [1,0,3,2]
    }
  }
  if constexpr (B >= 4) {  // lane bit 1
    const bool p = l & 2;
#pragma unroll
    for (int j = 0; j < B / 4; j++) {
      const float keep = p ? v[2 * j + 1] : v[2 * j], send = p ? v[2 * j] : v[2 * j + 1];
      v[j] = keep + dpp_mov<0x4E>(send, 0.f);  // quad_perm [2,3,0,1]
    }
  }
  // lane bit 2: the partner l ^ 4 is l + 4 (row_shl 4) or l - 4 (row_shr 4).
  // Both moves run with every lane active (a DPP move reads 0 from a lane
  // that is off): the empty asm keeps the compiler from moving each into its
  // side of a branch on the lane's bit.
  const bool p2 = l & 4;
  auto xor4 = [&](float send) {
    float up = dpp_mov<0x104>(send, 0.f), down = dpp_mov<0x114>(send, 0.f);
    asm volatile("" : "+v"(up), "+v"(down));
    return p2 ? down : up;
  };
  float w;
  if constexpr (B >= 8) {
    const float keep = p2 ? v[1] : v[0], send = p2 ? v[0] : v[1];
    w = keep + xor4(send);
  } else {
    w = v[0];
    if constexpr (B == 2) w += dpp_mov<0x4E>(w, 0.f);  // lane bit 1
    w += xor4(w);
  }
  w += dpp_mov<0x128>(w, 0.f);  // lane bit 3: row_ror 8
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(w), __float_as_uint(w), false, false);
    w = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // lane bit 4
  }
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(w), __float_as_uint(w), false, false);
    w = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // lane bit 5
  }
  return w;
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v, -INFINITY));
  v = fmaxf(v, dpp_mov<0x4E>(v, -INFINITY));
  v = fmaxf(v, dpp_mov<0x141>(v, -INFINITY));
  v = fmaxf(v, dpp_mov<0x140>(v, -INFINITY));
  v = fmaxf(v, dpp_mov<0x142, 0xA>(v, -INFINITY));
  v = fmaxf(v, dpp_mov<0x143, 0xC>(v, -INFINITY));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// ---- workspace views -----------------------------------------------------------
struct Ws {
  uint8_t* base;
  __device__ __forceinline__ uint16_t* resid(int i) const {
    return reinterpret_cast<uint16_t*>(base + OFF_RESID) + (size_t)(i & 1) * MAXB * H;
  }
  __device__ __forceinline__ uint16_t* hid_a() const { return reinterpret_cast<uint16_t*>(base + OFF_HID_A); }
  __device__ __forceinline__ uint16_t* hid_f() const { return reinterpret_cast<uint16_t*>(base + OFF_HID_F); }
  __device__ __forceinline__ uint16_t* qkv() const { return reinterpret_cast<uint16_t*>(base + OFF_QKV); }
  __device__ __forceinline__ uint16_t* attn() const { return reinterpret_cast<uint16_t*>(base + OFF_ATTN); }
  __device__ __forceinline__ uint16_t* act() const { return reinterpret_cast<uint16_t*>(base + OFF_ACT); }
  __device__ __forceinline__ float* apart(int b, int h, int s) const {
    return reinterpret_cast<float*>(base + OFF_APART) + (((size_t)b * NKV + h) * MAXS + s) * PART_STRIDE;
  }
  __device__ __forceinline__ uint2* lmpart(int slot) const {
    return reinterpret_cast<uint2*>(base + OFF_LMPART) + (size_t)slot * MAXB;
  }
  __device__ __forceinline__ uint64_t* tw(size_t word) const {
    return reinterpret_cast<uint64_t*>(base + OFF_TAGGED) + word;
  }
  __device__ __forceinline__ uint32_t* line(int i) const {
    return reinterpret_cast<uint32_t*>(base + OFF_CTR) + (size_t)i * CTR_LINE_U32;
  }
};

}  // namespace mkd
