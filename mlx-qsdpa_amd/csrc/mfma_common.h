// Device helpers, launch parameters and host-side set-up of the MFMA decode
// kernel (decode_mfma.hip).
#pragma once

#include <algorithm>

#include "abi_internal.h"
#include "common.h"

namespace qsdpa {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kTile = 32;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;
constexpr float kRescale = 8.0f;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

struct MfmaParams {
  int B, Hq, Hkv, N, G, hb_count, num_splits;
  float qscale;  // softmax scale * log2(e)
  int has_bias;
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint32_t* kp;
  int64_t kp_sb, kp_sh, kp_sn;
  const uint32_t* vp;
  int64_t vp_sb, vp_sh, vp_sn;
  const uint16_t* ks;
  int64_t ks_sb, ks_sh, ks_sn;
  const uint16_t* vs;
  int64_t vs_sb, vs_sh, vs_sn;
  const uint16_t* kb;
  int64_t kb_sb, kb_sh, kb_sn;
  const uint16_t* vb;
  int64_t vb_sb, vb_sh, vb_sn;
  uint16_t* out;
  int64_t o_sb, o_sh;
  const void* mask;
  int mask_kind;
  int64_t m_sb, m_sh, m_sn;
  const int32_t* kv_start;
  float* part_acc;
  float* part_ml;
  int units;   // > 0: stream-K schedule of a left-padded batch over this many units per kv head
  int* sched;  // (first partial column, count) per sequence, for the merge when units > 0
  // Split merge inside the launch (uniform splits, at most kFusedSplits):
  // null = the merge kernel combines the partials; otherwise kTicketWords
  // counters per block (batch, kv head, row block), zero between calls, and
  // the last workgroup of a block merges its partials.
  unsigned* tickets;
  // Query positions: the G * qL rows of a kv head are (position v / G, head
  // v % G); a block takes 16 consecutive rows.
  int qL, causal;
  int64_t q_sq, o_sq, m_sq;  // position strides of q, out and the mask
  // Folded append (null = none): the new K / V rows [B, H_kv, 1, D], which
  // the workgroup that reads key N - 1 quantizes into that key first.
  const uint16_t* knew;
  int64_t knew_sb, knew_sh;
  const uint16_t* vnew;
  int64_t vnew_sb, vnew_sh;
};

static_assert(kTile == kSchedTile, "the stream-K schedule counts the decode's key tiles");

__device__ __forceinline__ uint32_t bitop_and_or(uint32_t a, uint32_t mask, uint32_t c) {
  return __builtin_amdgcn_bitop3_b32(a, mask, c, 0xEA);  // (a & mask) | c
}
__device__ __forceinline__ uint32_t perm(uint32_t hi_src, uint32_t lo_src, uint32_t sel) {
  return __builtin_amdgcn_perm(hi_src, lo_src, sel);
}

constexpr uint32_t kNib = 0x000F000Fu;     // nibble of each 16-bit half
constexpr uint32_t kMagic = 0x64006400u;   // fp16 1024.0 in both halves
// A nibble at bits 4-7 of a half, or-ed into fp16 64.0 (ulp 1/16), reads as
// 64 + code: the second nibble of a half needs no shift.
constexpr uint32_t kNib1 = 0x00F000F0u;
constexpr uint32_t kMagic64 = 0x54005400u;
constexpr uint32_t kMagic8 = 0x64646464u;  // byte source for v_perm_b32
constexpr uint32_t kSelB01 = 0x04010400u;  // [src.b0, 0x64, src.b1, 0x64]
constexpr uint32_t kSelB23 = 0x04030402u;  // [src.b2, 0x64, src.b3, 0x64]

__device__ __forceinline__ uint32_t f16x2_sub1024(uint32_t t) {
  const f16x2 k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, t) - k1024);
}
__device__ __forceinline__ uint32_t f16x2_sub64(uint32_t t) {
  const f16x2 k64 = {static_cast<_Float16>(64.0f), static_cast<_Float16>(64.0f)};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, t) - k64);
}
// Codes (as exact fp16 pairs) of nibble k (0-3) of both halves of x, given
// x8 = x >> 8.  Nibbles 0 and 1 of a half come from x, 2 and 3 from x8.
__device__ __forceinline__ uint32_t nib_codes(uint32_t x, uint32_t x8, int k) {
  const uint32_t src = k < 2 ? x : x8;
  return (k & 1) ? f16x2_sub64(bitop_and_or(src, kNib1, kMagic64))
                 : f16x2_sub1024(bitop_and_or(src, kNib, kMagic));
}
__device__ __forceinline__ uint32_t f16x2_fma(uint32_t c, uint32_t s, uint32_t b) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, c),
                                                                __builtin_bit_cast(f16x2, s),
                                                                __builtin_bit_cast(f16x2, b)));
}
// Both halves = the low half of x (v_perm_b32 selector 0x01000100).
__device__ __forceinline__ uint32_t splat_lo(uint32_t x) { return perm(x, x, 0x01000100u); }

// K slice (8 dims of one token, BITS/4 packed words) -> A operand (4 pairs).
// f16: s2 / b2 hold the group's scale / bias in both halves.  bf16: sf / bf
// are the float scale / bias.
template <typename Tag, int BITS>
__device__ __forceinline__ void dequant_k(const uint32_t* w, uint32_t s2, uint32_t b2, float sf,
                                          float bf, uint32_t out[4]) {
  if constexpr (Tag::kId == QSDPA_F16) {
    uint32_t t[4];
    if constexpr (BITS == 4) {
      const uint32_t x = w[0], x8 = w[0] >> 8;
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = nib_codes(x, x8, i);  // codes (i, i + 4)
    } else {
      t[0] = f16x2_sub1024(perm(kMagic8, w[0], kSelB01));
      t[1] = f16x2_sub1024(perm(kMagic8, w[0], kSelB23));
      t[2] = f16x2_sub1024(perm(kMagic8, w[1], kSelB01));
      t[3] = f16x2_sub1024(perm(kMagic8, w[1], kSelB23));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = f16x2_fma(t[i], s2, b2);
  } else {
    float c[8];
    if constexpr (BITS == 4) {
      const uint32_t lo = w[0] & 0x0F0F0F0Fu;
      const uint32_t hi = (w[0] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        c[2 * i] = static_cast<float>((lo >> (8 * i)) & 0xFFu);
        c[2 * i + 1] = static_cast<float>((hi >> (8 * i)) & 0xFFu);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = static_cast<float>((w[i >> 2] >> (8 * (i & 3))) & 0xFFu);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = pack_T2<Tag>(fmaf(sf, c[2 * i], bf), fmaf(sf, c[2 * i + 1], bf));
  }
}

// bfloat16 inputs: the 8 values (dims in order, float32, not yet rounded to
// T) of an 8-dim slice.  A 16-bit half whose bits are a code c < 1024 is the
// float16 value c 2^-24 (a subnormal), so one mask or v_perm_b32 places two
// codes, and v_fma_mix_f32 (float32 fma of a float16 half, widened exactly)
// gives (c 2^-24)(s 2^24) + b, the value and the one rounding of fmaf(c, s,
// b), without a v_cvt_f32_ubyte per code.  S = s 2^24, and for 4-bit codes
// S16 = s 2^20 (the odd nibbles of a byte are read as 16 c).  Exact while S
// is finite: callers keep |s| below kMixScaleMax.
constexpr float kMixScaleMax = 0x1p100f;

template <int H>
__device__ __forceinline__ float fma_half(uint32_t t, float S, float B) {
  return fmaf(static_cast<float>(__builtin_bit_cast(f16x2, t)[H]), S, B);
}
template <int BITS>
__device__ __forceinline__ void mix_dequant8(const uint32_t* w, float S, float S16, float B, float (&y)[8]) {
  if constexpr (BITS == 8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t x = w[h];
      const uint32_t e = x & 0x00FF00FFu;          // codes of dims 0 and 2
      const uint32_t o = perm(x, x, 0x0C030C01u);  // dims 1 and 3
      y[4 * h + 0] = fma_half<0>(e, S, B);
      y[4 * h + 1] = fma_half<0>(o, S, B);
      y[4 * h + 2] = fma_half<1>(e, S, B);
      y[4 * h + 3] = fma_half<1>(o, S, B);
    }
  } else {
    static_assert(BITS == 4, "code width");
    const uint32_t x = w[0], x8 = x >> 8;
    const uint32_t a = x & kNib, c = x & kNib1, e = x8 & kNib, g = x8 & kNib1;  // dims (0,4) (1,5) (2,6) (3,7)
    y[0] = fma_half<0>(a, S, B);
    y[1] = fma_half<0>(c, S16, B);
    y[2] = fma_half<0>(e, S, B);
    y[3] = fma_half<0>(g, S16, B);
    y[4] = fma_half<1>(a, S, B);
    y[5] = fma_half<1>(c, S16, B);
    y[6] = fma_half<1>(e, S, B);
    y[7] = fma_half<1>(g, S16, B);
  }
}

template <typename Tag>
__device__ __forceinline__ f4 mfma(const uint32_t a[4], const uint32_t b[4], f4 c) {
  const uint4 av = {a[0], a[1], a[2], a[3]};
  const uint4 bv = {b[0], b[1], b[2], b[3]};
  if constexpr (Tag::kId == QSDPA_F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, av), __builtin_bit_cast(h8, bv), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, av), __builtin_bit_cast(b8, bv), c,
                                                   0, 0, 0);
}

// Mask values (log2 domain) at element offsets o[0..N) of the mask tensor:
// every load is issued before any is used, so a caller that issues them
// ahead of its next tile's loads waits for them alone.
template <int N>
__device__ __forceinline__ void mask_values(const MfmaParams& p, const int64_t (&o)[N], float (&mv)[N]) {
  switch (p.mask_kind) {
    case QSDPA_BOOL: {
      const uint8_t* m = static_cast<const uint8_t*>(p.mask);
      uint8_t x[N];
#pragma unroll
      for (int e = 0; e < N; ++e) x[e] = m[o[e]];
#pragma unroll
      for (int e = 0; e < N; ++e) mv[e] = x[e] ? 0.0f : -__builtin_huge_valf();
      break;
    }
    case QSDPA_F16:
    case QSDPA_BF16: {
      const uint16_t* m = static_cast<const uint16_t*>(p.mask);
      uint16_t x[N];
#pragma unroll
      for (int e = 0; e < N; ++e) x[e] = m[o[e]];
      const bool h = p.mask_kind == QSDPA_F16;
#pragma unroll
      for (int e = 0; e < N; ++e) mv[e] = (h ? f16_bits_to_f32(x[e]) : bf16_bits_to_f32(x[e])) * kLog2e;
      break;
    }
    default: {
      const float* m = static_cast<const float*>(p.mask);
#pragma unroll
      for (int e = 0; e < N; ++e) mv[e] = m[o[e]];
#pragma unroll
      for (int e = 0; e < N; ++e) mv[e] *= kLog2e;
      break;
    }
  }
}

// Mask values of a lane's keys key0 + off(e), e < N (off: a pattern of
// constants), clamped to the last key.  `whole`: every key of the tile is
// below N.  Then, with adjacent keys in the mask (key stride 1), the offsets
// are one base plus constants, which the loads carry as immediate offsets;
// otherwise every key's offset is computed and clamped (64-bit products).
template <int N, typename Off>
__device__ __forceinline__ void mask_tile(const MfmaParams& p, int64_t mrow, int key0, bool whole, Off&& off,
                                          float (&mv)[N]) {
  int64_t o[N];
  if (whole && p.m_sn == 1) {
    const int64_t o0 = mrow + key0;
#pragma unroll
    for (int e = 0; e < N; ++e) o[e] = o0 + off(e);
    mask_values<N>(p, o, mv);
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) o[e] = mrow + static_cast<int64_t>(min(key0 + off(e), p.N - 1)) * p.m_sn;
    mask_values<N>(p, o, mv);
  }
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw buffer descriptor (gfx9 dword3: 32-bit data format, no swizzle).
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}

// Host side ---------------------------------------------------------------

inline bool aligned_view(const qsdpa_view& v, int bytes, int64_t elem_bytes) {
  if (v.ptr == nullptr) return true;
  if (reinterpret_cast<uintptr_t>(v.ptr) % bytes) return false;
  const int64_t m = bytes / elem_bytes;
  return m <= 1 || (v.stride_b % m == 0 && v.stride_h % m == 0 && v.stride_n % m == 0);
}

// Launch parameters of the decode arguments (pointers, strides, shapes).
inline MfmaParams mfma_params(const qsdpa_decode_args* a, int num_splits, float* part_acc, float* part_ml) {
  MfmaParams p;
  p.B = a->B; p.Hq = a->H_q; p.Hkv = a->H_kv; p.N = a->N;
  p.G = a->H_q / a->H_kv;
  p.qL = a->q_len > 1 ? a->q_len : 1;
  p.causal = a->causal != 0;
  p.hb_count = (p.G * p.qL + 15) / 16;
  p.num_splits = num_splits;
  p.qscale = a->scale * kLog2e;
  p.has_bias = a->k_biases.ptr != nullptr;
  p.q = static_cast<const uint16_t*>(a->q.ptr); p.q_sb = a->q.stride_b; p.q_sh = a->q.stride_h;
  p.q_sq = p.qL > 1 ? a->q.stride_n : 0;
  p.o_sq = p.qL > 1 ? a->out.stride_n : 0;
  p.m_sq = p.qL > 1 ? a->mask_stride_q : 0;
  p.kp = static_cast<const uint32_t*>(a->k_packed.ptr);
  p.kp_sb = a->k_packed.stride_b; p.kp_sh = a->k_packed.stride_h; p.kp_sn = a->k_packed.stride_n;
  p.vp = static_cast<const uint32_t*>(a->v_packed.ptr);
  p.vp_sb = a->v_packed.stride_b; p.vp_sh = a->v_packed.stride_h; p.vp_sn = a->v_packed.stride_n;
  p.ks = static_cast<const uint16_t*>(a->k_scales.ptr);
  p.ks_sb = a->k_scales.stride_b; p.ks_sh = a->k_scales.stride_h; p.ks_sn = a->k_scales.stride_n;
  p.vs = static_cast<const uint16_t*>(a->v_scales.ptr);
  p.vs_sb = a->v_scales.stride_b; p.vs_sh = a->v_scales.stride_h; p.vs_sn = a->v_scales.stride_n;
  p.kb = static_cast<const uint16_t*>(a->k_biases.ptr);
  p.kb_sb = a->k_biases.stride_b; p.kb_sh = a->k_biases.stride_h; p.kb_sn = a->k_biases.stride_n;
  p.vb = static_cast<const uint16_t*>(a->v_biases.ptr);
  p.vb_sb = a->v_biases.stride_b; p.vb_sh = a->v_biases.stride_h; p.vb_sn = a->v_biases.stride_n;
  if (!p.has_bias) {
    p.kb_sb = p.ks_sb; p.kb_sh = p.ks_sh; p.kb_sn = p.ks_sn;
    p.vb_sb = p.vs_sb; p.vb_sh = p.vs_sh; p.vb_sn = p.vs_sn;
  }
  p.out = static_cast<uint16_t*>(const_cast<void*>(a->out.ptr));
  p.o_sb = a->out.stride_b; p.o_sh = a->out.stride_h;
  p.mask = a->mask.ptr; p.mask_kind = a->mask_dtype;
  p.m_sb = a->mask.stride_b; p.m_sh = a->mask.stride_h; p.m_sn = a->mask.stride_n;
  p.kv_start = a->kv_start;
  p.part_acc = part_acc;
  p.part_ml = part_ml;
  p.units = 0;
  p.sched = nullptr;
  p.tickets = nullptr;
  p.knew = p.vnew = nullptr;
  p.knew_sb = p.knew_sh = p.vnew_sb = p.vnew_sh = 0;
  return p;
}

}  // namespace
}  // namespace qsdpa
