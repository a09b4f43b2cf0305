// The per-group quantizer of the MLX affine format, shared by the quantize
// and requant kernels (quant.hip) and the decode's folded append
// (decode_mfma.hip), so that every writer of a cache row produces the same
// bits.  The rule is the float32 edge-snapped affine quantizer restated in
// oracle/affine.py; every operation is an explicitly rounded intrinsic.
#ifndef QSDPA_QUANT_GROUP_H_
#define QSDPA_QUANT_GROUP_H_

#include "common.h"

namespace qsdpa {
namespace {

// Min / max over aligned groups of L consecutive lanes (L in {1, 2, 4, 8,
// 16}); every lane of a group gets the result.  Exact in any order.
template <int L>
__device__ __forceinline__ void group_minmax(float& lo, float& hi) {
  if constexpr (L == 1) return;
  lo = fminf(lo, dpp_f32<0xB1>(lo));
  hi = fmaxf(hi, dpp_f32<0xB1>(hi));
  if constexpr (L >= 4) {
    lo = fminf(lo, dpp_f32<0x4E>(lo));
    hi = fmaxf(hi, dpp_f32<0x4E>(hi));
  }
  if constexpr (L >= 8) {
    lo = fminf(lo, dpp_f32<0x141>(lo));
    hi = fmaxf(hi, dpp_f32<0x141>(hi));
  }
  if constexpr (L >= 16) {
    lo = fminf(lo, dpp_f32<0x140>(lo));
    hi = fmaxf(hi, dpp_f32<0x140>(hi));
  }
}

// Codes through the group's reciprocal.  A value's code is q = rint(fl(x /
// scale)), x = fl(v - bias).  inv = v_rcp_f32(scale) is within one ulp
// (relative error below 2^-23; scale is a normal number, at least about
// 5e-8 in magnitude).  With p = x inv (exact product) and z = x / scale,
// |p - z| <= |z| 2^-23 and |fl(z) - z| <= |z| 2^-24, so |p - fl(z)| <= 1.5
// |z| 2^-23.  q = rint(fl(p)) and e = fl(p - q) (one fma, within 2^-25 of p
// - q): when |e| < 1/2 - (|fl(p)| 2^-21 + 2^-24), fl(z) lies closer to q
// than 1/2, so rint(fl(z)) = q.  Otherwise -- within about |z| 2^-21 of a
// half-integer (one value in ten thousand at |z| ~ 100), or not finite --
// the exactly rounded quotient decides.  The check is per value, the branch
// to the divisions once per wave: an exact division costs about ten VALU
// instructions, one of them an 8-cycle v_rcp_f32, and a per-value branch
// about as much again.  (The fma is written out: this compiler contracts a
// multiply and a subtract even when both are spelled __fmul_rn / __fsub_rn.)
__device__ __forceinline__ float code_near(float x, float inv, bool& tie) {
  const float r = __fmul_rn(x, inv);
  const float q = rintf(r);
  const float e = __builtin_fmaf(x, inv, -q);
  tie = !(fabsf(e) < __builtin_fmaf(fabsf(r), -0x1p-21f, 0.5f - 0x1p-24f));
  return q;
}

// Code j of a word set to q (an integral float or NaN), clamped to [0,
// 2^BITS - 1] with NaN to 0.  8-bit: one v_cvt_pk_u8_f32 (round to nearest
// even, saturating to [0, 255], NaN to 0: measured, the same as fminf(fmaxf(q,
// 0), 255) for the integral q here).
template <int BITS>
__device__ __forceinline__ uint32_t put_code(uint32_t word, float q, int j) {
  if constexpr (BITS == 8) {
    return __builtin_amdgcn_cvt_pk_u8_f32(q, static_cast<uint32_t>(j), word);
  } else {
    constexpr float kBins = static_cast<float>((1 << BITS) - 1);
    const uint32_t mask = ((1u << BITS) - 1u) << (j * BITS);
    return (word & ~mask) | (static_cast<uint32_t>(fminf(fmaxf(q, 0.0f), kBins)) << (j * BITS));
  }
}

// Quantize one group of GS values spread over L consecutive lanes (VALS =
// GS / L values per lane, val(i) the lane's i-th T value as float; lo / hi:
// the min / max of the lane's own values): min / max across the lanes, then
// the edge-snapped affine rule, every operation an explicitly rounded
// intrinsic; each lane packs its own VALS codes to `dst` and lane 0 of the
// group stores the scale and bias.  Shared by quantize_kernel and
// requant_kernel so the two stay bit-identical.
template <typename Tag, int BITS, int GS, int L, bool DST16 = false, typename Val>
__device__ __forceinline__ void quantize_group(Val&& val, float w_min, float w_max, int part, uint32_t* dst,
                                               uint16_t* scale_dst, uint16_t* bias_dst) {
  constexpr int VALS = GS / L;
  constexpr int PER = 32 / BITS;
  constexpr int WORDS = VALS / PER;
  constexpr float kBins = static_cast<float>((1 << BITS) - 1);
  group_minmax<L>(w_min, w_max);
  float scale = fmaxf(__fdiv_rn(__fsub_rn(w_max, w_min), kBins), 1e-7f);
  const bool side = fabsf(w_min) > fabsf(w_max);
  scale = side ? scale : -scale;
  const float edge = side ? w_min : w_max;
  const float q0 = rintf(__fdiv_rn(edge, scale));
  const bool nz = q0 != 0.0f;
  if (nz) scale = __fdiv_rn(edge, q0);
  const float bias = nz ? edge : 0.0f;
  const float inv = __builtin_amdgcn_rcpf(scale);
  uint32_t words[WORDS];
  bool tie = false;
#pragma unroll
  for (int w = 0; w < WORDS; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      bool t;
      word = put_code<BITS>(word, code_near(__fsub_rn(val(w * PER + j), bias), inv, t), j);
      tie |= t;
    }
    words[w] = word;
  }
  if (__builtin_amdgcn_ballot_w64(tie)) {
#pragma unroll
    for (int w = 0; w < WORDS; ++w)
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        const float x = __fsub_rn(val(w * PER + j), bias);
        bool t;
        code_near(x, inv, t);
        if (t) words[w] = put_code<BITS>(words[w], rintf(__fdiv_rn(x, scale)), j);
      }
  }
  // DST16: dst is 16-byte aligned, one 16-byte store per 4 words (the
  // requant kernel measured 15.4 against 19.2 us at the C5 chunk with
  // single-word stores).
  if constexpr (DST16) {
    static_assert(WORDS % 4 == 0, "16-byte code stores");
#pragma unroll
    for (int w = 0; w < WORDS; w += 4)
      *reinterpret_cast<uint4*>(dst + w) = uint4{words[w], words[w + 1], words[w + 2], words[w + 3]};
  } else {
#pragma unroll
    for (int w = 0; w < WORDS; ++w) dst[w] = words[w];
  }
  if (part == 0) {
    *scale_dst = from_f32<Tag>(scale);
    *bias_dst = from_f32<Tag>(bias);
  }
}

// Min / max of a lane's N values val(i) (fminf / fmaxf: a NaN is ignored).
template <int N, typename Val>
__device__ __forceinline__ void lane_minmax(Val&& val, float& lo, float& hi) {
  lo = __builtin_huge_valf();
  hi = -__builtin_huge_valf();
#pragma unroll
  for (int i = 0; i < N; ++i) {
    lo = fminf(lo, val(i));
    hi = fmaxf(hi, val(i));
  }
}

}  // namespace
}  // namespace qsdpa

#endif  // QSDPA_QUANT_GROUP_H_
