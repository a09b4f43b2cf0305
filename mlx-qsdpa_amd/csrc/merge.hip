// Log-sum-exp merge of split-K partials (pass 2 of the two-pass decode).
//
// Reference: mlx_qsdpa/kernels.py:342-418 (online merge over blocks at
// 369-386, zero-sum guard at 408).  The reference stores partials in T
// (dispatch.py:235-239); here, per row r = (b*H_q + h)*qL + i and split s:
//   part_acc[r*splits + s][D]   float32 unnormalised sum of p * v, or (the
//                               MFMA kernels with float16 inputs, HALF) the
//                               normalised row acc / l as float16, in the
//                               first half of the same area
//   part_ml [r*splits + s][2]   (m, l): running max (log2 domain) and sum of
//                               p = exp2(score - m)
// out[b, h, i, :] = sum_s acc_s * exp2(m_s - M) / sum_s l_s * exp2(m_s - M),
// M = max_s m_s, and 0 when every split is empty (l = 0).
//
// Launch: grid (B*H_q, D/32), 256 threads = 32 split groups x 8 dim
// quads.  Thread (g, q) owns dims 4q..4q+3 of the block's 32 (one 16-byte
// load per split) and splits g, g + 32, ...; it issues all its loads of a
// round of 32 * kPer splits at once and keeps a running (m, l, acc) with
// rescaling, so 128 splits cost one memory round trip.  The 32 groups then
// merge with shuffles (8 per wave) and LDS (4 waves).
#include "abi_internal.h"
#include "common.h"

namespace qsdpa {
namespace {

constexpr int kMaxSplits = 1024;
constexpr int kGroups = 32;  // split groups per block
constexpr int kPer = 4;      // splits per thread per round
constexpr float kNegBig = -1.0e30f;

// HALF: the partial rows are float16 and normalised (acc / l), as the MFMA
// decode stores them for float16 inputs; the weight of split s is then
// l_s * exp2(m_s - M) for its row as well as for the sum.
//
// Rows are (b, h, i) for the qL query positions i, numbered
// (b * H_q + h) * qL + i; each holds `splits` partials.  sched != null
// (stream-K schedule of a left-padded batch): the partials of (h, i) are
// rows (h * qL + i) * units + c for `units` columns c, and sequence b owns
// columns sched[2b] .. sched[2b] + sched[2b + 1] - 1.
template <typename Tag, bool HALF>
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ part_acc,
                                                    const float* __restrict__ part_ml, int D,
                                                    int splits, int Hq, int qL, uint16_t* __restrict__ out,
                                                    int64_t o_sb, int64_t o_sh, int64_t o_sq,
                                                    const int* __restrict__ sched, int units) {
  const int bh = blockIdx.x;
  const int tid = threadIdx.x;
  const int q = tid & 7;
  const int g = tid >> 3;
  const int wave = tid >> 6;
  const int d = blockIdx.y * 32 + 4 * q;
  int64_t first = static_cast<int64_t>(bh) * splits;
  const int rows_b = Hq * qL;  // rows per sequence
  if (sched) {
    const int2 e = *reinterpret_cast<const int2*>(sched + 2 * (bh / rows_b));
    first = static_cast<int64_t>(bh % rows_b) * units + e.x;
    splits = e.y;
  }
  const float2* ml = reinterpret_cast<const float2*>(part_ml) + first;
  const float* pa = part_acc + first * D + d;
  const uint16_t* ph = reinterpret_cast<const uint16_t*>(part_acc) + first * D + d;

  float m = kNegBig, l = 0.0f;
  float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < splits; s0 += kGroups * kPer) {
    float4 x[kPer];
    float2 w[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = s0 + g + kGroups * k;
      const bool ok = s < splits;
      if constexpr (HALF) {
        const uint2 hv = ok ? *reinterpret_cast<const uint2*>(ph + static_cast<int64_t>(s) * D) : uint2{0u, 0u};
        x[k] = float4{f16_bits_to_f32(static_cast<uint16_t>(hv.x)), f16_bits_to_f32(static_cast<uint16_t>(hv.x >> 16)),
                      f16_bits_to_f32(static_cast<uint16_t>(hv.y)), f16_bits_to_f32(static_cast<uint16_t>(hv.y >> 16))};
      } else {
        x[k] = ok ? *reinterpret_cast<const float4*>(pa + static_cast<int64_t>(s) * D) : float4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      w[k] = ok ? ml[s] : float2{kNegBig, 0.0f};
    }
    float mr = m;
#pragma unroll
    for (int k = 0; k < kPer; ++k) mr = fmaxf(mr, w[k].x);
    const float f = fast_exp2(m - mr);
    l *= f;
    acc.x *= f; acc.y *= f; acc.z *= f; acc.w *= f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const float e = fast_exp2(w[k].x - mr);
      l = fmaf(w[k].y, e, l);
      const float ex = HALF ? w[k].y * e : e;  // weight of the row
      acc.x = fmaf(x[k].x, ex, acc.x); acc.y = fmaf(x[k].y, ex, acc.y);
      acc.z = fmaf(x[k].z, ex, acc.z); acc.w = fmaf(x[k].w, ex, acc.w);
    }
    m = mr;
  }

  // Block max of m (the same for every dim quad of a group).
  __shared__ float s_m[4];
  __shared__ float s_l[4];
  __shared__ float4 s_acc[4][8];
  float mw = m;
#pragma unroll
  for (int o = 8; o < 64; o <<= 1) mw = fmaxf(mw, shfl_xor_f32(mw, o));
  if ((tid & 63) == 0) s_m[wave] = mw;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
  const float f = fast_exp2(m - M);
  l *= f;
  acc.x *= f; acc.y *= f; acc.z *= f; acc.w *= f;
#pragma unroll
  for (int o = 8; o < 64; o <<= 1) {
    l += shfl_xor_f32(l, o);
    acc.x += shfl_xor_f32(acc.x, o); acc.y += shfl_xor_f32(acc.y, o);
    acc.z += shfl_xor_f32(acc.z, o); acc.w += shfl_xor_f32(acc.w, o);
  }
  if ((tid & 63) < 8) s_acc[wave][q] = acc;
  if ((tid & 63) == 0) s_l[wave] = l;
  __syncthreads();
  if (tid < 8) {
    const float L = (s_l[0] + s_l[1]) + (s_l[2] + s_l[3]);
    const float4 a0 = s_acc[0][tid], a1 = s_acc[1][tid], a2 = s_acc[2][tid], a3 = s_acc[3][tid];
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    const float o[4] = {((a0.x + a1.x) + (a2.x + a3.x)) * inv, ((a0.y + a1.y) + (a2.y + a3.y)) * inv,
                        ((a0.z + a1.z) + (a2.z + a3.z)) * inv, ((a0.w + a1.w) + (a2.w + a3.w)) * inv};
    const int b = bh / rows_b, h = (bh % rows_b) / qL, i = bh % qL;
    uint16_t* dst = out + static_cast<int64_t>(b) * o_sb + static_cast<int64_t>(h) * o_sh +
                    static_cast<int64_t>(i) * o_sq + blockIdx.y * 32 + 4 * tid;
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = from_f32<Tag>(o[e]);
  }
}

// Many rows with few splits each (prefill partials): one thread per (row,
// W dims), the splits in order with the same online rescaling as above,
// four splits' loads in flight at a time, one 16-byte load per split: W = 8
// for float16 rows (HALF), 4 for float32 rows.  (8 dims of float32 rows --
// two loads per split, half the threads -- took C5's prefill at q_len = 256
// 74.6-75.5 against 71.1-71.3 us per call; float16 rows with 8 dims took
// C3's heads at q_len = 512 128.6 against 130.5-130.9.)  Rows numbered as
// above, no stream-K schedule.  ALIGNED: every output row piece is
// 2W-byte aligned (one store; otherwise 16-bit stores).
template <typename Tag, bool HALF, bool ALIGNED>
__global__ __launch_bounds__(256) void merge_rows_kernel(const float* __restrict__ part_acc,
                                                         const float* __restrict__ part_ml, int D, int splits,
                                                         int Hq, int qL, int64_t rows, uint16_t* __restrict__ out,
                                                         int64_t o_sb, int64_t o_sh, int64_t o_sq) {
  constexpr int W = HALF ? 8 : 4;
  const int pieces = D / W;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= rows * pieces) return;
  const int64_t bh = idx / pieces;
  const int d = static_cast<int>(idx % pieces) * W;
  const int64_t first = bh * splits;
  const float2* ml = reinterpret_cast<const float2*>(part_ml) + first;
  const float* pa = part_acc + first * D + d;
  const uint16_t* ph = reinterpret_cast<const uint16_t*>(part_acc) + first * D + d;
  float m = kNegBig, l = 0.0f;
  float acc[W];
#pragma unroll
  for (int e = 0; e < W; ++e) acc[e] = 0.0f;
  for (int s0 = 0; s0 < splits; s0 += kPer) {
    float x[kPer][W];
    float2 w[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int s = s0 + k;
      const bool ok = s < splits;
      if constexpr (HALF) {
        const uint4 hv = ok ? *reinterpret_cast<const uint4*>(ph + static_cast<int64_t>(s) * D) : uint4{0u, 0u, 0u, 0u};
        const uint32_t u[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[k][2 * e] = f16_bits_to_f32(static_cast<uint16_t>(u[e]));
          x[k][2 * e + 1] = f16_bits_to_f32(static_cast<uint16_t>(u[e] >> 16));
        }
      } else {
        const float4 a0 = ok ? *reinterpret_cast<const float4*>(pa + static_cast<int64_t>(s) * D)
                             : float4{0.0f, 0.0f, 0.0f, 0.0f};
        x[k][0] = a0.x; x[k][1] = a0.y; x[k][2] = a0.z; x[k][3] = a0.w;
      }
      w[k] = ok ? ml[s] : float2{kNegBig, 0.0f};
    }
    float mr = m;
#pragma unroll
    for (int k = 0; k < kPer; ++k) mr = fmaxf(mr, w[k].x);
    const float f = fast_exp2(m - mr);
    l *= f;
#pragma unroll
    for (int e = 0; e < W; ++e) acc[e] *= f;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const float ek = fast_exp2(w[k].x - mr);
      l = fmaf(w[k].y, ek, l);
      const float ex = HALF ? w[k].y * ek : ek;
#pragma unroll
      for (int e = 0; e < W; ++e) acc[e] = fmaf(x[k][e], ex, acc[e]);
    }
    m = mr;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const int rows_b = Hq * qL;
  const int64_t b = bh / rows_b;
  const int h = static_cast<int>((bh % rows_b) / qL), i = static_cast<int>(bh % qL);
  uint16_t* dst = out + b * o_sb + static_cast<int64_t>(h) * o_sh + static_cast<int64_t>(i) * o_sq + d;
  uint32_t o[W / 2];
#pragma unroll
  for (int e = 0; e < W / 2; ++e)
    o[e] = from_f32<Tag>(acc[2 * e] * inv) | (static_cast<uint32_t>(from_f32<Tag>(acc[2 * e + 1] * inv)) << 16);
  if constexpr (ALIGNED && W == 8) {
    *reinterpret_cast<uint4*>(dst) = uint4{o[0], o[1], o[2], o[3]};
  } else if constexpr (ALIGNED) {
    *reinterpret_cast<uint2*>(dst) = uint2{o[0], o[1]};
  } else {
#pragma unroll
    for (int e = 0; e < W / 2; ++e) {
      dst[2 * e] = static_cast<uint16_t>(o[e]);
      dst[2 * e + 1] = static_cast<uint16_t>(o[e] >> 16);
    }
  }
}

template <typename Tag, bool HALF>
void launch_merge_rows(dim3 g, const float* part_acc, const float* part_ml, const qsdpa_decode_args* a, int splits,
                       int qL, int64_t rows, uint16_t* out, int64_t o_sq, hipStream_t stream) {
  // Aligned pieces (W = 8 or 4 values): the base and every stride a multiple of W elements.
  constexpr int W = HALF ? 8 : 4;
  const bool al = aligned(out, 2 * W) && a->out.stride_b % W == 0 && a->out.stride_h % W == 0 && o_sq % W == 0;
  if (al)
    merge_rows_kernel<Tag, HALF, true><<<g, dim3(256), 0, stream>>>(part_acc, part_ml, a->D, splits, a->H_q, qL, rows,
                                                                     out, a->out.stride_b, a->out.stride_h, o_sq);
  else
    merge_rows_kernel<Tag, HALF, false><<<g, dim3(256), 0, stream>>>(part_acc, part_ml, a->D, splits, a->H_q, qL, rows,
                                                                      out, a->out.stride_b, a->out.stride_h, o_sq);
}

}  // namespace

int launch_merge(const qsdpa_decode_args* a, int num_splits, const float* part_acc,
                 const float* part_ml, bool half_parts, const int* sched, int units, hipStream_t stream) {
  if (num_splits > kMaxSplits)
    return fail(QSDPA_ERR_INVALID, "merge: %d splits exceed %d", num_splits, kMaxSplits);
  uint16_t* out = static_cast<uint16_t*>(const_cast<void*>(a->out.ptr));
  const int qL = a->q_len > 1 ? a->q_len : 1;
  const int64_t o_sq = qL > 1 ? a->out.stride_n : 0;
  const int64_t rows = static_cast<int64_t>(a->B) * a->H_q * qL;
  if (!sched && num_splits <= 16 && rows >= 2048) {
    const int64_t threads = rows * (a->D / (a->dtype == QSDPA_F16 && half_parts ? 8 : 4));
    const dim3 g(static_cast<unsigned>((threads + 255) / 256));
    if (a->dtype == QSDPA_F16 && half_parts)
      launch_merge_rows<F16, true>(g, part_acc, part_ml, a, num_splits, qL, rows, out, o_sq, stream);
    else if (a->dtype == QSDPA_F16)
      launch_merge_rows<F16, false>(g, part_acc, part_ml, a, num_splits, qL, rows, out, o_sq, stream);
    else
      launch_merge_rows<BF16, false>(g, part_acc, part_ml, a, num_splits, qL, rows, out, o_sq, stream);
    return check_launch("merge_rows");
  }
  const dim3 grid(a->B * a->H_q * qL, a->D / 32);
  if (a->dtype == QSDPA_F16 && half_parts)
    merge_kernel<F16, true><<<grid, dim3(256), 0, stream>>>(part_acc, part_ml, a->D, num_splits, a->H_q, qL,
                                                            out, a->out.stride_b, a->out.stride_h, o_sq, sched, units);
  else if (a->dtype == QSDPA_F16)
    merge_kernel<F16, false><<<grid, dim3(256), 0, stream>>>(part_acc, part_ml, a->D, num_splits, a->H_q, qL,
                                                             out, a->out.stride_b, a->out.stride_h, o_sq, sched, units);
  else
    merge_kernel<BF16, false><<<grid, dim3(256), 0, stream>>>(part_acc, part_ml, a->D, num_splits, a->H_q, qL,
                                                              out, a->out.stride_b, a->out.stride_h, o_sq, sched, units);
  return check_launch("merge");
}

}  // namespace qsdpa
