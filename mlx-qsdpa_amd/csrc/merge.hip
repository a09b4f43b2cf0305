// Log-sum-exp merge of split-K partials (pass 2 of the two-pass decode).
//
// Reference: mlx_qsdpa/kernels.py:342-418 (online merge over blocks at
// 369-386, zero-sum guard at 408).  Partials here are float32 (the reference
// stores them in T, dispatch.py:235-239):
//   part_acc[(b*H_q + h)*splits + s][D]   unnormalised sum of p * v
//   part_ml [(b*H_q + h)*splits + s][2]   (m, l): running max (log2 domain)
//                                          and sum of p = exp2(score - m)
// out[b, h, :] = sum_s acc_s * exp2(m_s - M) / sum_s l_s * exp2(m_s - M),
// M = max_s m_s, and 0 when every split is empty (l = 0).
//
// Launch: grid (B*H_q, D/16), 256 threads = 16 split lanes x 16 dims.  A
// thread's first kPrefetch partial loads are issued before the block
// reductions of (m, l), so one memory round trip covers up to 128 splits.
#include "abi_internal.h"
#include "common.h"

namespace qsdpa {
namespace {

constexpr int kMaxSplits = 1024;
constexpr int kPrefetch = 8;
constexpr float kNegBig = -1.0e30f;

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, shfl_xor_f32(x, m));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += shfl_xor_f32(x, m);
  return x;
}

template <typename Tag>
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ part_acc,
                                                    const float* __restrict__ part_ml, int D,
                                                    int splits, int Hq, uint16_t* __restrict__ out,
                                                    int64_t o_sb, int64_t o_sh) {
  const int bh = blockIdx.x;
  const int tid = threadIdx.x;
  const int dd = tid & 15;
  const int sg = tid >> 4;
  const int wave = tid >> 6;
  const int d = blockIdx.y * 16 + dd;
  const float* ml = part_ml + static_cast<int64_t>(bh) * splits * 2;
  const float* pa = part_acc + static_cast<int64_t>(bh) * splits * D + d;

  float x[kPrefetch];
#pragma unroll
  for (int k = 0; k < kPrefetch; ++k) {
    const int s = sg + 16 * k;
    x[k] = s < splits ? pa[static_cast<int64_t>(s) * D] : 0.0f;
  }

  __shared__ float s_w[kMaxSplits];
  __shared__ float s_red[2][4];
  __shared__ float s_acc[16][17];

  float mloc = kNegBig;
  for (int s = tid; s < splits; s += 256) mloc = fmaxf(mloc, ml[2 * s]);
  mloc = wave_max(mloc);
  if ((tid & 63) == 0) s_red[0][wave] = mloc;
  __syncthreads();
  const float M = fmaxf(fmaxf(s_red[0][0], s_red[0][1]), fmaxf(s_red[0][2], s_red[0][3]));
  float lloc = 0.0f;
  for (int s = tid; s < splits; s += 256) {
    const float w = fast_exp2(ml[2 * s] - M);
    s_w[s] = w;
    lloc = fmaf(ml[2 * s + 1], w, lloc);
  }
  lloc = wave_sum(lloc);
  if ((tid & 63) == 0) s_red[1][wave] = lloc;
  __syncthreads();
  const float L = (s_red[1][0] + s_red[1][1]) + (s_red[1][2] + s_red[1][3]);

  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < kPrefetch; ++k) {
    const int s = sg + 16 * k;
    if (s < splits) acc = fmaf(x[k], s_w[s], acc);
  }
  for (int s = sg + 16 * kPrefetch; s < splits; s += 16)
    acc = fmaf(pa[static_cast<int64_t>(s) * D], s_w[s], acc);
  s_acc[sg][dd] = acc;
  __syncthreads();
  if (tid < 16) {
    float t = 0.0f;
#pragma unroll
    for (int g = 0; g < 16; ++g) t += s_acc[g][tid];
    const int b = bh / Hq, h = bh % Hq;
    const float o = L > 0.0f ? t / L : 0.0f;
    out[static_cast<int64_t>(b) * o_sb + static_cast<int64_t>(h) * o_sh + blockIdx.y * 16 + tid] =
        from_f32<Tag>(o);
  }
}

}  // namespace

int launch_merge(const qsdpa_decode_args* a, int num_splits, const float* part_acc,
                 const float* part_ml, hipStream_t stream) {
  if (num_splits > kMaxSplits)
    return fail(QSDPA_ERR_INVALID, "merge: %d splits exceed %d", num_splits, kMaxSplits);
  uint16_t* out = static_cast<uint16_t*>(const_cast<void*>(a->out.ptr));
  const dim3 grid(a->B * a->H_q, a->D / 16);
  if (a->dtype == QSDPA_F16)
    merge_kernel<F16><<<grid, dim3(256), 0, stream>>>(part_acc, part_ml, a->D, num_splits, a->H_q,
                                                      out, a->out.stride_b, a->out.stride_h);
  else
    merge_kernel<BF16><<<grid, dim3(256), 0, stream>>>(part_acc, part_ml, a->D, num_splits, a->H_q,
                                                       out, a->out.stride_b, a->out.stride_h);
  return check_launch("merge");
}

}  // namespace qsdpa
