// Split-K quantized decode on the VALU (any GQA factor; the MFMA kernel in
// decode_mfma.hip takes over for head groups of 16).
//
// Reference: the single-pass kernel mlx_qsdpa/kernels.py:42-160 and the
// split-K pass 1 / pass 2 kernels kernels.py:224-318 / 342-418.
//
// Work decomposition (gfx950, wave64):
//   grid  = (num_splits, H_kv * head_blocks, B); 256 threads = 4 waves.
//   A workgroup serves HB query heads that share one KV head, over one
//   contiguous token chunk, so every K/V byte it streams is reused HB times
//   from registers (the reference re-reads and re-dequantizes per head,
//   kernels.py:241, 265-305).
//   Inside a wave, L = D/E lanes cover one token row (E dims per lane, one
//   16/8/4-byte load each), so 64/L tokens are in flight per wave step and
//   every K/V row is read with one coalesced vector load per lane.
//   Every K/V element is dequantized as the reference's mx.dequantize does
//   (scale*code + bias, rounded to T with v_cvt_pk_{f16,bf16}_f32); q.k runs
//   on T pairs with v_dot2c_f32_{f16,bf16} and p*v accumulates in float.
//   Softmax is online in the log2 domain with a lazy rescale: the running
//   max only moves when a score exceeds it by more than 8 (so p <= 256).
// Partials are float32: acc[D], m, l per (batch, head, split); the merge
// kernel combines them with the log-sum-exp rule.  num_splits == 1 writes
// the normalised output directly (the single-pass case).
#include "abi_internal.h"
#include "common.h"

namespace qsdpa {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;  // running-max start (finite: no inf-inf)
constexpr float kRescale = 8.0f;
constexpr int kWaves = 4;

struct DecodeParams {
  int B, Hq, Hkv, N, D, gs, G, hb_count, num_splits;
  float qscale;  // softmax scale * log2(e)
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
  const uint16_t* kb;  // null => zero biases
  int64_t kb_sb, kb_sh, kb_sn;
  const uint16_t* vb;
  int64_t vb_sb, vb_sh, vb_sn;
  uint16_t* out;
  int64_t o_sb, o_sh;
  const void* mask;
  int mask_kind;
  int64_t m_sb, m_sh, m_sn;
  const int32_t* kv_start;
  float* part_acc;  // [B][Hq][splits][D]
  float* part_ml;   // [B][Hq][splits][2]
  void* ev_begin;   // profiling events (host side only)
  void* ev_end;
};

template <int WORDS>
struct Words {
  uint32_t w[WORDS];
};

template <int WORDS>
__device__ __forceinline__ Words<WORDS> load_words(const uint32_t* p) {
  Words<WORDS> r;
  if constexpr (WORDS % 4 == 0) {
#pragma unroll
    for (int i = 0; i < WORDS / 4; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[i];
      r.w[4 * i + 0] = v.x; r.w[4 * i + 1] = v.y; r.w[4 * i + 2] = v.z; r.w[4 * i + 3] = v.w;
    }
  } else if constexpr (WORDS == 2) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    r.w[0] = v.x; r.w[1] = v.y;
  } else {
    r.w[0] = p[0];
  }
  return r;
}

// Codes of E elements -> float (element e of the lane = word e/PER, slot e%PER).
template <int BITS, int E>
__device__ __forceinline__ void unpack_codes(const uint32_t* w, float* c) {
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < E / 4; ++i) {
      c[4 * i + 0] = static_cast<float>(w[i] & 0xFFu);
      c[4 * i + 1] = static_cast<float>((w[i] >> 8) & 0xFFu);
      c[4 * i + 2] = static_cast<float>((w[i] >> 16) & 0xFFu);
      c[4 * i + 3] = static_cast<float>(w[i] >> 24);
    }
  } else {
#pragma unroll
    for (int i = 0; i < E / 8; ++i) {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu;         // codes 0,2,4,6 as bytes
      const uint32_t hi = (w[i] >> 4) & 0x0F0F0F0Fu;  // codes 1,3,5,7 as bytes
      c[8 * i + 0] = static_cast<float>(lo & 0xFFu);
      c[8 * i + 1] = static_cast<float>(hi & 0xFFu);
      c[8 * i + 2] = static_cast<float>((lo >> 8) & 0xFFu);
      c[8 * i + 3] = static_cast<float>((hi >> 8) & 0xFFu);
      c[8 * i + 4] = static_cast<float>((lo >> 16) & 0xFFu);
      c[8 * i + 5] = static_cast<float>((hi >> 16) & 0xFFu);
      c[8 * i + 6] = static_cast<float>(lo >> 24);
      c[8 * i + 7] = static_cast<float>(hi >> 24);
    }
  }
}

template <typename Tag>
__device__ __forceinline__ float mask_value(const DecodeParams& p, int b, int h, int t) {
  const int64_t o = off3(b, h, t, p.m_sb, p.m_sh, p.m_sn);
  switch (p.mask_kind) {
    case QSDPA_BOOL:
      return static_cast<const uint8_t*>(p.mask)[o] ? 0.0f : -__builtin_huge_valf();
    case QSDPA_F16:
      return f16_bits_to_f32(static_cast<const uint16_t*>(p.mask)[o]) * kLog2e;
    case QSDPA_BF16:
      return bf16_bits_to_f32(static_cast<const uint16_t*>(p.mask)[o]) * kLog2e;
    default:
      return static_cast<const float*>(p.mask)[o] * kLog2e;
  }
}

template <typename Tag, int D, int BITS, int HB, int E>
__global__ __launch_bounds__(256) void decode_valu_kernel(DecodeParams p) {
  constexpr int L = D / E;            // lanes per token row
  constexpr int TPW = 64 / L;         // tokens per wave step
  constexpr int WORDS = E * BITS / 32;
  static_assert(64 % L == 0 && L >= 1, "bad lane split");

  const int split = blockIdx.x;
  const int hblk = blockIdx.y % p.hb_count;
  const int kvh = blockIdx.y / p.hb_count;
  const int b = blockIdx.z;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tok = lane / L;
  const int part = lane % L;
  const int d0 = part * E;
  const int grp = d0 / p.gs;
  const int h0 = kvh * p.G + hblk * HB;

  // Token range of this split (keys before kv_start[b] are never read).
  const int s0 = p.kv_start ? min(max(p.kv_start[b], 0), p.N) : 0;
  const int len = p.N - s0;
  const int chunk = (len + p.num_splits - 1) / p.num_splits;
  const int n0 = s0 + split * chunk;
  const int n1 = min(n0 + chunk, p.N);

  // q stays in T (exact) as packed pairs; the softmax scale is applied to
  // the float dot product.
  uint32_t q2[HB][E / 2];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    const uint16_t* qp = p.q + static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(h0 + h) * p.q_sh + d0;
#pragma unroll
    for (int e = 0; e < E / 2; ++e)
      q2[h][e] = static_cast<uint32_t>(qp[2 * e]) | (static_cast<uint32_t>(qp[2 * e + 1]) << 16);
  }

  float m[HB], l[HB], acc[HB][E];
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    m[h] = kNegBig;
    l[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[h][e] = 0.0f;
  }

  const uint32_t* kbase = p.kp + off3(b, kvh, 0, p.kp_sb, p.kp_sh, 0) + part * WORDS;
  const uint32_t* vbase = p.vp + off3(b, kvh, 0, p.vp_sb, p.vp_sh, 0) + part * WORDS;
  const uint16_t* ksb = p.ks + off3(b, kvh, 0, p.ks_sb, p.ks_sh, 0) + grp;
  const uint16_t* vsb = p.vs + off3(b, kvh, 0, p.vs_sb, p.vs_sh, 0) + grp;
  const uint16_t* kbb = p.kb ? p.kb + off3(b, kvh, 0, p.kb_sb, p.kb_sh, 0) + grp : nullptr;
  const uint16_t* vbb = p.vb ? p.vb + off3(b, kvh, 0, p.vb_sb, p.vb_sh, 0) + grp : nullptr;

  for (int tb = n0 + wave * TPW; tb < n1; tb += kWaves * TPW) {
    const int t = tb + tok;
    const bool valid = t < n1;
    const int tc = valid ? t : n0;  // clamp loads of idle lanes in-bounds
    const Words<WORDS> kw = load_words<WORDS>(kbase + static_cast<int64_t>(tc) * p.kp_sn);
    const Words<WORDS> vw = load_words<WORDS>(vbase + static_cast<int64_t>(tc) * p.vp_sn);
    const float ksf = to_f32<Tag>(ksb[static_cast<int64_t>(tc) * p.ks_sn]);
    const float vsf = to_f32<Tag>(vsb[static_cast<int64_t>(tc) * p.vs_sn]);
    const float kbf = kbb ? to_f32<Tag>(kbb[static_cast<int64_t>(tc) * p.kb_sn]) : 0.0f;
    const float vbf = vbb ? to_f32<Tag>(vbb[static_cast<int64_t>(tc) * p.vb_sn]) : 0.0f;

    // K: dequantize each element exactly as the reference's mx.dequantize
    // (scale*q + bias, rounded to T), then dot with q in T pairs.
    float code[E];
    unpack_codes<BITS, E>(kw.w, code);
    uint32_t k2[E / 2];
#pragma unroll
    for (int e = 0; e < E / 2; ++e)
      k2[e] = pack_T2<Tag>(fmaf(ksf, code[2 * e], kbf), fmaf(ksf, code[2 * e + 1], kbf));
    float sc[HB];
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      float dot = 0.0f;
#pragma unroll
      for (int e = 0; e < E / 2; ++e) dot = dot2<Tag>(q2[h][e], k2[e], dot);
      sc[h] = dot * p.qscale;
    }
#pragma unroll
    for (int h = 0; h < HB; ++h) sc[h] = group_sum<L>(sc[h]);
    if (p.mask) {
#pragma unroll
      for (int h = 0; h < HB; ++h) sc[h] += valid ? mask_value<Tag>(p, b, h0 + h, tc) : 0.0f;
    }

    // V: dequantize + round to T, back to float for the accumulation.
    unpack_codes<BITS, E>(vw.w, code);
#pragma unroll
    for (int e = 0; e < E / 2; ++e) {
      const uint32_t v2 = pack_T2<Tag>(fmaf(vsf, code[2 * e], vbf), fmaf(vsf, code[2 * e + 1], vbf));
      code[2 * e] = unpack_T2_lo<Tag>(v2);
      code[2 * e + 1] = unpack_T2_hi<Tag>(v2);
    }
#pragma unroll
    for (int h = 0; h < HB; ++h) {
      const float s = valid ? sc[h] : -__builtin_huge_valf();
      if (s > m[h] + kRescale) {
        const float f = fast_exp2(m[h] - s);
        m[h] = s;
        l[h] *= f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[h][e] *= f;
      }
      const float pr = fast_exp2(s - m[h]);
      l[h] += pr;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[h][e] = fmaf(pr, code[e], acc[h][e]);
    }
  }

  // ---- combine the TPW token streams of this wave (lanes with equal part) ----
#pragma unroll
  for (int h = 0; h < HB; ++h) {
    float mm = m[h];
#pragma unroll
    for (int x = L; x < 64; x <<= 1) mm = fmaxf(mm, shfl_xor_f32(mm, x));
    const float f = fast_exp2(m[h] - mm);
    float ll = l[h] * f;
#pragma unroll
    for (int x = L; x < 64; x <<= 1) ll += shfl_xor_f32(ll, x);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float a = acc[h][e] * f;
#pragma unroll
      for (int x = L; x < 64; x <<= 1) a += shfl_xor_f32(a, x);
      acc[h][e] = a;
    }
    m[h] = mm;
    l[h] = ll;
  }

  // ---- combine the waves through LDS ----
  __shared__ float sm_acc[kWaves][HB][D];
  __shared__ float sm_m[kWaves][HB];
  __shared__ float sm_l[kWaves][HB];
  if (tok == 0) {
#pragma unroll
    for (int h = 0; h < HB; ++h) {
#pragma unroll
      for (int e = 0; e < E; ++e) sm_acc[wave][h][d0 + e] = acc[h][e];
      if (part == 0) {
        sm_m[wave][h] = m[h];
        sm_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();

  for (int i = threadIdx.x; i < HB * D; i += blockDim.x) {
    const int h = i / D;
    const int d = i % D;
    float mm = sm_m[0][h];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mm = fmaxf(mm, sm_m[w][h]);
    float a = 0.0f, ll = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(sm_m[w][h] - mm);
      a = fmaf(sm_acc[w][h][d], f, a);
      ll = fmaf(sm_l[w][h], f, ll);
    }
    const int hq = h0 + h;
    if (p.num_splits == 1) {
      const float o = ll > 0.0f ? a / ll : 0.0f;
      p.out[static_cast<int64_t>(b) * p.o_sb + static_cast<int64_t>(hq) * p.o_sh + d] = from_f32<Tag>(o);
    } else {
      const int64_t slot = (static_cast<int64_t>(b) * p.Hq + hq) * p.num_splits + split;
      p.part_acc[slot * D + d] = a;
      if (d == 0) {
        p.part_ml[slot * 2 + 0] = mm;
        p.part_ml[slot * 2 + 1] = ll;
      }
    }
  }
}

template <typename Tag, int D, int BITS, int HB>
void launch_valu(const DecodeParams& p, hipStream_t stream) {
  constexpr int E = (HB == 1) ? 32 : (HB <= 4 ? 16 : 8);
  const dim3 grid(p.num_splits, p.Hkv * p.hb_count, p.B);
  launch_profiled(decode_valu_kernel<Tag, D, BITS, HB, E>, grid, dim3(256), stream, p.ev_begin, p.ev_end, p);
}

template <typename Tag, int D, int BITS>
void dispatch_hb(const DecodeParams& p, int hb, hipStream_t stream) {
  switch (hb) {
    case 1: launch_valu<Tag, D, BITS, 1>(p, stream); break;
    case 2: launch_valu<Tag, D, BITS, 2>(p, stream); break;
    case 4: launch_valu<Tag, D, BITS, 4>(p, stream); break;
    default: launch_valu<Tag, D, BITS, 8>(p, stream); break;
  }
}

template <typename Tag>
void dispatch_shape(const DecodeParams& p, int bits, int hb, hipStream_t stream) {
  switch (p.D) {
    case 64:
      if (bits == 4) dispatch_hb<Tag, 64, 4>(p, hb, stream); else dispatch_hb<Tag, 64, 8>(p, hb, stream);
      break;
    case 128:
      if (bits == 4) dispatch_hb<Tag, 128, 4>(p, hb, stream); else dispatch_hb<Tag, 128, 8>(p, hb, stream);
      break;
    default:
      if (bits == 4) dispatch_hb<Tag, 256, 4>(p, hb, stream); else dispatch_hb<Tag, 256, 8>(p, hb, stream);
      break;
  }
}

}  // namespace

// Heads per workgroup: the largest of 8, 4, 2, 1 dividing the GQA factor.
int valu_heads_per_block(int G) {
  for (int hb = 8; hb > 1; hb >>= 1)
    if (G % hb == 0) return hb;
  return 1;
}

int launch_decode_valu(const qsdpa_decode_args* a, int num_splits, float* part_acc,
                       float* part_ml, hipStream_t stream) {
  DecodeParams p;
  p.B = a->B; p.Hq = a->H_q; p.Hkv = a->H_kv; p.N = a->N; p.D = a->D; p.gs = a->group_size;
  p.G = a->H_q / a->H_kv;
  const int hb = valu_heads_per_block(p.G);
  p.hb_count = p.G / hb;
  p.num_splits = num_splits;
  p.qscale = a->scale * kLog2e;
  p.q = static_cast<const uint16_t*>(a->q.ptr); p.q_sb = a->q.stride_b; p.q_sh = a->q.stride_h;
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
  p.out = static_cast<uint16_t*>(const_cast<void*>(a->out.ptr));
  p.o_sb = a->out.stride_b; p.o_sh = a->out.stride_h;
  p.mask = a->mask.ptr; p.mask_kind = a->mask_dtype;
  p.m_sb = a->mask.stride_b; p.m_sh = a->mask.stride_h; p.m_sn = a->mask.stride_n;
  p.kv_start = a->kv_start;
  p.part_acc = part_acc;
  p.part_ml = part_ml;
  p.ev_begin = a->prof_begin;
  p.ev_end = a->prof_end;
  if (a->dtype == QSDPA_F16) dispatch_shape<F16>(p, a->bits, hb, stream);
  else dispatch_shape<BF16>(p, a->bits, hb, stream);
  return check_launch("decode_valu");
}

}  // namespace qsdpa
