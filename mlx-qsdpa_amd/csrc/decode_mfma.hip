// Head-grouped split-K quantized decode on the gfx950 matrix cores.
//
// Used when the GQA group is a multiple of 16 query heads (BASELINE config
// 3: 16 query heads per KV head), where the 16 heads sharing a KV head form
// a dense 16-wide MFMA tile.  Reference: kernels.py:224-318 (split-K pass 1),
// which instead runs one simdgroup per query head and re-dequantizes every
// K/V row once per head (kernels.py:241, 265-305).
//
// One workgroup = 8 waves = one (batch, kv head, 16-head block, token chunk).
// Each wave streams its own 32-token tiles of the chunk; every global load of
// a tile is issued one tile ahead (two register sets used alternately):
//
//   S^T[t, h] = K[t, :] . Q[h, :]   v_mfma_f32_16x16x32_{f16,bf16}: A = K
//       rows (a lane loads a contiguous quarter row of one token, 128-bit
//       loads), B = Q^T held in registers for the whole chunk.  K is
//       dequantized in registers exactly as mx.dequantize (T-rounded).
//   online softmax in the log2 domain on the C fragment: a lane owns one head
//       and 4 tokens per 16-token tile; the running max moves only when a
//       tile max exceeds it by more than 8 (p <= 256).
//   out^T[d, h] += V^T[d, t] P^T[t, h]   MFMA with A = V^T and B = P^T, where
//       P^T is exactly the lane's own softmax fragment (the k order of the
//       token axis is chosen to match the S^T C layout, so P never moves).
//       V is dequantized in registers, stored token-major to a wave-private
//       LDS tile and read back transposed with ds_read_b64_tr_b16.
//
// Float16: the fp16 dequantize is one v_pk_fma_f16 per pair (the "1024 + q"
// exponent trick makes the 4-bit codes exact fp16 without a conversion), P
// goes to fp16.  Bfloat16: the dequantize runs in fp32 and is rounded with
// v_cvt_pk_bf16_f32; P is split into two bf16 terms (hi + lo) so the P.V
// product keeps 16 significant bits.
//
// The four waves' (m, l, acc) states merge through LDS; a single split
// writes the normalised output, otherwise float32 partials for the LSE merge
// kernel in decode_valu.hip.
#include <algorithm>

#include "abi_internal.h"
#include "common.h"

namespace qsdpa {

int launch_merge(const qsdpa_decode_args* a, int num_splits, const float* part_acc,
                 const float* part_ml, hipStream_t stream);

namespace {

#ifndef QSDPA_MFMA_WAVES
#define QSDPA_MFMA_WAVES 8
#endif
constexpr int kWaves = QSDPA_MFMA_WAVES;  // waves per workgroup
constexpr int kThreads = kWaves * 64;
// Scheduling fence between the phases of a tile: keeps the compiler from
// hoisting one phase's loads / dequantization into another, which would
// raise register pressure past the 2-waves-per-SIMD budget.
#ifndef QSDPA_PHASE_FENCE
#define QSDPA_PHASE_FENCE 1
#endif
#define PHASE_FENCE()                                   \
  do {                                                  \
    if constexpr (QSDPA_PHASE_FENCE) __builtin_amdgcn_sched_barrier(0); \
  } while (0)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegBig = -1.0e30f;
constexpr float kRescale = 8.0f;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

struct MfmaParams {
  int B, Hq, Hkv, N, gs, G, hb_count, num_splits;
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
  float* part_acc;
  float* part_ml;
};

// Order of the 8 dims of one MFMA k-slice as the dequantizer produces them:
// slot j holds dim perm8(j) of the slice.
template <typename Tag, int BITS>
__device__ __forceinline__ constexpr int perm8(int j) {
  if constexpr (Tag::kId == QSDPA_F16 && BITS == 4) return (j >> 1) + 4 * (j & 1);
  else return j;
}

// Dequantize one 8-dim slice (BITS/4 packed words) to four T pairs,
// value = round_T(scale * code + bias), in perm8 order.
template <typename Tag, int BITS>
__device__ __forceinline__ void dequant8(const uint32_t* w, uint16_t s_bits, uint16_t b_bits,
                                         uint32_t out[4]) {
  if constexpr (Tag::kId == QSDPA_F16) {
    const f16x2 s2 = __builtin_bit_cast(f16x2, static_cast<uint32_t>(s_bits) * 0x10001u);
    const f16x2 b2 = __builtin_bit_cast(f16x2, static_cast<uint32_t>(b_bits) * 0x10001u);
    const f16x2 k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    uint32_t t[4];
    if constexpr (BITS == 4) {
      const uint32_t x = w[0];
      t[0] = (x & 0x000F000Fu) | 0x64006400u;          // codes 0, 4
      t[1] = ((x >> 4) & 0x000F000Fu) | 0x64006400u;   // codes 1, 5
      t[2] = ((x >> 8) & 0x000F000Fu) | 0x64006400u;   // codes 2, 6
      t[3] = ((x >> 12) & 0x000F000Fu) | 0x64006400u;  // codes 3, 7
    } else {
      t[0] = __builtin_amdgcn_perm(0x64646464u, w[0], 0x04010400u);  // codes 0, 1
      t[1] = __builtin_amdgcn_perm(0x64646464u, w[0], 0x04030402u);  // codes 2, 3
      t[2] = __builtin_amdgcn_perm(0x64646464u, w[1], 0x04010400u);
      t[3] = __builtin_amdgcn_perm(0x64646464u, w[1], 0x04030402u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f16x2 c = __builtin_bit_cast(f16x2, t[i]) - k1024;  // exact codes
      out[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, s2, b2));
    }
  } else {
    const float sf = bf16_bits_to_f32(s_bits);
    const float bf = bf16_bits_to_f32(b_bits);
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

template <int WORDS>
__device__ __forceinline__ void load_words(const uint32_t* p, uint32_t* w) {
  if constexpr (WORDS % 4 == 0) {
#pragma unroll
    for (int i = 0; i < WORDS / 4; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(p)[i];
      w[4 * i] = v.x; w[4 * i + 1] = v.y; w[4 * i + 2] = v.z; w[4 * i + 3] = v.w;
    }
  } else if constexpr (WORDS == 2) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else {
    w[0] = p[0];
  }
}

__device__ __forceinline__ float mask_value(const MfmaParams& p, int b, int h, int t) {
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

// Per-tile loads of one lane: two 16-token halves of K and V (the lane's
// quarter row of token tb + 16u + r16) plus their scales / biases for the
// (at most two) quantization groups the quarter row touches.
template <int WPL>
struct TileRegs {
  uint32_t kw[2][WPL];
  uint32_t vw[2][WPL];
  uint32_t ks[2], kb[2], vs[2], vb[2];  // low half: group g0, high half: g0 + 1
};

// Load the 16-bit (one group) or 2 x 16-bit (two groups) metadata of a row.
template <int NGL>
__device__ __forceinline__ uint32_t load_meta(const uint16_t* p) {
  if constexpr (NGL == 2) return *reinterpret_cast<const uint32_t*>(p);
  else return static_cast<uint32_t>(p[0]);
}

template <typename Tag, int D, int BITS, bool HAS_BIAS>
__global__ __launch_bounds__(kThreads) void decode_mfma_kernel(MfmaParams p) {
  constexpr int NM = D / 32;           // QK MFMAs (32 dims each)
  constexpr int NB = D / 16;           // PV MFMAs (16 output dims each)
  constexpr int QD = D / 4;            // dims per lane quarter row
  constexpr int NS = QD / 8;           // 8-dim slices per quarter row (= NM)
  constexpr int WPS = BITS / 4;        // packed words per slice
  constexpr int WPL = NS * WPS;        // packed words per quarter row
  constexpr int ROWB = D * 2 + 32;     // LDS bytes per V row (padded)
  static_assert(NS == NM, "slice count");
  constexpr int kTileBytes = 32 * ROWB;
  constexpr int kMergeBytes = kWaves * (D * 16 + 32) * 4;
  constexpr int kLdsBytes = kWaves * kTileBytes > kMergeBytes ? kWaves * kTileBytes : kMergeBytes;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int quad = lane >> 4;
  const int r16 = lane & 15;
  const int split = blockIdx.x;
  const int hblk = blockIdx.y % p.hb_count;
  const int kvh = blockIdx.y / p.hb_count;
  const int b = blockIdx.z;
  const int hq = kvh * p.G + hblk * 16 + r16;  // this lane's query head

  const int s0 = p.kv_start ? min(max(p.kv_start[b], 0), p.N) : 0;
  const int len = p.N - s0;
  const int chunk = (len + p.num_splits - 1) / p.num_splits;
  const int n0 = s0 + split * chunk;
  const int n1 = min(n0 + chunk, p.N);

  // Groups of the quarter row: g0 (and g0 + 1 when the row spans two).
  const int g0 = (quad * QD) / p.gs;
  const bool two_groups = QD > p.gs;  // uniform

  // Q^T as the B operand of the QK MFMAs (head r16, this quad's dims).
  uint32_t qb[NM][4];
  {
    const uint16_t* qp = p.q + static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(hq) * p.q_sh;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const int base = quad * QD + 8 * m;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        qb[m][i] = static_cast<uint32_t>(qp[base + perm8<Tag, BITS>(2 * i)]) |
                   (static_cast<uint32_t>(qp[base + perm8<Tag, BITS>(2 * i + 1)]) << 16);
    }
  }

  f4 acc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) acc[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun = kNegBig;
  float lrun = 0.0f;

  const uint32_t* kbase = p.kp + off3(b, kvh, 0, p.kp_sb, p.kp_sh, 0) + quad * WPL;
  const uint32_t* vbase = p.vp + off3(b, kvh, 0, p.vp_sb, p.vp_sh, 0) + quad * WPL;
  const uint16_t* ksb = p.ks + off3(b, kvh, 0, p.ks_sb, p.ks_sh, 0) + g0;
  const uint16_t* vsb = p.vs + off3(b, kvh, 0, p.vs_sb, p.vs_sh, 0) + g0;
  const uint16_t* kbb = HAS_BIAS ? p.kb + off3(b, kvh, 0, p.kb_sb, p.kb_sh, 0) + g0 : nullptr;
  const uint16_t* vbb = HAS_BIAS ? p.vb + off3(b, kvh, 0, p.vb_sb, p.vb_sh, 0) + g0 : nullptr;

  uint8_t* vt = lds + wave * kTileBytes;
  lds_u8* vl = (lds_u8*)vt;  // generic -> LDS address space
  const int rsel = 4 * quad + (r16 >> 2);
  const int csel = 4 * (r16 & 3) * 2;

  // Issue every global load of the tile starting at tb (no waits here).
  auto load_tile = [&](TileRegs<WPL>& R, int tb) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t tc = min(tb + 16 * u + r16, n1 - 1);
      load_words<WPL>(kbase + tc * p.kp_sn, R.kw[u]);
      load_words<WPL>(vbase + tc * p.vp_sn, R.vw[u]);
      if (two_groups) {
        R.ks[u] = load_meta<2>(ksb + tc * p.ks_sn);
        R.vs[u] = load_meta<2>(vsb + tc * p.vs_sn);
        if constexpr (HAS_BIAS) {
          R.kb[u] = load_meta<2>(kbb + tc * p.kb_sn);
          R.vb[u] = load_meta<2>(vbb + tc * p.vb_sn);
        }
      } else {
        R.ks[u] = load_meta<1>(ksb + tc * p.ks_sn);
        R.vs[u] = load_meta<1>(vsb + tc * p.vs_sn);
        if constexpr (HAS_BIAS) {
          R.kb[u] = load_meta<1>(kbb + tc * p.kb_sn);
          R.vb[u] = load_meta<1>(vbb + tc * p.vb_sn);
        }
      }
      if constexpr (!HAS_BIAS) {
        R.kb[u] = 0;
        R.vb[u] = 0;
      }
    }
  };

  // Scale / bias bits of slice m (its group is g0 or g0 + 1).
  auto meta_of = [&](uint32_t packed, int m) -> uint16_t {
    const bool hi = two_groups && (8 * m >= p.gs);
    return static_cast<uint16_t>(hi ? (packed >> 16) : (packed & 0xFFFFu));
  };

  auto compute_tile = [&](const TileRegs<WPL>& R, int tb) {
    // ---- S^T = K Q^T for the two 16-token halves ----
    f4 S[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      S[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        uint32_t a[4];
        dequant8<Tag, BITS>(R.kw[u] + m * WPS, meta_of(R.ks[u], m), meta_of(R.kb[u], m), a);
        S[u] = mfma<Tag>(a, qb[m], S[u]);
      }
    }
    PHASE_FENCE();
    // ---- V: dequantize to T, token-major into the wave's LDS tile ----
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      uint8_t* row = vt + (16 * u + r16) * ROWB + quad * QD * 2;
#pragma unroll
      for (int m = 0; m < NS; ++m) {
        uint32_t v[4];
        dequant8<Tag, BITS>(R.vw[u] + m * WPS, meta_of(R.vs[u], m), meta_of(R.vb[u], m), v);
        *reinterpret_cast<uint4*>(row + m * 16) = uint4{v[0], v[1], v[2], v[3]};
      }
    }
    PHASE_FENCE();
    // ---- scores (head r16, tokens tb + 16u + 4*quad + i), online softmax ----
    float sc[8];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[4 * u + i] = S[u][i] * p.qscale;
    if (p.mask) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = min(tb + 16 * (j >> 2) + 4 * quad + (j & 3), n1 - 1);
        sc[j] += mask_value(p, b, hq, t);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (tb + 16 * (j >> 2) + 4 * quad + (j & 3) >= n1) sc[j] = -__builtin_huge_valf();
    float tmax = sc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, sc[i]);
    tmax = fmaxf(tmax, shfl_xor_f32(tmax, 16));
    tmax = fmaxf(tmax, shfl_xor_f32(tmax, 32));
    if (tmax > mrun + kRescale) {
      const float f = fast_exp2(mrun - tmax);
      mrun = tmax;
      lrun *= f;
#pragma unroll
      for (int i = 0; i < NB; ++i) acc[i] *= f;
    }
    float pr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pr[i] = fast_exp2(sc[i] - mrun);
      lrun += pr[i];
    }
    // ---- P^T operand (k order = tokens 4q..4q+3 of half 0, then of half 1) ----
    uint32_t pb[4], pb_lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = pack_T2<Tag>(pr[2 * i], pr[2 * i + 1]);
    if constexpr (Tag::kId == QSDPA_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pb_lo[i] = pack_T2<Tag>(pr[2 * i] - unpack_T2_lo<Tag>(pb[i]),
                                pr[2 * i + 1] - unpack_T2_hi<Tag>(pb[i]));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- out^T += V^T P^T (V^T rows read transposed from the LDS tile) ----
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(vl + rsel * ROWB + nb * 32 + csel));
      const s4 hi =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(vl + (16 + rsel) * ROWB + nb * 32 + csel));
      const uint2 l2 = __builtin_bit_cast(uint2, lo);
      const uint2 h2 = __builtin_bit_cast(uint2, hi);
      const uint32_t a[4] = {l2.x, l2.y, h2.x, h2.y};
      acc[nb] = mfma<Tag>(a, pb, acc[nb]);
      if constexpr (Tag::kId == QSDPA_BF16) acc[nb] = mfma<Tag>(a, pb_lo, acc[nb]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // Software pipeline: the next tile's loads are in flight while the current
  // tile computes.  One loop body (the prefetched set is copied over), which
  // keeps the compiler from interleaving two inlined tile bodies.
  constexpr int kStride = kWaves * 32;
  TileRegs<WPL> A, Bt;
  int tb = n0 + wave * 32;
  if (tb < n1) load_tile(A, tb);
  while (tb < n1) {
    const int tb2 = tb + kStride;
    if (tb2 < n1) load_tile(Bt, tb2);
    compute_tile(A, tb);
    A = Bt;
    tb = tb2;
  }

  // ---- per-head totals over the four quads ----
  lrun += shfl_xor_f32(lrun, 16);
  lrun += shfl_xor_f32(lrun, 32);

  // ---- merge the waves through LDS: acc[w][h][d] in natural dim order ----
  __syncthreads();
  float* sm = reinterpret_cast<float*>(lds);
  float* sacc = sm + wave * (D * 16 + 32);
  float* sml = sacc + D * 16;  // [16 heads][2]
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int dp = 16 * nb + 4 * quad + r;               // slot (physical) dim
      const int d = (dp & ~7) + perm8<Tag, BITS>(dp & 7);  // real dim
      sacc[r16 * D + d] = acc[nb][r];
    }
  }
  if (quad == 0) {
    sml[2 * r16] = mrun;
    sml[2 * r16 + 1] = lrun;
  }
  __syncthreads();

  for (int i = threadIdx.x; i < 16 * D; i += kThreads) {
    const int h = i / D;
    const int d = i % D;
    float mm = kNegBig;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mm = fmaxf(mm, sm[w * (D * 16 + 32) + D * 16 + 2 * h]);
    float a = 0.0f, ll = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float* base = sm + w * (D * 16 + 32);
      const float f = fast_exp2(base[D * 16 + 2 * h] - mm);
      a = fmaf(base[h * D + d], f, a);
      ll = fmaf(base[D * 16 + 2 * h + 1], f, ll);
    }
    const int hh = kvh * p.G + hblk * 16 + h;
    if (p.num_splits == 1) {
      const float o = ll > 0.0f ? a / ll : 0.0f;
      p.out[static_cast<int64_t>(b) * p.o_sb + static_cast<int64_t>(hh) * p.o_sh + d] = from_f32<Tag>(o);
    } else {
      const int64_t slot = (static_cast<int64_t>(b) * p.Hq + hh) * p.num_splits + split;
      p.part_acc[slot * D + d] = a;
      if (d == 0) {
        p.part_ml[slot * 2] = mm;
        p.part_ml[slot * 2 + 1] = ll;
      }
    }
  }
}

template <typename Tag, int D, int BITS>
void launch_b(const MfmaParams& p, bool has_bias, hipStream_t stream) {
  const dim3 grid(p.num_splits, p.Hkv * p.hb_count, p.B);
  if (has_bias) decode_mfma_kernel<Tag, D, BITS, true><<<grid, dim3(kThreads), 0, stream>>>(p);
  else decode_mfma_kernel<Tag, D, BITS, false><<<grid, dim3(kThreads), 0, stream>>>(p);
}

template <typename Tag, int D>
void launch_d(const MfmaParams& p, int bits, bool has_bias, hipStream_t stream) {
  if (bits == 4) launch_b<Tag, D, 4>(p, has_bias, stream);
  else launch_b<Tag, D, 8>(p, has_bias, stream);
}

// LDS bytes one workgroup of the MFMA kernel uses for head dimension D.
constexpr int mfma_lds_bytes(int D) {
  return kWaves * 32 * (D * 2 + 32) > kWaves * (D * 16 + 32) * 4 ? kWaves * 32 * (D * 2 + 32)
                                                                  : kWaves * (D * 16 + 32) * 4;
}

bool meta_aligned4(const qsdpa_view& v) {
  return v.ptr == nullptr || ((reinterpret_cast<uintptr_t>(v.ptr) & 3) == 0 && v.stride_b % 2 == 0 &&
                              v.stride_h % 2 == 0 && v.stride_n % 2 == 0);
}

}  // namespace

// MFMA path: head groups that are a multiple of 16 wide.  When a lane's
// quarter row spans two quantization groups their scales are read as one
// 32-bit word, which needs 4-byte aligned scale / bias rows.
bool mfma_supports(const qsdpa_decode_args* a) {
  const int G = a->H_q / a->H_kv;
  if (G < 16 || G % 16 != 0) return false;
  if (a->D != 64 && a->D != 128 && a->D != 256) return false;
  if (a->D / 4 > a->group_size)
    return meta_aligned4(a->k_scales) && meta_aligned4(a->v_scales) && meta_aligned4(a->k_biases) &&
           meta_aligned4(a->v_biases);
  return true;
}

// As many workgroups as fit on the GPU at once (LDS-limited), but at least
// two 32-token tiles per wave.
int mfma_num_splits(const qsdpa_decode_args* a, int cus) {
  const int G = a->H_q / a->H_kv;
  const int64_t units = static_cast<int64_t>(a->B) * a->H_kv * (G / 16);
  const int per_cu = std::max(1, std::min(2, (160 * 1024) / mfma_lds_bytes(a->D)));
  const int64_t target = static_cast<int64_t>(per_cu) * cus;
  int64_t s = (target + units - 1) / units;
  s = std::min<int64_t>(s, std::max<int64_t>(1, a->N / (kWaves * 64)));
  s = std::min<int64_t>(s, 1024);
  return static_cast<int>(std::max<int64_t>(s, 1));
}

int launch_decode_mfma(const qsdpa_decode_args* a, int num_splits, float* part_acc, float* part_ml,
                       hipStream_t stream) {
  MfmaParams p;
  p.B = a->B; p.Hq = a->H_q; p.Hkv = a->H_kv; p.N = a->N; p.gs = a->group_size;
  p.G = a->H_q / a->H_kv;
  p.hb_count = p.G / 16;
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
  const bool f16 = a->dtype == QSDPA_F16;
  const bool hb = a->k_biases.ptr != nullptr;
  switch (a->D) {
    case 64: if (f16) launch_d<F16, 64>(p, a->bits, hb, stream); else launch_d<BF16, 64>(p, a->bits, hb, stream); break;
    case 128: if (f16) launch_d<F16, 128>(p, a->bits, hb, stream); else launch_d<BF16, 128>(p, a->bits, hb, stream); break;
    default: if (f16) launch_d<F16, 256>(p, a->bits, hb, stream); else launch_d<BF16, 256>(p, a->bits, hb, stream); break;
  }
  return check_launch("decode_mfma");
}

}  // namespace qsdpa
