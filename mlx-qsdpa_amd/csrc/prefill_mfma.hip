// Quantized attention for many query positions (prefill, chunked and
// speculative decoding) on the gfx950 matrix cores.
//
// Reference: the reference sends every qL > 1 call through dequantize +
// mx.fast.scaled_dot_product_attention (mlx_qsdpa/dispatch.py:68-83); the
// decode kernel (decode_mfma.hip) takes such calls in blocks of 16 query rows,
// each of which loads and dequantizes the kv head's whole K / V again.  Here
// one workgroup takes 128 rows of a kv head -- 8 waves x 16 rows -- and every
// K / V tile (64 tokens at D = 128, 32 at D = 256: the same number of
// values) is loaded once per workgroup, dequantized once into LDS, and read
// from LDS by all eight waves.  Per tile j, in each wave (described for
// D = 128; PGeo gives the D = 256 shapes):
//
//   QK         S^T = K Q^T (A = K rows from LDS buffer j % 4, B = Q^T in
//              registers): 4 token blocks x D/32 steps of v_mfma_f32_16x16x32
//              in the input type T, steps outer so that consecutive MFMAs
//              feed four independent accumulators (D = 256: 2 token blocks,
//              each with two accumulators for alternate steps);
//   dequant    every thread turns its piece of tile j + 2 (raw codes, scales
//              and biases loaded two tiles ahead into one of two register
//              sets) into values in LDS buffer (j + 2) % 4 -- K row-major
//              (token, dims) in T, V transposed (dim, tokens) as float16,
//              with the tokens of each 32-token half in the order of the S^T
//              fragment so that the P^T operand is a lane's own softmax
//              values -- and reissues that register set's loads for tile
//              j + 4.  Waves 4-7 do this after their QK MFMAs, waves 0-3
//              after their P.V, so that the two waves of a SIMD alternate
//              MFMA and VALU phases (120 against 124 us at the C5 chunk).
//              The SIMD's arbiter favours the older wave (0-3), which left
//              waves 4-7 the longer path per tile (their dequantization
//              contends with the other wave's softmax): they raise their
//              priority from their dequantization to the end of the tile
//              (117 against 121 us; without it 113-115 against 108-109 us
//              with four buffers, where the other placements lose 1.5-3.5 us);
//   softmax    online, in the log2 domain, rescaled when the maximum grows
//              by more than 8 (the decode kernel's); without a mask tensor
//              the score scale is applied inside the exponent's fma; the
//              tile maximum over a row's four lanes by row swaps (VALU)
//              rather than LDS permutes;
//   PV         out^T += V^T P^T in float16 (A = V^T rows from LDS, B = P^T);
//   barrier    one per pair of tiles (four buffers, 155,648 B of LDS at
//              D = 128, 151,552 B at D = 256): a
//              buffer is rewritten two tiles after its last reads, and read
//              two tiles after its writes, so one barrier after every odd
//              tile orders both, and the waves drift by up to two tiles
//              between barriers (108.4-108.9 against 109.9-110.1 us at the
//              C5 chunk with a barrier per tile and two buffers).
//
// P.V runs in float16 for bfloat16 inputs too.  V is rounded to bfloat16
// exactly as mx.dequantize rounds it, then scaled by 2^-k and converted to
// float16, which is exact for magnitudes from 2^-17 up (below that the error
// is at most 2^-25 * 2^k).  A scan of the workgroup's V scales and biases
// gives max |V| (at code 0 or 2^bits - 1 of each group): k is 0 unless it
// reaches kVBound (the output is scaled back by 2^k), and P (in [0, 256])
// enters as one float16 term -- the float16 path's 11 significant bits, one
// MFMA per block -- while max |V| is at most kPVSingle, as two terms (hi +
// lo, 22 bits) above it.
//
// Rows of a kv head are (position v / G, head v % G) as in the decode
// kernel; a causal mask (aligned to the last key), kv_start (keys before it
// are skipped) and a bool / additive mask are applied per score.  Calls with
// a mask tensor run their own instantiation (MASK), whose lanes load their 16
// mask values per tile from one base address with immediate offsets when the
// mask's keys are adjacent (C5 chunk with a bool mask: 142 against 186 us
// with per-key 64-bit offsets).  The grid
// maps the row groups of one (batch, kv head) to one XCD, so its K / V is
// fetched into one L2.
#include <type_traits>

#include "mfma_common.h"

namespace qsdpa {
namespace {

// Workgroup shape: 8 waves x 16 rows (two waves per SIMD).  Measured at the
// C5 chunk (B=4, H_q=16, H_kv=4, N=4096, q_len=512, bf16 8-bit) with
// bfloat16 P.V: 144 us; 4 waves x 32 rows (one wave per SIMD, about 380
// registers) 171-174 us; 4 waves x 16 rows (64-row groups, two per CU)
// 172 us.
constexpr int kPWaves = 8;
constexpr int kPThreads = kPWaves * 64;
constexpr int kPGroupRows = kPWaves * 16;    // query rows per workgroup
// Up to 256 key splits, so that one row group per kv head still covers every
// CU (with 64, C3's heads at q_len = 8 over 128K keys left half the CUs idle:
// 109-111 against 75-80 us per call).
constexpr int kMaxPrefillSplits = 256;
constexpr float kVBound = 64000.0f;          // largest |V| staged in float16 unscaled
// bfloat16 inputs: the largest max |V| for which P enters the P.V MFMAs as
// one float16 term (11 significant bits); above it, as two (hi + lo, 22
// bits).  P's rounding moves an output by up to 2^-11 max|V| (about 2^-12
// max|V| in the random tests), so one term keeps 2e-3 for |V| <= 8.
constexpr float kPVSingle = 8.0f;

// Tile geometry.  D = 128: 64-token tiles; D = 256: 32-token tiles, so that
// a tile holds the same number of K / V values (and the four LDS buffers
// still fit): the same MFMA, dequantization and LDS work per tile.
//
// LDS rows are padded.  Measured at the C5 chunk (D = 128): with 16-byte
// padding (K 272 B, V^T 144 B per row) the 16-byte operand reads of the 16
// rows of an MFMA block spend 1.8e7 bank-conflict cycles per call, with 32
// bytes 2.0e6, and the kernel takes 121-123 us instead of 129-130; 48 and
// 64 bytes conflict like 16.  D = 256 keeps K's row pitch modulo 256 bytes
// (544 = 2 * 256 + 32) and pads V^T's 64-byte rows by 16 (80 B, 20 dwords:
// the 16 rows of an operand read start on 16 distinct 4-dword bank groups),
// which is what fits four buffers in the LDS.
template <int D>
struct PGeo {
  static constexpr int Tile = D == 256 ? 32 : 64;  // tokens per tile
  static constexpr int KPitch = D * 2 + 32;        // bytes per K row (token) in LDS
  static constexpr int VPitch = Tile * 2 + (D == 256 ? 16 : 32);  // bytes per V^T row (dim)
  static constexpr int KBytes = Tile * KPitch;
  static constexpr int VBytes = D * VPitch;
  static constexpr int BufBytes = KBytes + VBytes;
  static constexpr int NM = D / 32;                // QK k-steps
  static constexpr int NB = D / 16;                // PV dim blocks
  static constexpr int NT = Tile / 16;             // S^T token blocks
  static constexpr int NU = Tile / 32;             // P^T k-steps (32-token halves)
  // QK accumulators per token block: with two token blocks, the k-steps
  // alternate between two (summed after the last) so that four independent
  // MFMA chains run, as with four token blocks.
  static constexpr int KS = NT < 4 ? 2 : 1;
  // The workgroup's threads split a tile: K token tid / KPT, dims
  // [c D / KPT, (c + 1) D / KPT) with c = tid % KPT; V tokens 2 pr + e
  // (pr = tid % Pairs, e = 0, 1), dims [cv D / VPT, (cv + 1) D / VPT) with
  // cv = tid / Pairs.
  static constexpr int KPT = kPThreads / Tile;
  static constexpr int Pairs = Tile / 2;
  static constexpr int VPT = kPThreads / Pairs;
  static_assert(4 * BufBytes + 64 <= 160 * 1024, "four LDS buffers");
};

// Column of token t (0..Tile-1) of a tile in the V^T rows: within each 32-token
// half, the slot order of the S^T fragment (lane quad q holds tokens
// 16 * (j >> 2) + 4 q + (j & 3), j = 0..7, as its k slots 8 q + j).
__device__ __forceinline__ int vcol(int t) {
  const int u = t >> 5, tt = t & 31;
  return 32 * u + 8 * ((tt >> 2) & 3) + 4 * (tt >> 4) + (tt & 3);
}

// Element pair i of a dequantized 8-dim slice (dequant_k's output): the two
// dims it holds (float16 4-bit: i and i + 4; otherwise 2i and 2i + 1).
template <typename Tag, int BITS>
__device__ __forceinline__ int pair_dim(int i, int half) {
  if constexpr (Tag::kId == QSDPA_F16 && BITS == 4) return i + 4 * half;
  else return 2 * i + half;
}

// Loads at the thread's byte offset `voff` plus the uniform `soff` (the
// buffer instruction's scalar offset, which the range check includes: words
// past the descriptor's size read as zero either way).
template <int W>
__device__ __forceinline__ void load_words(rsrc_t rs, uint32_t voff, uint32_t soff, uint32_t* w) {
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  if constexpr (W % 4 == 0) {
#pragma unroll
    for (int i = 0; i < W / 4; ++i) {
      const u4 x = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16 * i, soff, 0);
      w[4 * i] = x[0]; w[4 * i + 1] = x[1]; w[4 * i + 2] = x[2]; w[4 * i + 3] = x[3];
    }
  } else if constexpr (W == 2) {
    const u2 x = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0);
    w[0] = x[0]; w[1] = x[1];
  } else {
    static_assert(W == 1, "piece size");
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0);
  }
}

// Raw registers of one tile for one thread (the split above).  Single
// scale / bias half-words stay 16-bit values: widened, the compiler masks
// them as soon as they arrive, and that mask waits for every load in flight.
template <int D, int BITS, int GS>
struct PRaw {
  static constexpr int KW = D / PGeo<D>::KPT * BITS / 32;
  static constexpr int VW = D / PGeo<D>::VPT * BITS / 32;
  using KMeta = std::conditional_t<(D / PGeo<D>::KPT > GS), uint32_t, uint16_t>;  // two groups: both half-words
  uint32_t k[KW];
  KMeta ks, kb;
  uint32_t v[2][VW];
  uint16_t vs[2], vb[2];
};

// Two bfloat16 values (a packed pair) -> the float16 pair of the same values.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t x) {
  return pack_T2<F16>(__builtin_bit_cast(float, x << 16), __builtin_bit_cast(float, x & 0xFFFF0000u));
}

template <typename Tag, int D, int BITS, int GS>
struct Prefill {
  using PG = PGeo<D>;
  using Raw = PRaw<D, BITS, GS>;
  static constexpr int kKPT = PG::KPT, kPairs = PG::Pairs;
  static constexpr int kVPitch = PG::VPitch;
  static constexpr int kQD = D / kKPT;                    // K dims per thread
  static constexpr int kKG = kQD > GS ? kQD / GS : 1;     // groups per K piece (1 or 2)
  static constexpr int kVD = D / PG::VPT;                 // V dims per thread and token
  static_assert(kKG <= 2, "groups per K quarter");
  static_assert(kVD <= GS, "a V piece lies in one group");

  struct Src {
    rsrc_t k, v, ks, vs, kb, vb;
    uint32_t k_sn, v_sn, ks_sn, vs_sn, kb_sn, vb_sn;  // bytes per token
    uint32_t k_l, ks_l, kb_l, v_l[2], vs_l[2], vb_l[2];  // the thread's fixed byte offsets
  };

  // The thread's fixed part of every load offset (its token in the tile
  // times the stride, plus its dims), once per kernel.  Opaque to the
  // optimizer: seeing token * stride inside, it folds a load's uniform
  // row * stride + offset into a per-lane (row + token) * stride, one
  // quarter-rate v_mul_lo_u32 per load and tile.
  static __device__ __forceinline__ void lanes(Src& s, int tid) {
    const uint32_t kt = static_cast<uint32_t>(tid / kKPT);
    const int c = tid % kKPT;
    const uint32_t g0 = static_cast<uint32_t>(c * kQD / GS);
    s.k_l = kt * s.k_sn + static_cast<uint32_t>(c * Raw::KW * 4);
    s.ks_l = kt * s.ks_sn + g0 * 2;
    s.kb_l = kt * s.kb_sn + g0 * 2;
    const int pr = tid % kPairs, cv = tid / kPairs;
    const uint32_t gv = static_cast<uint32_t>(cv * kVD / GS);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t vt = static_cast<uint32_t>(2 * pr + e);
      s.v_l[e] = vt * s.v_sn + static_cast<uint32_t>(cv * Raw::VW * 4);
      s.vs_l[e] = vt * s.vs_sn + gv * 2;
      s.vb_l[e] = vt * s.vb_sn + gv * 2;
    }
    asm("" : "+v"(s.k_l), "+v"(s.ks_l), "+v"(s.kb_l), "+v"(s.v_l[0]), "+v"(s.v_l[1]));
    asm("" : "+v"(s.vs_l[0]), "+v"(s.vs_l[1]), "+v"(s.vb_l[0]), "+v"(s.vb_l[1]));
  }

  // Issue the loads of the tile whose first token is `rel0` tokens past the
  // sequence's first key (rows past the end read as zero): the thread's
  // fixed part as the vector offset, the tile's row times the row stride
  // (uniform) as the scalar offset, so that no load takes a VALU add.
  static __device__ __forceinline__ void load(Raw& R, const Src& s, int rel0) {
    const uint32_t row = static_cast<uint32_t>(rel0);
    load_words<Raw::KW>(s.k, s.k_l, row * s.k_sn, R.k);
    if constexpr (kKG == 2) {
      R.ks = __builtin_amdgcn_raw_buffer_load_b32(s.ks, s.ks_l, row * s.ks_sn, 0);
      R.kb = __builtin_amdgcn_raw_buffer_load_b32(s.kb, s.kb_l, row * s.kb_sn, 0);
    } else {
      R.ks = __builtin_amdgcn_raw_buffer_load_b16(s.ks, s.ks_l, row * s.ks_sn, 0);
      R.kb = __builtin_amdgcn_raw_buffer_load_b16(s.kb, s.kb_l, row * s.kb_sn, 0);
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      load_words<Raw::VW>(s.v, s.v_l[e], row * s.v_sn, R.v[e]);
      R.vs[e] = __builtin_amdgcn_raw_buffer_load_b16(s.vs, s.vs_l[e], row * s.vs_sn, 0);
      R.vb[e] = __builtin_amdgcn_raw_buffer_load_b16(s.vb, s.vb_l[e], row * s.vb_sn, 0);
    }
  }

  // Dequantize the thread's piece of a tile into the LDS buffer `buf`: K in
  // T, V in float16 (bfloat16 inputs: the bfloat16 values times vsc = 2^-k).
  static __device__ __forceinline__ void stage(const Raw& R, uint8_t* buf, int tid, float vsc) {
    // K: token tid / KPT, dims [c D/KPT, (c + 1) D/KPT), row-major.
    {
      const int t = tid / kKPT, c = tid % kKPT;
      uint8_t* dst = buf + t * PG::KPitch + c * kQD * 2;
      auto k_scale = [&](int g) { return g ? static_cast<uint32_t>(R.ks >> 16) : static_cast<uint32_t>(R.ks); };
      auto k_bias = [&](int g) { return g ? static_cast<uint32_t>(R.kb >> 16) : static_cast<uint32_t>(R.kb); };
      bool mix = false;
      if constexpr (Tag::kId == QSDPA_BF16) {
        // Wave-uniform: every scale of the wave's slices below kMixScaleMax
        // (NaN and infinities included in the other path).
        bool ok = fabsf(to_f32<Tag>(static_cast<uint16_t>(k_scale(0)))) < kMixScaleMax;
        if constexpr (kKG == 2) ok = ok && fabsf(to_f32<Tag>(static_cast<uint16_t>(k_scale(1)))) < kMixScaleMax;
        mix = __builtin_amdgcn_ballot_w64(!ok) == 0;
      }
      if (mix) {
#pragma unroll
        for (int s = 0; s < kQD / 8; ++s) {
          const int g = kKG == 2 ? (8 * s) / GS : 0;
          const float sf = to_f32<Tag>(static_cast<uint16_t>(k_scale(g)));
          float y[8];
          mix_dequant8<BITS>(R.k + s * (BITS / 4), sf * 0x1p24f, sf * 0x1p20f, to_f32<Tag>(static_cast<uint16_t>(k_bias(g))),
                             y);
          *reinterpret_cast<u4*>(dst + s * 16) = u4{pack_T2<Tag>(y[0], y[1]), pack_T2<Tag>(y[2], y[3]),
                                                    pack_T2<Tag>(y[4], y[5]), pack_T2<Tag>(y[6], y[7])};
        }
      } else {
#pragma unroll
        for (int s = 0; s < kQD / 8; ++s) {
          const int g = kKG == 2 ? (8 * s) / GS : 0;
          const uint32_t sw = k_scale(g), bw = k_bias(g);
          uint32_t a[4];
          dequant_k<Tag, BITS>(R.k + s * (BITS / 4), splat_lo(sw), splat_lo(bw), to_f32<Tag>(static_cast<uint16_t>(sw)),
                               to_f32<Tag>(static_cast<uint16_t>(bw)), a);
          *reinterpret_cast<u4*>(dst + s * 16) = u4{a[0], a[1], a[2], a[3]};
        }
      }
    }
    // V: tokens 2 pr, 2 pr + 1, dims [cv D/VPT, (cv + 1) D/VPT), transposed.
    {
      const int pr = tid % kPairs, cv = tid / kPairs;
      uint8_t* vt = buf + PG::KBytes + vcol(2 * pr) * 2;
      if constexpr (Tag::kId == QSDPA_F16) {
        uint32_t a[2][4];
#pragma unroll
        for (int s = 0; s < kVD / 8; ++s) {
#pragma unroll
          for (int e = 0; e < 2; ++e)
            dequant_k<Tag, BITS>(R.v[e] + s * (BITS / 4), splat_lo(R.vs[e]), splat_lo(R.vb[e]), to_f32<Tag>(R.vs[e]),
                                 to_f32<Tag>(R.vb[e]), a[e]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int d0 = cv * kVD + 8 * s;
            *reinterpret_cast<uint32_t*>(vt + (d0 + pair_dim<Tag, BITS>(i, 0)) * kVPitch) =
                perm(a[1][i], a[0][i], 0x05040100u);
            *reinterpret_cast<uint32_t*>(vt + (d0 + pair_dim<Tag, BITS>(i, 1)) * kVPitch) =
                perm(a[1][i], a[0][i], 0x07060302u);
          }
        }
      } else {
        // bfloat16(fma(s, c, b)) * 2^-k = bfloat16(fma(s 2^-k, c, b 2^-k)),
        // by mix_dequant8: the scan that chose k bounds |s| 2^-k by
        // 2 kVBound / (2^bits - 1), far below kMixScaleMax.  The two tokens'
        // values of a dim are rounded as one pair, which is the V^T word.
        float S[2], S16[2], Bv[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          S[e] = to_f32<Tag>(R.vs[e]) * (vsc * 0x1p24f);
          S16[e] = to_f32<Tag>(R.vs[e]) * (vsc * 0x1p20f);
          Bv[e] = to_f32<Tag>(R.vb[e]) * vsc;
        }
#pragma unroll
        for (int s = 0; s < kVD / 8; ++s) {
          float y[2][8];
#pragma unroll
          for (int e = 0; e < 2; ++e) mix_dequant8<BITS>(R.v[e] + s * (BITS / 4), S[e], S16[e], Bv[e], y[e]);
          const int d0 = cv * kVD + 8 * s;
#pragma unroll
          for (int d = 0; d < 8; ++d)
            *reinterpret_cast<uint32_t*>(vt + (d0 + d) * kVPitch) = bf16x2_to_f16x2(pack_T2<Tag>(y[0][d], y[1][d]));
        }
      }
    }
  }
};

// Parameters beyond the decode's: none; the same MfmaParams (q_len > 1).
// MASK: calls with a mask tensor (an instantiation of their own, so that the
// unmasked kernel carries none of the mask code).
template <typename Tag, int D, int BITS, int GS, bool MASK>
__global__ __launch_bounds__(kPThreads) void prefill_mfma_kernel(MfmaParams p, int groups_per_head) {
  // p.num_splits: key splits per row group (1: the output; more: split-K
  // partials in the decode's layout, merged by merge_kernel).
  using PG = PGeo<D>;
  using P = Prefill<Tag, D, BITS, GS>;
  __shared__ __attribute__((aligned(16))) uint8_t s_buf[4 * PG::BufBytes];
  __shared__ float s_red[kPWaves];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int quad = lane >> 4;
  const int r = lane & 15;

  // XCD-aware work order: workgroups are dispatched to the 8 XCDs round
  // robin, so the work of workgroup id w goes to XCD w % 8 in consecutive
  // runs: the row groups of one (batch, kv head) share one XCD's L2.
  const int total = gridDim.x;
  int w = blockIdx.x;
  if (total % 8 == 0) w = (w % 8) * (total / 8) + w / 8;
  const int S = p.num_splits;
  const int split = w % S;
  w /= S;
  const int grp = w % groups_per_head;
  const int kvh = (w / groups_per_head) % p.Hkv;
  const int b = w / (groups_per_head * p.Hkv);

  const int rows = p.G * p.qL;
  const int v_first = grp * kPGroupRows;
  const int nrows = min(kPGroupRows, rows - v_first);    // real rows of the group
  // Keys: [s0, n_end) of this sequence; causal: the group's last position's limit.
  const int s0 = p.kv_start ? min(max(p.kv_start[b], 0), p.N) : 0;
  const int n_end = p.causal ? min(p.N, max(0, p.N - p.qL + (v_first + nrows - 1) / p.G + 1)) : p.N;
  const int len = max(n_end - s0, 0);
  constexpr int kTile = PG::Tile, NT = PG::NT, NU = PG::NU, KS = PG::KS;
  const int T_all = (len + kTile - 1) / kTile;
  // This split's tiles: [j_base, j_base + T) of the group's T_all.
  const int j_base = static_cast<int>(static_cast<int64_t>(split) * T_all / S);
  const int T = static_cast<int>(static_cast<int64_t>(split + 1) * T_all / S) - j_base;

  // The lane's row: v = v_first + 16 wave + r (clamped to the last real row).
  int n_lane, n_wave;  // the lane's key limit; the wave's smallest
  int64_t mrow;
  uint32_t qt[PG::NM][4];
  {
    const uint8_t* q0 = reinterpret_cast<const uint8_t*>(p.q) +
                        (static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(kvh) * p.G * p.q_sh) * 2;
    const rsrc_t rq = make_rsrc(
        q0, static_cast<uint32_t>(((p.G - 1) * p.q_sh + static_cast<int64_t>(p.qL - 1) * p.q_sq) * 2 + D * 2));
    const int v = v_first + min(16 * wave + r, nrows - 1);
    const int hq = kvh * p.G + v % p.G, iq = v / p.G;
    n_lane = p.causal ? min(n_end, max(0, p.N - p.qL + iq + 1)) : n_end;
    mrow = static_cast<int64_t>(b) * p.m_sb + static_cast<int64_t>(hq) * p.m_sh + static_cast<int64_t>(iq) * p.m_sq;
    const uint32_t off =
        static_cast<uint32_t>((static_cast<int64_t>(v % p.G) * p.q_sh + static_cast<int64_t>(iq) * p.q_sq) * 2);
#pragma unroll
    for (int m = 0; m < PG::NM; ++m) {
      const u4 x = __builtin_amdgcn_raw_buffer_load_b128(rq, off + (32 * m + 8 * quad) * 2, 0, 0);
      uint32_t d0 = x[0], d1 = x[1], d2 = x[2], d3 = x[3];
      if constexpr (Tag::kId == QSDPA_F16 && BITS == 4) {  // the K slice order: dims 0, 4, 1, 5, ...
        qt[m][0] = perm(d2, d0, 0x05040100u);
        qt[m][1] = perm(d2, d0, 0x07060302u);
        qt[m][2] = perm(d3, d1, 0x05040100u);
        qt[m][3] = perm(d3, d1, 0x07060302u);
      } else {
        qt[m][0] = d0; qt[m][1] = d1; qt[m][2] = d2; qt[m][3] = d3;
      }
    }
    int m = n_lane;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) m = min(m, __shfl_xor(m, o));
    n_wave = __builtin_amdgcn_readfirstlane(m);
  }

  // K / V descriptors over rows [s0, N) of this (batch, kv head).
  typename P::Src src;
  {
    const int64_t tok0 = s0;
    const int avail = p.N - s0;
    auto rsrc = [&](const void* base, int64_t sb, int64_t sh, int64_t sn, int esz, int row_bytes, bool present) {
      const uint8_t* p0 = static_cast<const uint8_t*>(base) +
                          (static_cast<int64_t>(b) * sb + static_cast<int64_t>(kvh) * sh + tok0 * sn) * esz;
      const uint32_t bytes =
          (present && avail > 0) ? static_cast<uint32_t>((avail - 1) * sn * esz + row_bytes) : 0u;
      return make_rsrc(p0, bytes);
    };
    constexpr int kRow = D * BITS / 8, kMeta = D / GS * 2;
    src.k = rsrc(p.kp, p.kp_sb, p.kp_sh, p.kp_sn, 4, kRow, true);
    src.v = rsrc(p.vp, p.vp_sb, p.vp_sh, p.vp_sn, 4, kRow, true);
    src.ks = rsrc(p.ks, p.ks_sb, p.ks_sh, p.ks_sn, 2, kMeta, true);
    src.vs = rsrc(p.vs, p.vs_sb, p.vs_sh, p.vs_sn, 2, kMeta, true);
    src.kb = rsrc(p.has_bias ? p.kb : p.ks, p.kb_sb, p.kb_sh, p.kb_sn, 2, kMeta, p.has_bias);
    src.vb = rsrc(p.has_bias ? p.vb : p.vs, p.vb_sb, p.vb_sh, p.vb_sn, 2, kMeta, p.has_bias);
    src.k_sn = static_cast<uint32_t>(p.kp_sn * 4);
    src.v_sn = static_cast<uint32_t>(p.vp_sn * 4);
    src.ks_sn = static_cast<uint32_t>(p.ks_sn * 2);
    src.vs_sn = static_cast<uint32_t>(p.vs_sn * 2);
    src.kb_sn = static_cast<uint32_t>(p.kb_sn * 2);
    src.vb_sn = static_cast<uint32_t>(p.vb_sn * 2);
    P::lanes(src, tid);
  }

  f4 acc[PG::NB];
#pragma unroll
  for (int i = 0; i < PG::NB; ++i) acc[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun = kNegBig, lrun = 0.0f;
  float vsc = 1.0f, osc = 1.0f;  // V scale 2^-k in LDS, output scale 2^k (bfloat16)

  // Without a mask tensor and with a positive scale, the scale goes inside
  // the exponent's fma (max(S) q = max(S q) for q > 0).
  const bool fold = !MASK && p.qscale > 0.0f;
  const float ea = fold ? p.qscale : 1.0f;

  // One tile: S^T from buffer `cur` (first key s0 + tb0), the next tile's
  // dequantization from the register set `Rn` into `nxt` and that set's
  // reload from row `nrow`, the softmax, then P.V from `cur`.
  // two_c: P as two float16 terms (std::true_type) or one.
  auto tile = [&](auto two_c, const uint8_t* cur, uint8_t* nxt, typename P::Raw& Rn, int nrow,
                  int tb0) __attribute__((always_inline)) {
    constexpr bool kTwo = decltype(two_c)::value;
    const int tb = s0 + tb0;
    float mv[4 * NT];
    if constexpr (MASK)  // keys tb + 16 t + 4 quad + i of the lane's mask row
      mask_tile<4 * NT>(p, mrow, tb + 4 * quad, tb + kTile <= p.N, [](int e) { return 16 * (e >> 2) + (e & 3); }, mv);
    // ---- S^T = K Q^T ----
    // The A operands of step m + 1 are read while the MFMAs of step m run
    // (scheduling fences keep that order: left to itself the compiler
    // reuses one register set and waits for each read).
    f4 S4[NT][KS];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int k = 0; k < KS; ++k) S4[t][k] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    u4 ka[2][NT];
    auto read_k = [&](u4* x, int m) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        x[t] = *reinterpret_cast<const u4*>(cur + (16 * t + r) * PG::KPitch + (32 * m + 8 * quad) * 2);
    };
    read_k(ka[0], 0);
#pragma unroll
    for (int m = 0; m < PG::NM; ++m) {
      __builtin_amdgcn_sched_barrier(0);
      if (m + 1 < PG::NM) read_k(ka[(m + 1) & 1], m + 1);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const u4 x = ka[m & 1][t];
        const uint32_t a[4] = {x[0], x[1], x[2], x[3]};
        S4[t][m % KS] = mfma<Tag>(a, qt[m], S4[t][m % KS]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- the next tile: dequantize into the other buffer, reissue its loads
    // (waves 4-7 here, waves 0-3 after the P.V: the two waves of a SIMD then
    // alternate MFMA and VALU phases) ----
    if (wave >= 4) {
      __builtin_amdgcn_s_setprio(1);  // back to 0 at the end of the tile
      P::stage(Rn, nxt, tid, vsc);
      P::load(Rn, src, nrow);
    }
    // ---- scores: lane (quad, r) holds keys tb + 16 t + 4 quad + i of row r ----
    constexpr int NE = 4 * NT;
    float sc[NE];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[4 * t + i] = KS == 2 ? S4[t][0][i] + S4[t][KS - 1][i] : S4[t][0][i];
    if (!fold) {
#pragma unroll
      for (int e = 0; e < NE; ++e) sc[e] *= p.qscale;
      if constexpr (MASK) {
#pragma unroll
        for (int e = 0; e < NE; ++e) sc[e] += mv[e];
      }
    }
    if (tb + kTile > n_wave) {  // keys past a row's limit (causal, or the sequence's end)
      const int lim = n_lane - tb - 4 * quad;  // key tb + 4 quad + k is past the limit when k >= lim
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (16 * t + i >= lim) sc[4 * t + i] = -__builtin_huge_valf();
    }
    float tmax = sc[0];
#pragma unroll
    for (int e = 1; e < NE; ++e) tmax = fmaxf(tmax, sc[e]);
    tmax = max_over_rows(tmax) * ea;
    const bool grow = tmax > mrun + kRescale;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float mnew = grow ? tmax : mrun;
      const float f = fast_exp2(mrun - mnew);
      mrun = mnew;
      lrun *= f;
#pragma unroll
      for (int i = 0; i < PG::NB; ++i) acc[i] *= f;
    }
    const float nm = -mrun;
    float pr[NE];
#pragma unroll
    for (int e = 0; e < NE; ++e) pr[e] = fast_exp2(fmaf(sc[e], ea, nm));
    float s4[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) s4[t] = (pr[4 * t] + pr[4 * t + 1]) + (pr[4 * t + 2] + pr[4 * t + 3]);
    if constexpr (NT == 4) lrun += (s4[0] + s4[1]) + (s4[2] + s4[3]);
    else lrun += s4[0] + s4[1];
    // P^T of half u: k slots 2i, 2i + 1 = tokens tau(quad, 2i), tau(quad, 2i + 1):
    // blocks 2u (i = 0, 1) and 2u + 1 (i = 2, 3).
    uint32_t pb[NU][4], pl[NU][4];
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = 4 * (2 * u + (i >> 1)) + 2 * (i & 1);
        pb[u][i] = pack_T2<F16>(pr[e], pr[e + 1]);
        if constexpr (kTwo)
          pl[u][i] = pack_T2<F16>(pr[e] - unpack_T2_lo<F16>(pb[u][i]), pr[e + 1] - unpack_T2_hi<F16>(pb[u][i]));
      }
    // ---- out^T += V^T P^T (two terms: the hi terms of all dim blocks, then the lo terms) ----
    const uint8_t* vt = cur + PG::KBytes;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      uint32_t a[PG::NB][4];
#pragma unroll
      for (int db = 0; db < PG::NB; ++db) {
        const u4 x = *reinterpret_cast<const u4*>(vt + (16 * db + r) * PG::VPitch + (32 * u + 8 * quad) * 2);
        a[db][0] = x[0]; a[db][1] = x[1]; a[db][2] = x[2]; a[db][3] = x[3];
        acc[db] = mfma<F16>(a[db], pb[u], acc[db]);
      }
      if constexpr (kTwo) {
#pragma unroll
        for (int db = 0; db < PG::NB; ++db) acc[db] = mfma<F16>(a[db], pl[u], acc[db]);
      }
    }
    if (wave < 4) {
      P::stage(Rn, nxt, tid, vsc);
      P::load(Rn, src, nrow);
    } else {
      __builtin_amdgcn_s_setprio(0);
    }
  };

  // ---- the tile pipeline: four LDS buffers, tile j in buffer j % 4,
  // dequantized two tiles ahead from raw registers loaded two tiles before
  // that; one barrier per pair of tiles.  Tile j writes buffer (j + 2) % 4,
  // last read by tile j - 2, which every wave left before the barrier after
  // tile j - 1 or j - 2 (the last odd tile); tile j reads what tile j - 2
  // wrote, before that same barrier.  Between barriers the waves drift by up
  // to two tiles. ----
  typename P::Raw R0, R1;
  auto buf = [&](int j) { return s_buf + (j & 3) * PG::BufBytes; };
  const int oob = len + 2 * kTile;  // rows past every descriptor: the loads read zero
  auto row_of = [&](int j) { return j < T ? (j_base + j) * kTile : oob; };
  // Keys of tile j; past the split's tiles, the sequence end (every score
  // masked: an odd tile count's last pair computes one empty tile).
  auto keys_of = [&](int j) { return j < T ? (j_base + j) * kTile : len; };
  auto run = [&](auto two_c) __attribute__((always_inline)) {
    for (int j = 0; j < T; j += 2) {
      // tiles j, j + 1 in buf(j), buf(j + 1); R0 holds tile j + 2, R1 tile j + 3.
      tile(two_c, buf(j), buf(j + 2), R0, row_of(j + 4), keys_of(j));
      tile(two_c, buf(j + 1), buf(j + 3), R1, row_of(j + 5), keys_of(j + 1));
      __syncthreads();
    }
  };
  if (T > 0) {
    P::load(R0, src, row_of(0));
    P::load(R1, src, row_of(1));
    bool two = false;
    if constexpr (Tag::kId == QSDPA_BF16) {
      // max |V| of this workgroup's keys: a group's values are affine in
      // the code, so its largest magnitude is at code 0 or 2^bits - 1.
      constexpr int NG = D / GS;
      constexpr float kCodeMax = static_cast<float>((1 << BITS) - 1);
      // Eight rows per thread in flight (rows past the range read the
      // range's first row again: no effect on the maximum).
      constexpr int kRows = 8;
      float bound = 0.0f;
      const int t_lo = j_base * kTile, t_hi = min((j_base + T) * kTile, len);
      for (int t0 = t_lo + tid; t0 < t_hi; t0 += kRows * kPThreads) {
        uint16_t sv[kRows][NG], bv[kRows][NG];
#pragma unroll
        for (int u = 0; u < kRows; ++u) {
          const int t = t0 + u * kPThreads < t_hi ? t0 + u * kPThreads : t_lo;
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            sv[u][g] = __builtin_amdgcn_raw_buffer_load_b16(src.vs, static_cast<uint32_t>(t) * src.vs_sn + 2 * g, 0, 0);
            bv[u][g] = __builtin_amdgcn_raw_buffer_load_b16(src.vb, static_cast<uint32_t>(t) * src.vb_sn + 2 * g, 0, 0);
          }
        }
#pragma unroll
        for (int u = 0; u < kRows; ++u)
#pragma unroll
          for (int g = 0; g < NG; ++g) {
            const float s = bf16_bits_to_f32(sv[u][g]), b = bf16_bits_to_f32(bv[u][g]);
            bound = fmaxf(bound, fmaxf(fabsf(b), fabsf(fmaf(s, kCodeMax, b))));
          }
      }
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) bound = fmaxf(bound, shfl_xor_f32(bound, o));
      if (lane == 0) s_red[wave] = bound;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kPWaves; ++i) bound = fmaxf(bound, s_red[i]);
      two = !(bound <= kPVSingle);
      if (bound > kVBound) {
        // k = 1 + floor(log2(bound / kVBound)), so that bound 2^-k < kVBound.
        // A finite bfloat16 bound (< 2^128) needs k <= 113; the clamp keeps
        // k <= 126 when the scan overflowed to Inf, so that 2^-k and 2^k
        // stay normal floats.
        const float x = fminf(bound * (1.0f / kVBound), 0x1p125f);
        const int k = static_cast<int>((__builtin_bit_cast(uint32_t, x) >> 23) & 0xFFu) - 126;
        vsc = __builtin_bit_cast(float, static_cast<uint32_t>(127 - k) << 23);
        osc = __builtin_bit_cast(float, static_cast<uint32_t>(127 + k) << 23);
      }
    }
    P::stage(R0, buf(0), tid, vsc);
    P::load(R0, src, row_of(2));
    P::stage(R1, buf(1), tid, vsc);
    P::load(R1, src, row_of(3));
    __syncthreads();
    if constexpr (Tag::kId == QSDPA_BF16) {
      if (two) run(std::true_type{});
      else run(std::false_type{});
    } else {
      run(std::false_type{});
    }
  }

  // ---- normalise and store: lane (quad, r) holds dims 16 db + 4 quad + i of row r ----
  float l = lrun;
  l += shfl_xor_f32(l, 16);
  l += shfl_xor_f32(l, 32);
  const int vr = 16 * wave + r;
  if (vr >= nrows) return;
  const int v = v_first + vr;
  const int hq = kvh * p.G + v % p.G, iq = v / p.G;
  if (S == 1) {
    const float inv = (l > 0.0f ? 1.0f / l : 0.0f) * osc;
    uint16_t* dst = p.out + static_cast<int64_t>(b) * p.o_sb + static_cast<int64_t>(hq) * p.o_sh +
                    static_cast<int64_t>(iq) * p.o_sq + 4 * quad;
#pragma unroll
    for (int db = 0; db < PG::NB; ++db) {
      const uint32_t lo = pack_T2<Tag>(acc[db][0] * inv, acc[db][1] * inv);
      const uint32_t hi = pack_T2<Tag>(acc[db][2] * inv, acc[db][3] * inv);
      uint16_t* o = dst + 16 * db;  // out rows are only 2-byte aligned in general
      o[0] = static_cast<uint16_t>(lo);
      o[1] = static_cast<uint16_t>(lo >> 16);
      o[2] = static_cast<uint16_t>(hi);
      o[3] = static_cast<uint16_t>(hi >> 16);
    }
  } else {
    // The split's partial of row (b, hq, iq), column `split`, then (m, l):
    // float16 inputs store the normalised row acc / l as float16 (as the
    // decode kernel does); bfloat16 inputs store it as float32, with
    // (m + log2 l, 1) -- the same partial to the merge, whose weight for it
    // is l 2^(m - M) either way, but a sum that stays below max |V| where
    // acc itself would overflow float32 (rows of V near the bfloat16
    // maximum).
    const int64_t slot = ((static_cast<int64_t>(b) * p.Hq + hq) * p.qL + iq) * S + split;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int db = 0; db < PG::NB; ++db) {
      const int d = 16 * db + 4 * quad;
      if constexpr (Tag::kId == QSDPA_F16) {
        typedef uint32_t u2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u2*>(reinterpret_cast<uint16_t*>(p.part_acc) + slot * D + d) =
            u2{pack_T2<Tag>(acc[db][0] * inv, acc[db][1] * inv), pack_T2<Tag>(acc[db][2] * inv, acc[db][3] * inv)};
      } else {
        __builtin_nontemporal_store(acc[db] * (inv * osc), reinterpret_cast<f4*>(p.part_acc + slot * D + d));
      }
    }
    if (quad == 0) {
      const bool norm = Tag::kId != QSDPA_F16 && l > 0.0f;
      p.part_ml[slot * 2] = norm ? mrun + __log2f(l) : mrun;
      p.part_ml[slot * 2 + 1] = norm ? 1.0f : l;
    }
  }
}

template <typename Tag, int D, int BITS, bool MASK>
void launch_prefill_mask(const MfmaParams& p, int gs, int groups, hipStream_t stream, const qsdpa_decode_args* a) {
  const dim3 grid(groups * p.Hkv * p.B * p.num_splits);
  void (*k)(MfmaParams, int) = gs == 32 ? prefill_mfma_kernel<Tag, D, BITS, 32, MASK>
                               : gs == 64 ? prefill_mfma_kernel<Tag, D, BITS, 64, MASK>
                                          : prefill_mfma_kernel<Tag, D, BITS, 128, MASK>;
  if (a->prof_begin || a->prof_end)
    hipExtLaunchKernelGGL(k, grid, dim3(kPThreads), 0, stream, static_cast<hipEvent_t>(a->prof_begin),
                          static_cast<hipEvent_t>(a->prof_end), 0, p, groups);
  else
    hipLaunchKernelGGL(k, grid, dim3(kPThreads), 0, stream, p, groups);
}

template <typename Tag, int D, int BITS>
void launch_prefill_gs(const MfmaParams& p, int gs, int groups, hipStream_t stream, const qsdpa_decode_args* a) {
  if (p.mask) launch_prefill_mask<Tag, D, BITS, true>(p, gs, groups, stream, a);
  else launch_prefill_mask<Tag, D, BITS, false>(p, gs, groups, stream, a);
}

}  // namespace

bool mfma_supports(const qsdpa_decode_args* a);

// Tokens per tile (PGeo<D>::Tile) on the host.
static int prefill_tile(int D) { return D == 256 ? PGeo<256>::Tile : PGeo<128>::Tile; }

// The prefill kernel takes q_len > 1 calls on the MFMA path's layouts whose
// kv heads have at least one full 128-row group (D = 128 or 256); others stay
// on the decode kernel's 16-row blocks (a half-empty group would leave half
// its waves computing padding rows).  K / V rows are read in 16-byte pieces
// (8-byte V pieces at 4-bit), so the packed views must be aligned to the
// pieces.  A thread's K piece (16 dims) always lies in one quantization group.
bool prefill_supports(const qsdpa_decode_args* a) {
  if (a->q_len <= 1 || (a->D != 128 && a->D != 256) || !mfma_supports(a)) return false;
  const int64_t rows = static_cast<int64_t>(a->H_q / a->H_kv) * a->q_len;
  if (rows < kPGroupRows) return false;
  // D = 256 only for calls with at least 2^24 (query row, key) pairs; below
  // that the decode kernel, whose 16-row blocks each stream the kv head, was
  // as fast or faster in all but one case measured (wall time per call,
  // decode kernel against this one with up to 256 key splits: C3's heads at
  // q_len = 8 over 16K /
  // 32K / 64K / 128K keys 23.1-23.2 / 34.0-34.3 / 57-59 / 109-111 against
  // 28.2-28.4 / 34.4 / 47.6-49.2 / 75-84 us, q_len = 16 over 8K / 16K 23.6 /
  // 34.0-34.2 against 29.4-29.7 / 35.8-35.9; C2's heads at q_len = 128 over
  // 32K / 128K 45.8-46.6 / 145-148 against 43.3-43.4 / 101-105, q_len = 256
  // over 8K 31.5 against 35.1-35.2).  A half-filled row group loses: C3's
  // heads at q_len = 4 over 128K 58-59 against 73-75 us.
  if (a->D == 256 && static_cast<int64_t>(a->B) * a->H_q * a->q_len * a->N < (int64_t(1) << 24))
    return false;
  // One row group per kv head at D = 256 goes to the 32-row decode kernel
  // where that takes the call (4-bit codes, no mask tensor, ...): C3's heads
  // at q_len = 8 over 64K / 128K keys 44.3-44.7 / 72.2-77.0 against
  // 47.9-48.0 / 78.1-79.3 us per call here, q_len = 12 over 64K 66.3-72.3
  // against 75.5-80.9.  From two groups on this kernel is as fast or faster
  // (q_len = 16 over 32K / 64K / 128K 46.4-47.3 / 77.9-78.5 / 145.3-147.8
  // there against 48.9-49.3 / 76.8-80.6 / 140.4-143.6 here, q_len = 64 over
  // 128K 486.6-487.7 against 444.6-447.0).
  if (a->D == 256 && rows < 2 * kPGroupRows && rows32_supports(a)) return false;
  const int64_t groups = (rows + kPGroupRows - 1) / kPGroupRows;
  if (groups * a->H_kv * a->B * kMaxPrefillSplits >= (int64_t(1) << 31)) return false;
  const int kq_bytes = a->D / 4 * a->bits / 8, vp_bytes = a->D / 8 * a->bits / 8;
  if (!aligned_view(a->k_packed, std::min(kq_bytes, 16), 4)) return false;
  if (!aligned_view(a->v_packed, std::min(vp_bytes, 16), 4)) return false;
  static_assert(128 / PGeo<128>::KPT == 16 && 256 / PGeo<256>::KPT == 16, "K pieces of 16 dims");
  // Row byte offsets up to 4 tiles past the last key stay within 32 bits.
  const int64_t max_sn = std::max({a->k_packed.stride_n * 4, a->v_packed.stride_n * 4, a->k_scales.stride_n * 2,
                                   a->v_scales.stride_n * 2, a->k_biases.stride_n * 2, a->v_biases.stride_n * 2});
  if (max_sn < 0 || max_sn * (static_cast<int64_t>(a->N) + 4 * prefill_tile(a->D)) >= (int64_t(1) << 31))
    return false;
  return true;
}

// Key splits of the prefill kernel: as many workgroups as CUs, rounded down
// (one workgroup fits a CU, and a few past the CU count run as a second
// round), each split at least 4 tiles (an explicit num_splits > 0 is kept,
// up to the same bounds).  At the C5 chunk (256 row groups) one split; with
// q_len = 128 (64 groups) 4 splits: 38 against 126 us in one.  (At D = 256,
// 8 tiles -- the same 256 keys -- made C3's heads at q_len = 16, N = 4096
// 25.9 instead of 21.3 us.)
int prefill_num_splits(const qsdpa_decode_args* a, int cus) {
  const int64_t rows = static_cast<int64_t>(a->H_q / a->H_kv) * a->q_len;
  const int64_t grid = (rows + kPGroupRows - 1) / kPGroupRows * a->H_kv * a->B;
  const int tile = prefill_tile(a->D);
  const int64_t tiles = (static_cast<int64_t>(a->N) + tile - 1) / tile;
  int64_t s = a->num_splits > 0 ? a->num_splits : cus / grid;  // one round of workgroups
  s = std::min<int64_t>(s, std::max<int64_t>(1, tiles / 4));
  s = std::min<int64_t>(s, kMaxPrefillSplits);
  return static_cast<int>(std::max<int64_t>(s, 1));
}

int launch_prefill_mfma(const qsdpa_decode_args* a, int splits, float* part_acc, float* part_ml,
                        hipStream_t stream) {
  MfmaParams p = mfma_params(a, splits, part_acc, part_ml);
  const int groups = (p.G * p.qL + kPGroupRows - 1) / kPGroupRows;
  const bool f16 = a->dtype == QSDPA_F16;
  auto bits = [&](auto tag) {
    using Tag = decltype(tag);
    if (a->D == 256) {
      if (a->bits == 4) launch_prefill_gs<Tag, 256, 4>(p, a->group_size, groups, stream, a);
      else launch_prefill_gs<Tag, 256, 8>(p, a->group_size, groups, stream, a);
    } else {
      if (a->bits == 4) launch_prefill_gs<Tag, 128, 4>(p, a->group_size, groups, stream, a);
      else launch_prefill_gs<Tag, 128, 8>(p, a->group_size, groups, stream, a);
    }
  };
  if (f16) bits(F16{});
  else bits(BF16{});
  return check_launch("prefill_mfma");
}

}  // namespace qsdpa

