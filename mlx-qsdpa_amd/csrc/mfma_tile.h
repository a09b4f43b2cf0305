// Per-tile building blocks of the matrix-core decode kernel
// (decode_mfma.hip): tile geometry, the register layout of one 32-token K / V
// tile, its QK / online softmax / PV step on v_mfma_f32_16x16x32_{f16,bf16}
// tiles, and the cross-wave merge of a workgroup's rows.  The MFMA operand
// layouts are described at the top of decode_mfma.hip.
#pragma once

#include "mfma_common.h"

namespace qsdpa {
namespace {
// Cache policy of the K / V / scale / bias loads (the aux operand of the
// buffer loads): non-temporal, as each row is read once per step; streaming
// it past the caches keeps the split-K partials and Q resident (C3 25.7
// against 26.4 us per step, C5 13.2 against 13.7).  Not where a lane reads
// 64 contiguous bytes of a K row in four pieces (D = 256, 8-bit: C2 36.6
// against 31.5 us with it).
template <int D, int BITS>
constexpr int load_policy() {
  return D == 256 && BITS == 8 ? 0 : 2;
}

// Geometry of one (D, BITS, GS) instantiation.
template <int D, int BITS, int GS>
struct Geo {
  static constexpr int NM = D / 32;             // QK MFMAs per 16-token half
  static constexpr int NB = D / 16;             // PV MFMAs (dims per lane row)
  static constexpr int QD = D / 4;              // K dims per lane (quarter row)
  static constexpr int KW = QD * BITS / 32;     // K words per lane per half
  static constexpr int WPS = BITS / 4;          // words per 8-dim slice
  static constexpr int KG = QD >= GS ? QD / GS : 1;  // groups per K quarter (1 or 2)
  static constexpr int VW = NB * BITS / 32;     // V words per lane per token
  static constexpr int RW = D * BITS / 32;      // words per row
  static constexpr int NG = D / GS;             // groups (scales) per row
  static constexpr int ND = NG >= 2 ? NG / 2 : 1;  // 32-bit meta words per row
  // D = 256 4-bit: 32-byte K quarters of 128-byte rows.  Each 16-byte K
  // load covers 8 whole rows (lanes r and r + 8 read the two halves of row
  // r & 7 of its 8), and a DPP exchange between lanes r and r ^ 8 gives
  // every lane its own row's quarter (load_k, qk_half; in the kernels
  // without a mask tensor: with a bool or additive mask, C3 measured the
  // same either way, 24.8-25.0 us kernel p50).  Loaded as quarters, every K
  // line was requested
  // by two loads of half a line.  Measured at C3 (three rounds on one box):
  // kernel p50 21.0-21.3 against 21.7-22.4 us, 24.3-24.5 against 24.7-25.5
  // us per step; C5 (D = 128 8-bit, the same quarter shape) was 0.1 us
  // slower with it and keeps the quarter loads.
  static constexpr bool PairK = D == 256 && BITS == 4;
  static_assert(KG == 1 || KG == 2, "groups per quarter");
  static_assert(VW >= 1, "V piece");
};

// Registers of one tile: K (A layout, two halves), V (transposed pieces of the
// lane's 8 tokens) and their scales / biases.
template <int D, int BITS, int GS>
struct TileRegs {
  using G = Geo<D, BITS, GS>;
  uint32_t kw[2][G::KW];
  uint32_t ks[2];            // KG == 2: both groups (16-bit each); else low half
  uint32_t kb[2];            // the K bias word(s) of the lane's group(s), as ks
  uint32_t vw[8][G::VW];
  uint32_t vs[2], vb[2];     // V scale / bias row words (A layout, per half)
};

// Per-lane constant byte offsets of a lane's loads relative to the tile's
// first row: its row within the tile plus its piece of that row.
struct LaneOffsets {
  uint32_t k_r, ks_r, kb_r, v_r, vs_r, vb_r;
};

// Buffer descriptors of one workgroup's rows and the token strides in bytes.
struct Rsrcs {
  rsrc_t k, ks, kb, v, vs, vb;
  uint32_t k_sn, ks_sn, kb_sn, v_sn, vs_sn, vb_sn;
};

// Words at the lane's byte offset `voff` plus the uniform `soff` (the buffer
// instruction's scalar offset, which the range check includes: a uniform row
// offset costs no VALU add).
template <int WORDS, int AUX>
__device__ __forceinline__ void buffer_words(rsrc_t rs, uint32_t voff, uint32_t soff, uint32_t* w) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  if constexpr (WORDS % 4 == 0) {
#pragma unroll
    for (int i = 0; i < WORDS / 4; ++i) {
      const u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + 16 * i, soff, AUX);
      w[4 * i] = v[0]; w[4 * i + 1] = v[1]; w[4 * i + 2] = v[2]; w[4 * i + 3] = v[3];
    }
  } else if constexpr (WORDS == 2) {
    const u2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, AUX);
    w[0] = v[0]; w[1] = v[1];
  } else {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, AUX);
  }
}

// Where a lane finds the V scale / bias of its group for its tokens:
// ds_bpermute byte addresses of the source lanes for token slots j & 3, the
// v_perm_b32 selector taking the right 16-bit half of two words, and the
// shift that moves that half to the top (bf16 -> f32).
struct VMetaLane {
  int src[4];
  uint32_t sel;
  uint32_t shift;
};

// Buffer descriptors over rows [s0, s0 + len) of (batch b, kv head kvh) of
// the six K / V tensors, and their token strides in bytes.  Rows past them
// (and every row of an absent bias) read as zero.
template <int D, int BITS, int GS>
__device__ __forceinline__ Rsrcs tile_rsrcs(const MfmaParams& p, int b, int kvh, int s0, int len) {
  using G = Geo<D, BITS, GS>;
  const int64_t tok0 = s0;
  auto rsrc = [&](const void* base, int64_t sb, int64_t sh, int64_t sn, int esz, int row_bytes, bool present) {
    const uint8_t* p0 = static_cast<const uint8_t*>(base) +
                        (static_cast<int64_t>(b) * sb + static_cast<int64_t>(kvh) * sh + tok0 * sn) * esz;
    const uint32_t bytes = (present && len > 0) ? static_cast<uint32_t>((len - 1) * sn * esz + row_bytes) : 0u;
    return make_rsrc(p0, bytes);
  };
  constexpr int kRow = D * BITS / 8;
  constexpr int kMeta = G::NG * 2;
  Rsrcs rs;
  rs.k = rsrc(p.kp, p.kp_sb, p.kp_sh, p.kp_sn, 4, kRow, true);
  rs.v = rsrc(p.vp, p.vp_sb, p.vp_sh, p.vp_sn, 4, kRow, true);
  rs.ks = rsrc(p.ks, p.ks_sb, p.ks_sh, p.ks_sn, 2, kMeta, true);
  rs.vs = rsrc(p.vs, p.vs_sb, p.vs_sh, p.vs_sn, 2, kMeta, true);
  rs.kb = rsrc(p.has_bias ? p.kb : p.ks, p.kb_sb, p.kb_sh, p.kb_sn, 2, kMeta, p.has_bias);
  rs.vb = rsrc(p.has_bias ? p.vb : p.vs, p.vb_sb, p.vb_sh, p.vb_sn, 2, kMeta, p.has_bias);
  rs.k_sn = static_cast<uint32_t>(p.kp_sn * 4);
  rs.v_sn = static_cast<uint32_t>(p.vp_sn * 4);
  rs.ks_sn = static_cast<uint32_t>(p.ks_sn * 2);
  rs.vs_sn = static_cast<uint32_t>(p.vs_sn * 2);
  rs.kb_sn = static_cast<uint32_t>(p.kb_sn * 2);
  rs.vb_sn = static_cast<uint32_t>(p.vb_sn * 2);
  return rs;
}

// Lane (quad, r)'s byte offsets of its loads within a tile (PK: whole-row K
// loads, Geo::PairK) and where it gathers its tokens' V scales / biases.
template <int D, int BITS, int GS, bool PK>
__device__ __forceinline__ void lane_setup(const Rsrcs& rs, int quad, int r, LaneOffsets& L, VMetaLane& vm) {
  using G = Geo<D, BITS, GS>;
  const int kg0 = (quad * G::QD) / GS;  // first group of the lane's K quarter
  const int gv = (r * G::NB) / GS;      // group of the lane's V dims
  const int vword = G::NG >= 2 ? quad % G::ND : 0;  // V meta word this lane loads
  L.k_r = PK ? quad * G::KW * 4 + (r >> 3) * 16 + (r & 7) * rs.k_sn : quad * G::KW * 4 + r * rs.k_sn;
  L.ks_r = kg0 * 2 + r * rs.ks_sn;
  L.kb_r = kg0 * 2 + r * rs.kb_sn;
  L.v_r = r * G::VW * 4 + 4 * quad * rs.v_sn;
  L.vs_r = vword * 4 + r * rs.vs_sn;
  L.vb_r = vword * 4 + r * rs.vb_sn;
  // Opaque to the optimizer: seeing r * stride inside, it folds a load's
  // uniform row * stride + L into a per-lane (row + r) * stride, one
  // quarter-rate v_mul_lo_u32 per load and tile.
  asm("" : "+v"(L.k_r), "+v"(L.ks_r), "+v"(L.kb_r), "+v"(L.v_r), "+v"(L.vs_r), "+v"(L.vb_r));
  // Token tau(quad, j) of a half sits in row 4*quad + (j & 3); its meta word
  // gv / 2 was loaded by quad gv / 2.
  const int dw = G::NG >= 2 ? gv / 2 : 0;
  const int half = G::NG >= 2 ? gv % 2 : 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) vm.src[k] = (16 * dw + 4 * quad + k) * 4;
  vm.sel = half ? 0x07060302u : 0x05040100u;
  vm.shift = half ? 0u : 16u;
}

template <typename Tag, int D, int BITS, int GS>
struct Kernel {
  static constexpr int kAux = load_policy<D, BITS>();
  using G = Geo<D, BITS, GS>;
  using Regs = TileRegs<D, BITS, GS>;
  // Every K / V element is dequantized as mx.dequantize rounds it, T(fma(
  // scale, code, bias)): float16 builds the code as an exact half (the
  // 1024 + code bit trick, minus 1024) and uses one v_pk_fma_f16 per pair.
  // (Rounding scale * code first and adding the bias afterwards saves an
  // op per pair but is off by up to half an ulp of |scale * code|, which
  // outruns the parity tolerance where a few keys carry a row.)

  // Token of slot j (0..7) of quad q within a 32-token tile (the S^T C layout).
  static __device__ __forceinline__ int tau(int q, int j) { return 16 * (j >> 2) + 4 * q + (j & 3); }

  // Issue the K (load_k) or V (load_v) loads of the tile whose first token is
  // `rel0` rows past the sequence's first key.  Rows past the end fall
  // outside the buffer descriptors and read as zero (only the sequence's
  // last tile has such rows; their scores are set to -inf).
  // PK: the PairK load (and, in qk_half, exchange); G::PairK && !MASK.
  template <bool PK>
  static __device__ __forceinline__ void load_k(Regs& R, const Rsrcs& rs, const LaneOffsets& L, int rel0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t row = static_cast<uint32_t>(rel0 + 16 * u);
      if constexpr (PK) {
        // Rows row + (r & 7) and row + 8 + (r & 7), 16-byte piece 2 quad + (r >> 3).
        buffer_words<4, kAux>(rs.k, L.k_r, row * rs.k_sn, R.kw[u]);
        buffer_words<4, kAux>(rs.k, L.k_r, (row + 8) * rs.k_sn, R.kw[u] + 4);
      } else {
        buffer_words<G::KW, kAux>(rs.k, L.k_r, row * rs.k_sn, R.kw[u]);
      }
      if constexpr (G::KG == 2)
        R.ks[u] = __builtin_amdgcn_raw_buffer_load_b32(rs.ks, L.ks_r, row * rs.ks_sn, kAux);
      else
        R.ks[u] = __builtin_amdgcn_raw_buffer_load_b16(rs.ks, L.ks_r, row * rs.ks_sn, kAux);
      if constexpr (G::KG == 2) {
        R.kb[u] = __builtin_amdgcn_raw_buffer_load_b32(rs.kb, L.kb_r, row * rs.kb_sn, kAux);
      } else {
        R.kb[u] = __builtin_amdgcn_raw_buffer_load_b16(rs.kb, L.kb_r, row * rs.kb_sn, kAux);
      }
    }
  }

  static __device__ __forceinline__ void load_v(Regs& R, const Rsrcs& rs, const LaneOffsets& L, int rel0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t row = static_cast<uint32_t>(rel0 + 16 * u);
      if constexpr (G::NG >= 2) {
        R.vs[u] = __builtin_amdgcn_raw_buffer_load_b32(rs.vs, L.vs_r, row * rs.vs_sn, kAux);
        R.vb[u] = __builtin_amdgcn_raw_buffer_load_b32(rs.vb, L.vb_r, row * rs.vb_sn, kAux);
      } else {
        R.vs[u] = __builtin_amdgcn_raw_buffer_load_b16(rs.vs, L.vs_r, row * rs.vs_sn, kAux);
        R.vb[u] = __builtin_amdgcn_raw_buffer_load_b16(rs.vb, L.vb_r, row * rs.vb_sn, kAux);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t row = static_cast<uint32_t>(rel0 + 16 * (j >> 2) + (j & 3));
      buffer_words<G::VW, kAux>(rs.v, L.v_r, row * rs.v_sn, R.vw[j]);
    }
  }

  // S^T for one 16-token half u: K dequantized into the A operand (scale *
  // code + bias with the lane's group scales / biases), Q^T as B.
  template <bool PK>
  static __device__ __forceinline__ f4 qk_half(const Regs& R, int u, const uint32_t (&qt)[G::NM][4]) {
    uint32_t s2[2], b2[2];
    float sf[2], bf[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const uint32_t sw = (G::KG == 2 && g == 1) ? (R.ks[u] >> 16) : R.ks[u];
      const uint32_t bw = (G::KG == 2 && g == 1) ? (R.kb[u] >> 16) : R.kb[u];
      s2[g] = splat_lo(sw);
      sf[g] = to_f32<Tag>(static_cast<uint16_t>(sw));
      b2[g] = splat_lo(bw);
      bf[g] = to_f32<Tag>(static_cast<uint16_t>(bw));
    }
    // PairK: lane r < 8 holds piece 2 quad of row r (words 0-3) and of row
    // r + 8 (4-7), lane r >= 8 piece 2 quad + 1 of rows r - 8 and r; one
    // exchange with lane r ^ 8 (DPP row_ror:8) leaves both pieces of row r.
    uint32_t kw[G::KW];
    if constexpr (PK) {
      const bool lo8 = (threadIdx.x & 8) == 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t a0 = R.kw[u][i], a1 = R.kw[u][4 + i];
        const uint32_t x0 = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(a0), 0x128, 0xF, 0xF, false));
        const uint32_t x1 = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(a1), 0x128, 0xF, 0xF, false));
        kw[i] = lo8 ? a0 : x1;
        kw[4 + i] = lo8 ? x0 : a1;
      }
    } else {
#pragma unroll
      for (int i = 0; i < G::KW; ++i) kw[i] = R.kw[u][i];
    }
    f4 S = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < G::NM; ++m) {
      const int g = (G::KG == 2 && m >= G::NM / 2) ? 1 : 0;
      uint32_t a[4];
      dequant_k<Tag, BITS>(kw + m * G::WPS, s2[g], b2[g], sf[g], bf[g], a);
      S = mfma<Tag>(a, qt[m], S);
    }
    return S;
  }

  // out^T += V^T P^T: MFMA nb takes dim r*NB + nb of the lane's 8 tokens.
  // sv2 / bv2: V scale / bias pairs of tokens (2i, 2i+1) of the lane's group.
  template <typename IV>
  static __device__ __forceinline__ void pv_f16(Regs& R, const uint32_t (&sv2)[4], const uint32_t (&bv2)[4],
                                                const uint32_t (&pb)[4], f4 (&acc)[G::NB], IV&& issue_v) {
    if constexpr (BITS == 4) {
      // X: nibbles 0-3 of tokens (2i, 2i+1), Y: nibbles 4-7.
      uint32_t X[4][G::VW], Y[4][G::VW];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < G::VW; ++w) {
          X[i][w] = perm(R.vw[2 * i + 1][w], R.vw[2 * i][w], 0x05040100u);
          Y[i][w] = perm(R.vw[2 * i + 1][w], R.vw[2 * i][w], 0x07060302u);
        }
      issue_v(R);
#pragma unroll
      for (int nb = 0; nb < G::NB; ++nb) {
        const int w = nb >> 3, k = nb & 7;
        uint32_t a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t src = k < 4 ? X[i][w] : Y[i][w];
          a[i] = f16x2_fma(nib_codes(src, src >> 8, k & 3), sv2[i], bv2[i]);
        }
        acc[nb] = mfma<Tag>(a, pb, acc[nb]);
      }
    } else {
      // Z0: bytes 0-1 of tokens (2i, 2i+1) interleaved, Z1: bytes 2-3.
      uint32_t Z[4][G::VW][2];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < G::VW; ++w) {
          Z[i][w][0] = perm(R.vw[2 * i + 1][w], R.vw[2 * i][w], 0x05010400u);
          Z[i][w][1] = perm(R.vw[2 * i + 1][w], R.vw[2 * i][w], 0x07030602u);
        }
      issue_v(R);
#pragma unroll
      for (int nb = 0; nb < G::NB; ++nb) {
        const int w = nb >> 2, k = nb & 3;
        uint32_t a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t t = perm(kMagic8, Z[i][w][k >> 1], (k & 1) ? kSelB23 : kSelB01);
          a[i] = f16x2_fma(f16x2_sub1024(t), sv2[i], bv2[i]);
        }
        acc[nb] = mfma<Tag>(a, pb, acc[nb]);
      }
    }
  }

  // One tile: QK, online softmax, PV.  Keys t of the tile (first key tb)
  // outside [n0, n1) are masked (the sequence's first and last tiles may be
  // partial); MASK: a mask tensor adds its values (a kernel of its own, so
  // the unmasked kernel carries none of its code).  The next tile's K loads are issued (issue_k) as soon as this
  // tile's K has been consumed, and its V loads (issue_v) once V is in the PV
  // operands' pre-permuted form, so one register set suffices.
  template <bool MASK, typename IK, typename IV>
  static __device__ __forceinline__ void compute_tile(Regs& R, const MfmaParams& p, const uint32_t (&qt)[G::NM][4],
                                                      f4 (&acc)[G::NB], float& mrun, float& lrun, int tb, int n0,
                                                      int n1, int quad, int64_t mrow, const VMetaLane& vm,
                                                      IK&& issue_k, IV&& issue_v) {
    // Mask values of the lane's 8 keys, loaded before the next tile's K
    // loads are issued, so waiting for them does not wait for those.
    float mv[8];
    if constexpr (MASK)
      mask_tile<8>(p, mrow, tb + 4 * quad, tb + kTile <= p.N, [](int j) { return tau(0, j); }, mv);
    // ---- S^T = K Q^T (Q^T operand m: 16 B per lane, in registers) ----
    f4 S[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) S[u] = qk_half<G::PairK && !MASK>(R, u, qt);
    issue_k(R);

    // ---- scores of (the lane's row, tokens tau(quad, j)), online softmax ----
    // n1: this lane's end of keys (the sequence's, or its causal limit).
    // Without a mask tensor and with a positive scale, the scale goes into
    // the exponent's fma (max(S) q = max(S q) for q > 0): no multiply per
    // score.
    const bool fold = !MASK && p.qscale > 0.0f;
    const float ea = fold ? p.qscale : 1.0f;
    float sc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sc[j] = S[j >> 2][j & 3];
    if (!fold) {
#pragma unroll
      for (int j = 0; j < 8; ++j) sc[j] *= p.qscale;
    }
    if constexpr (MASK) {
#pragma unroll
      for (int j = 0; j < 8; ++j) sc[j] += mv[j];
    }
    if (__builtin_expect(tb + kTile > n1 || tb < n0, 0)) {  // a partial tile
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = tb + tau(quad, j);
        if (t >= n1 || t < n0) sc[j] = -__builtin_huge_valf();
      }
    }
    const float tmax = max_over_rows(max8(sc)) * ea;
    const bool grow = tmax > mrun + kRescale;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float mnew = grow ? tmax : mrun;
      const float f = fast_exp2(mrun - mnew);
      mrun = mnew;
      lrun *= f;
#pragma unroll
      for (int i = 0; i < G::NB; ++i) acc[i] *= f;
    }
    float pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(fmaf(sc[j], ea, -mrun));
    lrun += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));

    // ---- P^T operand: k slot 2i, 2i+1 = tokens tau(quad, 2i), tau(quad, 2i+1) ----
    uint32_t pb[4], pb_lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = pack_T2<Tag>(pr[2 * i], pr[2 * i + 1]);
    if constexpr (Tag::kId == QSDPA_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pb_lo[i] = pack_T2<Tag>(pr[2 * i] - unpack_T2_lo<Tag>(pb[i]),
                                pr[2 * i + 1] - unpack_T2_hi<Tag>(pb[i]));
    }

    // ---- out^T += V^T P^T: MFMA nb takes dim r*NB + nb of the lane's tokens ----
    // V scale / bias words of the lane's 8 tokens, gathered from the lanes
    // that loaded those rows (A layout: token 16u + r, word quad % ND).
    uint32_t dS[8], dB[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      dS[j] = __builtin_amdgcn_ds_bpermute(vm.src[j & 3], static_cast<int>(R.vs[j >> 2]));
      dB[j] = __builtin_amdgcn_ds_bpermute(vm.src[j & 3], static_cast<int>(R.vb[j >> 2]));
    }
    if constexpr (Tag::kId == QSDPA_F16) {
      uint32_t sv2[4], bv2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv2[i] = perm(dS[2 * i + 1], dS[2 * i], vm.sel);
        bv2[i] = perm(dB[2 * i + 1], dB[2 * i], vm.sel);
      }
      pv_f16(R, sv2, bv2, pb, acc, issue_v);
    } else {
      float svf[8], bvf[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        svf[j] = __builtin_bit_cast(float, (dS[j] << vm.shift) & 0xFFFF0000u);
        bvf[j] = __builtin_bit_cast(float, (dB[j] << vm.shift) & 0xFFFF0000u);
      }
      uint32_t lo[8][G::VW], hi[8][G::VW];
      if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int w = 0; w < G::VW; ++w) {
            lo[j][w] = R.vw[j][w] & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6 as bytes
            hi[j][w] = (R.vw[j][w] >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
          }
      }
#pragma unroll
      for (int nb = 0; nb < G::NB; ++nb) {
        uint32_t a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float c[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int j = 2 * i + e;
            if constexpr (BITS == 4) {
              const int w = nb >> 3, k = nb & 7;
              const uint32_t src = (k & 1) ? hi[j][w] : lo[j][w];
              c[e] = static_cast<float>((src >> (8 * (k >> 1))) & 0xFFu);
            } else {
              const int w = nb >> 2, k = nb & 3;
              c[e] = static_cast<float>((R.vw[j][w] >> (8 * k)) & 0xFFu);
            }
            c[e] = fmaf(svf[j], c[e], bvf[j]);
          }
          a[i] = pack_T2<Tag>(c[0], c[1]);
        }
        acc[nb] = mfma<Tag>(a, pb, acc[nb]);
        acc[nb] = mfma<Tag>(a, pb_lo, acc[nb]);
      }
      issue_v(R);
    }
  }

  // ---- Two 16-row halves per wave (decode_rows32.hip) ----
  // One dequantized K / V tile feeds the MFMAs of both halves of a 32-row
  // block.  Q^T does not fit in registers beside two accumulator sets, so
  // each QK step reads its B operands from the staged Q rows in LDS: qlds is
  // the lane's 16-byte piece of its row in half 0 (step m at +16 m), half 1
  // lies half_bytes further.

  // S^T of both token halves u (S[u][k]) for both row halves k.  Each QK
  // step's two Q^T pieces are read once, one step ahead (the scheduling
  // barrier keeps the compiler from hoisting every step's LDS reads, which
  // ran the kernel out of registers), and feed four MFMAs.
  static __device__ __forceinline__ void qk_tile2(const Regs& R, const uint8_t* qlds, int half_bytes,
                                                  f4 (&S)[2][2]) {
    uint32_t s2[2][2], b2[2][2];
    float sf[2][2], bf[2][2];
    uint32_t kw[2][G::KW];
    const bool lo8 = (threadIdx.x & 8) == 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const uint32_t sw = (G::KG == 2 && g == 1) ? (R.ks[u] >> 16) : R.ks[u];
        const uint32_t bw = (G::KG == 2 && g == 1) ? (R.kb[u] >> 16) : R.kb[u];
        s2[u][g] = splat_lo(sw);
        sf[u][g] = to_f32<Tag>(static_cast<uint16_t>(sw));
        b2[u][g] = splat_lo(bw);
        bf[u][g] = to_f32<Tag>(static_cast<uint16_t>(bw));
      }
      if constexpr (G::PairK) {
        // The whole-row exchange of qk_half (lanes r and r ^ 8).
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t a0 = R.kw[u][i], a1 = R.kw[u][4 + i];
          const uint32_t x0 = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(a0), 0x128, 0xF, 0xF, false));
          const uint32_t x1 = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(a1), 0x128, 0xF, 0xF, false));
          kw[u][i] = lo8 ? a0 : x1;
          kw[u][4 + i] = lo8 ? x0 : a1;
        }
      } else {
#pragma unroll
        for (int i = 0; i < G::KW; ++i) kw[u][i] = R.kw[u][i];
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) S[u][k] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    u4 q0 = *reinterpret_cast<const u4*>(qlds);
    u4 q1 = *reinterpret_cast<const u4*>(qlds + half_bytes);
#pragma unroll
    for (int m = 0; m < G::NM; ++m) {
      u4 n0 = q0, n1 = q1;
      if (m + 1 < G::NM) {
        n0 = *reinterpret_cast<const u4*>(qlds + 16 * (m + 1));
        n1 = *reinterpret_cast<const u4*>(qlds + half_bytes + 16 * (m + 1));
      }
      __builtin_amdgcn_sched_barrier(0x67F);  // everything but LDS reads may cross
      const uint32_t b0[4] = {q0[0], q0[1], q0[2], q0[3]};
      const uint32_t b1[4] = {q1[0], q1[1], q1[2], q1[3]};
      const int g = (G::KG == 2 && m >= G::NM / 2) ? 1 : 0;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        uint32_t a[4];
        dequant_k<Tag, BITS>(kw[u] + m * G::WPS, s2[u][g], b2[u][g], sf[u][g], bf[u][g], a);
        S[u][0] = mfma<Tag>(a, b0, S[u][0]);
        S[u][1] = mfma<Tag>(a, b1, S[u][1]);
      }
      q0 = n0;
      q1 = n1;
    }
  }

  // Online softmax of one half's scores (sc: the lane's 8 tokens, scaled
  // unless `fold`) into its running (m, l) and P^T operands (pb_lo: the
  // bfloat16 low terms).
  static __device__ __forceinline__ void softmax_half(float (&sc)[8], float ea, f4 (&acc)[G::NB], float& mrun,
                                                      float& lrun, uint32_t (&pb)[4], uint32_t (&pb_lo)[4]) {
    const float tmax = max_over_rows(max8(sc)) * ea;
    const bool grow = tmax > mrun + kRescale;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float mnew = grow ? tmax : mrun;
      const float f = fast_exp2(mrun - mnew);
      mrun = mnew;
      lrun *= f;
#pragma unroll
      for (int i = 0; i < G::NB; ++i) acc[i] *= f;
    }
    float pr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(fmaf(sc[j], ea, -mrun));
    lrun += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = pack_T2<Tag>(pr[2 * i], pr[2 * i + 1]);
    if constexpr (Tag::kId == QSDPA_BF16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pb_lo[i] = pack_T2<Tag>(pr[2 * i] - unpack_T2_lo<Tag>(pb[i]), pr[2 * i + 1] - unpack_T2_hi<Tag>(pb[i]));
    }
  }

  // One tile for a 32-row block: QK of both halves, their online softmax,
  // PV of both halves from one dequantized V^T.  n1[k]: the lane's end of
  // keys in half k.  MASK: a mask tensor's values for the lane's rows mrow[k]
  // (loaded before the next tile's K loads, as compute_tile does).
  template <bool MASK, typename IK, typename IV>
  static __device__ __forceinline__ void compute_tile2(Regs& R, const MfmaParams& p, const uint8_t* qlds,
                                                       int half_bytes, f4 (&acc)[2][G::NB], float (&mrun)[2],
                                                       float (&lrun)[2], int tb, int n0, const int (&n1)[2], int quad,
                                                       const int64_t (&mrow)[2], const VMetaLane& vm, IK&& issue_k,
                                                       IV&& issue_v) {
    float mv[2][8];
    if constexpr (MASK) {
#pragma unroll
      for (int k = 0; k < 2; ++k)
        mask_tile<8>(p, mrow[k], tb + 4 * quad, tb + kTile <= p.N, [](int j) { return tau(0, j); }, mv[k]);
    }
    f4 S[2][2];  // [token half u][row half k]
    qk_tile2(R, qlds, half_bytes, S);
    issue_k(R);

    const bool fold = !MASK && p.qscale > 0.0f;
    const float ea = fold ? p.qscale : 1.0f;
    const bool partial = tb + kTile > min(n1[0], n1[1]) || tb < n0;
    uint32_t pb[2][4], pb_lo[2][4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      float sc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) sc[j] = S[j >> 2][k][j & 3];
      if (!fold) {
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] *= p.qscale;
      }
      if constexpr (MASK) {
#pragma unroll
        for (int j = 0; j < 8; ++j) sc[j] += mv[k][j];
      }
      if (__builtin_expect(partial, 0)) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int t = tb + tau(quad, j);
          if (t >= n1[k] || t < n0) sc[j] = -__builtin_huge_valf();
        }
      }
      softmax_half(sc, ea, acc[k], mrun[k], lrun[k], pb[k], pb_lo[k]);
    }

    // V scale / bias words of the lane's 8 tokens (as in compute_tile).
    uint32_t dS[8], dB[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      dS[j] = __builtin_amdgcn_ds_bpermute(vm.src[j & 3], static_cast<int>(R.vs[j >> 2]));
      dB[j] = __builtin_amdgcn_ds_bpermute(vm.src[j & 3], static_cast<int>(R.vb[j >> 2]));
    }
    if constexpr (Tag::kId == QSDPA_F16) {
      uint32_t sv2[4], bv2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv2[i] = perm(dS[2 * i + 1], dS[2 * i], vm.sel);
        bv2[i] = perm(dB[2 * i + 1], dB[2 * i], vm.sel);
      }
      if constexpr (BITS == 4) {
        // X: nibbles 0-3 of tokens (2i, 2i+1), Y: nibbles 4-7 (as pv_f16).
        uint32_t X[4][G::VW], Y[4][G::VW];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int w = 0; w < G::VW; ++w) {
            X[i][w] = perm(R.vw[2 * i + 1][w], R.vw[2 * i][w], 0x05040100u);
            Y[i][w] = perm(R.vw[2 * i + 1][w], R.vw[2 * i][w], 0x07060302u);
          }
        issue_v(R);
#pragma unroll
        for (int nb = 0; nb < G::NB; ++nb) {
          const int w = nb >> 3, k = nb & 7;
          uint32_t a[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t src = k < 4 ? X[i][w] : Y[i][w];
            a[i] = f16x2_fma(nib_codes(src, src >> 8, k & 3), sv2[i], bv2[i]);
          }
          acc[0][nb] = mfma<Tag>(a, pb[0], acc[0][nb]);
          acc[1][nb] = mfma<Tag>(a, pb[1], acc[1][nb]);
        }
      } else {
        // Z0: bytes 0-1 of tokens (2i, 2i+1) interleaved, Z1: bytes 2-3 (as pv_f16).
        uint32_t Z[4][G::VW][2];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int w = 0; w < G::VW; ++w) {
            Z[i][w][0] = perm(R.vw[2 * i + 1][w], R.vw[2 * i][w], 0x05010400u);
            Z[i][w][1] = perm(R.vw[2 * i + 1][w], R.vw[2 * i][w], 0x07030602u);
          }
        issue_v(R);
#pragma unroll
        for (int nb = 0; nb < G::NB; ++nb) {
          const int w = nb >> 2, k = nb & 3;
          uint32_t a[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const uint32_t t = perm(kMagic8, Z[i][w][k >> 1], (k & 1) ? kSelB23 : kSelB01);
            a[i] = f16x2_fma(f16x2_sub1024(t), sv2[i], bv2[i]);
          }
          acc[0][nb] = mfma<Tag>(a, pb[0], acc[0][nb]);
          acc[1][nb] = mfma<Tag>(a, pb[1], acc[1][nb]);
        }
      }
    } else {
      float svf[8], bvf[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        svf[j] = __builtin_bit_cast(float, (dS[j] << vm.shift) & 0xFFFF0000u);
        bvf[j] = __builtin_bit_cast(float, (dB[j] << vm.shift) & 0xFFFF0000u);
      }
      uint32_t lo[8][G::VW], hi[8][G::VW];
      if constexpr (BITS == 4) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int w = 0; w < G::VW; ++w) {
            lo[j][w] = R.vw[j][w] & 0x0F0F0F0Fu;         // nibbles 0, 2, 4, 6 as bytes
            hi[j][w] = (R.vw[j][w] >> 4) & 0x0F0F0F0Fu;  // nibbles 1, 3, 5, 7
          }
      }
#pragma unroll
      for (int nb = 0; nb < G::NB; ++nb) {
        uint32_t a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float c[2];
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int j = 2 * i + e;
            if constexpr (BITS == 4) {
              const int w = nb >> 3, k = nb & 7;
              const uint32_t src = (k & 1) ? hi[j][w] : lo[j][w];
              c[e] = static_cast<float>((src >> (8 * (k >> 1))) & 0xFFu);
            } else {
              const int w = nb >> 2, k = nb & 3;
              c[e] = static_cast<float>((R.vw[j][w] >> (8 * k)) & 0xFFu);
            }
            c[e] = fmaf(svf[j], c[e], bvf[j]);
          }
          a[i] = pack_T2<Tag>(c[0], c[1]);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          acc[h][nb] = mfma<Tag>(a, pb[h], acc[h][nb]);
          acc[h][nb] = mfma<Tag>(a, pb_lo[h], acc[h][nb]);
        }
      }
      issue_v(R);
    }
  }
};

// Cache policy (the aux operand of buffer loads and stores) of the partials
// that workgroups of one launch hand to each other: sc1, coherent across
// the device's XCDs without a write-back of the whole L2 (what the compiler
// emits for relaxed agent-scope atomic loads and stores on gfx950).
constexpr int kCoherent = 16;

// A normalised output row piece: out[b, hh, iq, d .. d + 8) = v / L (0 when
// L = 0: every key of the row was masked or absent).  Output rows are only
// 2-byte aligned in general: stores of 16-bit halves.
template <typename Tag>
__device__ __forceinline__ void store_out8(const MfmaParams& p, int b, int hh, int iq, int d, const float (&v)[8],
                                           float L) {
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  uint32_t pk[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) pk[e] = pack_T2<Tag>(v[2 * e] * inv, v[2 * e + 1] * inv);
  uint16_t* dst = p.out + static_cast<int64_t>(b) * p.o_sb + static_cast<int64_t>(hh) * p.o_sh +
                  static_cast<int64_t>(iq) * p.o_sq + d;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    dst[2 * e] = static_cast<uint16_t>(pk[e]);
    dst[2 * e + 1] = static_cast<uint16_t>(pk[e] >> 16);
  }
}

// The partial rows of one block (batch b, kv head kvh) for the split merge
// inside the launch: rows (head, position) of the kv head, `cols` slots
// each, addressed through buffer descriptors from the block's first slot
// (the launcher keeps the span below 2^31 bytes).  Uniform splits: the
// block's own rows, cols = num_splits; the stream-K schedule: kv head kvh's
// rows of every sequence, cols = units + B (sequence b's partials are its
// consecutive columns).  Slot of query row v (position v / G of head
// kvh * G + v % G) and column x: local(v) + x.
template <typename Tag, int D>
struct PartRows {
  static constexpr int kEsz = Tag::kId == QSDPA_F16 ? 2 : 4;  // float16 normalised rows, or float32 sums
  rsrc_t acc, ml;
  int64_t first;
  __device__ __forceinline__ PartRows(const MfmaParams& p, int b, int kvh) {
    const int64_t cols = cols_of(p);
    const int64_t head0 = p.units ? static_cast<int64_t>(kvh) * p.G
                                  : static_cast<int64_t>(b) * p.Hq + static_cast<int64_t>(kvh) * p.G;
    first = head0 * p.qL * cols;
    const uint32_t rows = static_cast<uint32_t>(p.G * p.qL * cols);
    acc = make_rsrc(reinterpret_cast<const uint8_t*>(p.part_acc) + first * D * kEsz, rows * D * kEsz);
    ml = make_rsrc(p.part_ml + first * 2, rows * 8);
  }
  static __device__ __forceinline__ int64_t cols_of(const MfmaParams& p) {
    return p.units ? static_cast<int64_t>(p.units) + p.B : p.num_splits;
  }
  static __device__ __forceinline__ uint32_t local(const MfmaParams& p, int v) {
    return static_cast<uint32_t>(((v % p.G) * p.qL + v / p.G) * cols_of(p));
  }
};

// Merge the NWV waves' running (m, l, acc) of a block's 16 query rows and
// store the result: the normalised output (one split, or `direct`: a
// sequence whose keys one segment covers, merged inside the launch) or the
// split's partial at column `col`.  row_of(w, h): wave w's accumulator row of query row h
// (D floats, dims in order); ml_of(w, h): its (m, l).  Rows >= nh are
// padding.  Called by all `nthreads` threads after a barrier.
template <typename Tag, int D, int NWV, bool FUSED, typename RowF, typename MlF>
__device__ __forceinline__ void merge_store(const MfmaParams& p, RowF&& row_of, MlF&& ml_of, int nh, int v0,
                                            int kvh, int b, int col, int nthreads, bool direct = false) {
  // 16 heads x D dims; thread -> (head, 8 consecutive dims).
  constexpr int kPer = 8;
  for (int idx = threadIdx.x; idx < 16 * (D / kPer); idx += nthreads) {
    const int h = idx / (D / kPer);
    const int d = (idx % (D / kPer)) * kPer;
    if (h >= nh) continue;
    f32x2 ml[NWV];
#pragma unroll
    for (int w = 0; w < NWV; ++w) ml[w] = ml_of(w, h);
    float Mh = ml[0][0];
#pragma unroll
    for (int w = 1; w < NWV; ++w) Mh = fmaxf(Mh, ml[w][0]);
    float L = 0.0f;
    float v[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) v[e] = 0.0f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) {
      const float f = fast_exp2(ml[w][0] - Mh);
      L = fmaf(ml[w][1], f, L);
      const float* src = row_of(w, h) + d;
      const f4 a0 = *reinterpret_cast<const f4*>(src);
      const f4 a1 = *reinterpret_cast<const f4*>(src + 4);
      v[0] = fmaf(a0[0], f, v[0]); v[1] = fmaf(a0[1], f, v[1]);
      v[2] = fmaf(a0[2], f, v[2]); v[3] = fmaf(a0[3], f, v[3]);
      v[4] = fmaf(a1[0], f, v[4]); v[5] = fmaf(a1[1], f, v[5]);
      v[6] = fmaf(a1[2], f, v[6]); v[7] = fmaf(a1[3], f, v[7]);
    }
    const int vh = v0 + h;
    const int hh = kvh * p.G + vh % p.G;  // head and query position of the row
    const int iq = vh / p.G;
    if (p.num_splits == 1 || (FUSED && direct)) {
      store_out8<Tag>(p, b, hh, iq, d, v, L);
    } else if (FUSED) {
      // Partials merged inside this launch (split_merge): agent-coherent
      // stores through the block's descriptors.
      if constexpr (FUSED) {
      const PartRows<Tag, D> pr(p, b, kvh);
      const uint32_t slot = PartRows<Tag, D>::local(p, vh) + col;
      if constexpr (Tag::kId == QSDPA_F16) {
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        const u4 w = u4{pack_T2<Tag>(v[0] * inv, v[1] * inv), pack_T2<Tag>(v[2] * inv, v[3] * inv),
                        pack_T2<Tag>(v[4] * inv, v[5] * inv), pack_T2<Tag>(v[6] * inv, v[7] * inv)};
        __builtin_amdgcn_raw_buffer_store_b128(w, pr.acc, (slot * D + d) * 2, 0, kCoherent);
      } else {
#pragma unroll
        for (int e = 0; e < 2; ++e)
          __builtin_amdgcn_raw_buffer_store_b128(
              u4{__builtin_bit_cast(uint32_t, v[4 * e]), __builtin_bit_cast(uint32_t, v[4 * e + 1]),
                 __builtin_bit_cast(uint32_t, v[4 * e + 2]), __builtin_bit_cast(uint32_t, v[4 * e + 3])},
              pr.acc, (slot * D + d + 4 * e) * 4, 0, kCoherent);
      }
      if (d == 0) {
        typedef uint32_t u2 __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_raw_buffer_store_b64(u2{__builtin_bit_cast(uint32_t, Mh), __builtin_bit_cast(uint32_t, L)},
                                              pr.ml, slot * 8, 0, kCoherent);
      }
      }
    } else {
      // Partial rows: (b, head, position) rows, each with its splits.
      const int64_t prow = static_cast<int64_t>(hh) * p.qL + iq;
      const int64_t slot = p.units ? prow * (p.units + p.B) + col
                                   : (static_cast<int64_t>(b) * p.Hq * p.qL + prow) * p.num_splits + col;
      if constexpr (Tag::kId == QSDPA_F16) {
        // float16 rows of the split's normalised output (acc / L, within
        // the range of V), so the partials are half the bytes.  Plain
        // stores: with the K / V stream non-temporal the rows stay in the
        // caches for the merge (C3 25.2 against 25.6 us per step with
        // streaming stores).
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        uint16_t* dst = reinterpret_cast<uint16_t*>(p.part_acc) + slot * D + d;
        *reinterpret_cast<u4*>(dst) = u4{pack_T2<Tag>(v[0] * inv, v[1] * inv), pack_T2<Tag>(v[2] * inv, v[3] * inv),
                                         pack_T2<Tag>(v[4] * inv, v[5] * inv), pack_T2<Tag>(v[6] * inv, v[7] * inv)};
      } else {
        // Streaming stores: the partials are read once, by the merge kernel.
        float* dst = p.part_acc + slot * D + d;
        __builtin_nontemporal_store(f4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f4*>(dst));
        __builtin_nontemporal_store(f4{v[4], v[5], v[6], v[7]}, reinterpret_cast<f4*>(dst + 4));
      }
      if (d == 0) {
        p.part_ml[slot * 2] = Mh;
        p.part_ml[slot * 2 + 1] = L;
      }
    }
  }
}

}  // namespace
}  // namespace qsdpa
