// Head-grouped split-K quantized decode on the gfx950 matrix cores.
//
// Reference: mlx_qsdpa/kernels.py:224-318 (split-K pass 1) and 42-160 (the
// single pass).  The reference runs one simdgroup per query head and
// re-dequantizes every K/V row once per head (kernels.py:241, 265-305); here
// the query heads that share a KV head (up to 16, padded when the group is
// narrower) form the N side of 16x16x32 MFMA tiles, so each K/V element is
// read from HBM and dequantized exactly once per workgroup.
//
// Several query positions (qL > 1: speculative or chunked decoding,
// prefill; the reference dequantizes and runs SDPA for those,
// dispatch.py:68-83) extend the N side to the kv head's G * qL rows
// (position v / G, head v % G); a causal mask aligned to the last key ends
// each block's keys at its last row's limit and each lane's at its own.
//
// Workgroup = 8 waves = one split of a (batch, kv head, block of 16 query
// rows).  The sequence is cut into 32-token tiles; split s of S owns tiles
// s, s + S, s + 2S, ..., so the whole grid streams one compact window of the
// cache at a time.  Each wave streams its share of the split's tiles with
// one register set: the next tile's K loads are issued as soon as the
// current K has been consumed, its V loads once the current V has been
// re-arranged for the PV operands.  All K / V / scale / bias reads are raw
// buffer loads through descriptors that end at the sequence's last row
// (hardware range checking; out-of-range rows read as zero, and a missing
// bias is a zero-size descriptor).  Per 32-token tile:
//
//   S^T[t, h] = K[t, :] . Q[h, :]       v_mfma_f32_16x16x32_{f16,bf16}, two
//       16-token halves.  A = K rows: lane (quad, r) holds token r of the half
//       and the quad's quarter of the row (one contiguous 16/32/64-byte load);
//       B = Q^T, loaded once.  K is dequantized in registers (value =
//       scale * code + bias rounded to T, as mx.dequantize).
//   online softmax in the log2 domain on the S^T C fragment: a lane owns one
//       head and 8 tokens of the tile; the running max moves only when a tile
//       max exceeds it by more than 8 (so p <= 256).
//   out^T[d, h] += V^T[d, t] P^T[t, h]   A = V^T, B = P^T.  P^T is the lane's
//       own softmax fragment (token k-order = the S^T C layout).  V is loaded
//       already transposed: lane (quad, r) loads, for each of its 8 tokens,
//       the 8/16-byte piece of the row holding dims [r*D/16, (r+1)*D/16); each
//       load instruction reads 4 complete rows.  MFMA nb then takes dim
//       r*D/16 + nb of the 8 tokens as its A row r, so no LDS transpose is
//       needed.  Token pairs are interleaved with v_perm_b32 and dequantized
//       with the per-token scale / bias pairs.
//
// Float16: codes become exact fp16 values through the "1024 + code" exponent
// trick (v_bitop3_b32 / v_perm_b32; a nibble at bits 4-7 of a half uses
// 64 + code instead, so it needs no shift), then v_pk_fma_f16 applies scale
// and bias.  Bfloat16: dequantization runs in fp32 and is rounded with
// v_cvt_pk_bf16_f32; P is split into two bf16 terms (hi + lo) so the P.V
// product keeps 16 significant bits.
//
// Tiles start at multiples of 32 tokens from the sequence start, so only the
// sequence's last tile is partial; its rows past the end read as zero and
// their scores are set to -inf.  Each wave keeps Q^T in registers.  The 8
// waves merge through LDS; one split writes the normalised output, otherwise
// partials for the merge kernel (merge.hip): float16 inputs store the
// normalised row acc / l as float16 (half the bytes), bfloat16 float32 rows.
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

template <int WORDS, int AUX>
__device__ __forceinline__ void buffer_words(rsrc_t rs, uint32_t off, uint32_t* w) {
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  if constexpr (WORDS % 4 == 0) {
#pragma unroll
    for (int i = 0; i < WORDS / 4; ++i) {
      const u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * i, 0, AUX);
      w[4 * i] = v[0]; w[4 * i + 1] = v[1]; w[4 * i + 2] = v[2]; w[4 * i + 3] = v[3];
    }
  } else if constexpr (WORDS == 2) {
    const u2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, AUX);
    w[0] = v[0]; w[1] = v[1];
  } else {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, AUX);
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
  static __device__ __forceinline__ void load_k(Regs& R, const Rsrcs& rs, const LaneOffsets& L, int rel0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t row = static_cast<uint32_t>(rel0 + 16 * u);
      buffer_words<G::KW, kAux>(rs.k, row * rs.k_sn + L.k_r, R.kw[u]);
      if constexpr (G::KG == 2)
        R.ks[u] = __builtin_amdgcn_raw_buffer_load_b32(rs.ks, row * rs.ks_sn + L.ks_r, 0, kAux);
      else
        R.ks[u] = __builtin_amdgcn_raw_buffer_load_b16(rs.ks, row * rs.ks_sn + L.ks_r, 0, kAux);
      if constexpr (G::KG == 2) {
        R.kb[u] = __builtin_amdgcn_raw_buffer_load_b32(rs.kb, row * rs.kb_sn + L.kb_r, 0, kAux);
      } else {
        R.kb[u] = __builtin_amdgcn_raw_buffer_load_b16(rs.kb, row * rs.kb_sn + L.kb_r, 0, kAux);
      }
    }
  }

  static __device__ __forceinline__ void load_v(Regs& R, const Rsrcs& rs, const LaneOffsets& L, int rel0) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t row = static_cast<uint32_t>(rel0 + 16 * u);
      if constexpr (G::NG >= 2) {
        R.vs[u] = __builtin_amdgcn_raw_buffer_load_b32(rs.vs, row * rs.vs_sn + L.vs_r, 0, kAux);
        R.vb[u] = __builtin_amdgcn_raw_buffer_load_b32(rs.vb, row * rs.vb_sn + L.vb_r, 0, kAux);
      } else {
        R.vs[u] = __builtin_amdgcn_raw_buffer_load_b16(rs.vs, row * rs.vs_sn + L.vs_r, 0, kAux);
        R.vb[u] = __builtin_amdgcn_raw_buffer_load_b16(rs.vb, row * rs.vb_sn + L.vb_r, 0, kAux);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t row = static_cast<uint32_t>(rel0 + 16 * (j >> 2) + (j & 3));
      buffer_words<G::VW, kAux>(rs.v, row * rs.v_sn + L.v_r, R.vw[j]);
    }
  }

  // S^T for one 16-token half u: K dequantized into the A operand (scale *
  // code + bias with the lane's group scales / biases), Q^T as B.
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
    f4 S = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int m = 0; m < G::NM; ++m) {
      const int g = (G::KG == 2 && m >= G::NM / 2) ? 1 : 0;
      uint32_t a[4];
      dequant_k<Tag, BITS>(R.kw[u] + m * G::WPS, s2[g], b2[g], sf[g], bf[g], a);
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

  // One tile: QK, online softmax, PV.
  // The next tile's K loads are issued (issue_k) as soon as this tile's K
  // has been consumed, and its V loads (issue_v) once V is in the PV
  // operands' pre-permuted form, so one register set suffices.
  template <typename IK, typename IV>
  static __device__ __forceinline__ void compute_tile(Regs& R, const MfmaParams& p, const uint32_t (&qt)[G::NM][4],
                                                      f4 (&acc)[G::NB], float& mrun, float& lrun, int tb, int n1, int quad,
                                                      int64_t mrow, const VMetaLane& vm, IK&& issue_k,
                                                      IV&& issue_v) {
    // ---- S^T = K Q^T (Q^T operand m: 16 B per lane, in registers) ----
    f4 S[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) S[u] = qk_half(R, u, qt);
    issue_k(R);

    // ---- scores of (the lane's row, tokens tau(quad, j)), online softmax ----
    // n1: this lane's end of keys (the sequence's, or its causal limit).
    float sc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sc[j] = S[j >> 2][j & 3] * p.qscale;
    if (p.mask) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int t = min(tb + tau(quad, j), p.N - 1);
        sc[j] += mask_value(p, mrow + static_cast<int64_t>(t) * p.m_sn);
      }
    }
    if (__builtin_expect(tb + kTile > n1, 0)) {  // the sequence's last, partial tile
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (tb + tau(quad, j) >= n1) sc[j] = -__builtin_huge_valf();
    }
    float tmax = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                       fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
    tmax = fmaxf(tmax, shfl_xor_f32(tmax, 16));
    tmax = fmaxf(tmax, shfl_xor_f32(tmax, 32));
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
    for (int j = 0; j < 8; ++j) pr[j] = fast_exp2(sc[j] - mrun);
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
};

// One segment of a workgroup's work: tiles t_lo, t_lo + stride, ... (at
// most jmax of them) of sequence b for the block's 16 query rows.  Writes the
// normalised output (one split) or the partials at column `col` of the rows'
// partial slots.  Called by the whole workgroup.
template <typename Tag, int D, int BITS, int GS>
__device__ __forceinline__ void decode_segment(const MfmaParams& p, float* s_acc, float (*s_ml)[16][2],
                                               uint8_t* s_q, int lane, int wave, int quad, int r, int hblk,
                                               int kvh, int b, int t_lo, int stride, int jmax, int col) {
  using G = Geo<D, BITS, GS>;
  using K = Kernel<Tag, D, BITS, GS>;
  constexpr int kRowF = D + 4;       // LDS floats per (wave, head) row
  constexpr int kQRow = D * 2 + 16;  // bytes per staged Q row
  // The block's rows: v0 .. v0 + nh - 1 of the kv head's G * qL rows; row v
  // is query position v / G of head kvh * G + v % G (with one position, the
  // 16 heads of a GQA group).
  const int v0 = hblk * 16;
  const int nh = min(16, p.G * p.qL - v0);       // real rows in the block
  const int v_lane = v0 + min(r, nh - 1);        // this lane's row (clamped)
  const int hq_lane = kvh * p.G + v_lane % p.G;  // its head
  const int iq_lane = v_lane / p.G;              // its query position

  // Causal (aligned to the last key): position i sees keys t <= N - qL + i,
  // so the block needs keys below n_end and each lane below n_lane.
  const int n_end = p.causal ? min(p.N, max(0, p.N - p.qL + (v0 + nh - 1) / p.G + 1)) : p.N;
  const int n_lane = p.causal ? min(n_end, max(0, p.N - p.qL + iq_lane + 1)) : n_end;

  // Keys [s0, n_end) of this sequence, in 32-token tiles from s0.  The
  // segment owns tiles t_lo, t_lo + stride, ... (positions j = 0, 1, ...,
  // J - 1).  Uniform splits: split s of S owns tiles s, s + S, ..., so at any
  // moment the grid streams one compact window of the cache.
  const int s0 = p.kv_start ? min(max(p.kv_start[b], 0), p.N) : 0;
  const int len = max(n_end - s0, 0);
  const int T = (len + kTile - 1) / kTile;
  const int J = T > t_lo ? min(jmax, (T - t_lo + stride - 1) / stride) : 0;
  // Positions below J - E go round-robin to the 8 waves; the last E go to
  // waves 0-3 only.  Waves 4-7 share their SIMDs with waves 0-3, and the
  // older waves' loads are served first, so equal shares would leave 0-3
  // idle at the end.  D = 256 (HBM-bound): E = J / 2 (in whole rounds of 8)
  // gives 0-3 three tiles for every one of 4-7 (C3 24.6 against 25.9 us per
  // step with five for three, C2 33.5 against 34.2); D = 128 (VALU-bound):
  // E = J / 4, five for three (C4 62.5 against 65.5 us with three for one).
  // Every wave's first position (its index) must lie in the round-robin part
  // (J - E >= 8 whenever E > 0), or the waves' position sequences would
  // overlap; both ratios keep E <= J / 2 with E = 0 below 16 positions, and
  // the guard keeps it so.
  const int E0 = D == 256 ? 8 * (J / 16) : 8 * (J / 32);
  const int E = J - E0 >= kWaves ? E0 : 0;
  const int J8 = J - E;
  auto next_pos = [&](int j) -> int {
    if (j + kWaves < J8) return j + kWaves;
    if (wave >= 4) return J;
    return j < J8 ? J8 + wave : j + 4;
  };
  // Rows of a position relative to s0; past the end, rows outside every
  // descriptor (the loads read zero without touching memory).  Every tile
  // issues the same loads, so the compiler's vmcnt waits stay exact.
  const int oob = len + kTile;
  auto row_of = [&](int j) -> int { return j < J ? (t_lo + j * stride) * kTile : oob; };

  // Buffer descriptors over rows [s0, N) of this (batch, kv head).
  Rsrcs rs;
  {
    const int64_t tok0 = s0;
    auto rsrc = [&](const void* base, int64_t sb, int64_t sh, int64_t sn, int esz, int row_bytes,
                    bool present) {
      const uint8_t* p0 = static_cast<const uint8_t*>(base) +
                          (static_cast<int64_t>(b) * sb + static_cast<int64_t>(kvh) * sh + tok0 * sn) * esz;
      const uint32_t bytes =
          (present && len > 0) ? static_cast<uint32_t>((len - 1) * sn * esz + row_bytes) : 0u;
      return make_rsrc(p0, bytes);
    };
    constexpr int kRow = D * BITS / 8;
    constexpr int kMeta = G::NG * 2;
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
  }

  // Per-lane byte offsets.
  const int kg0 = (quad * G::QD) / GS;  // first group of the lane's K quarter
  const int gv = (r * G::NB) / GS;      // group of the lane's V dims
  const int vword = G::NG >= 2 ? quad % G::ND : 0;  // V meta word this lane loads
  LaneOffsets L;
  L.k_r = quad * G::KW * 4 + r * rs.k_sn;
  L.ks_r = kg0 * 2 + r * rs.ks_sn;
  L.kb_r = kg0 * 2 + r * rs.kb_sn;
  L.v_r = r * G::VW * 4 + 4 * quad * rs.v_sn;
  L.vs_r = vword * 4 + r * rs.vs_sn;
  L.vb_r = vword * 4 + r * rs.vb_sn;
  // Token tau(quad, j) of a half sits in row 4*quad + (j & 3); its meta word
  // gv / 2 was loaded by quad gv / 2.
  VMetaLane vm;
  {
    const int dw = G::NG >= 2 ? gv / 2 : 0;
    const int half = G::NG >= 2 ? gv % 2 : 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) vm.src[k] = (16 * dw + 4 * quad + k) * 4;
    vm.sel = half ? 0x07060302u : 0x05040100u;
    vm.shift = half ? 0u : 16u;
  }

  // The block's Q rows (16 rows x D, zero rows for padding) are read once
  // per workgroup, one 16-byte piece per thread, and staged in LDS (rows
  // padded by 16 bytes so the per-lane row reads below are conflict-free).
  constexpr int kQChunks = D / 8;  // 16-byte pieces per row
  const int qh = threadIdx.x / kQChunks, qc = threadIdx.x % kQChunks;
  u4 qv = u4{0u, 0u, 0u, 0u};
  if (qh < 16) {
    // Descriptor over the kv head's G heads x qL positions of this batch.
    const uint8_t* q0 = reinterpret_cast<const uint8_t*>(p.q) +
                        (static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(kvh) * p.G * p.q_sh) * 2;
    const rsrc_t rq = make_rsrc(
        q0, static_cast<uint32_t>(((p.G - 1) * p.q_sh + static_cast<int64_t>(p.qL - 1) * p.q_sq) * 2 + D * 2));
    const int v = v0 + min(qh, nh - 1);
    const int64_t off = (static_cast<int64_t>(v % p.G) * p.q_sh + static_cast<int64_t>(v / p.G) * p.q_sq) * 2;
    qv = __builtin_amdgcn_raw_buffer_load_b128(rq, static_cast<uint32_t>(off + qc * 16), 0, 0);
  }
  // Q is staged before any K / V load is issued: issued together, the
  // grid's first tiles (20 MB at C3) would queue in front of it.
  if (qh < 16) *reinterpret_cast<u4*>(s_q + qh * kQRow + qc * 16) = qh < nh ? qv : u4{0u, 0u, 0u, 0u};
  __syncthreads();
  typename K::Regs R;
  int j = wave;
  K::load_k(R, rs, L, row_of(j));
  __builtin_amdgcn_sched_barrier(0);
  K::load_v(R, rs, L, row_of(j));
  __builtin_amdgcn_sched_barrier(0);

  // Q^T B operands, one 16-byte piece per lane and QK step m: head r, dims
  // quad*QD + 8m + j, in the order the K dequantizer produces them (float16
  // 4-bit: j = 0, 4, 1, 5, 2, 6, 3, 7; otherwise 0..7).
  uint32_t qt[G::NM][4];
#pragma unroll
  for (int m = 0; m < G::NM; ++m) {
    const u4 v = *reinterpret_cast<const u4*>(s_q + r * kQRow + (quad * G::QD + 8 * m) * 2);
    qt[m][0] = v[0]; qt[m][1] = v[1]; qt[m][2] = v[2]; qt[m][3] = v[3];
  }
#pragma unroll
  for (int m = 0; m < G::NM; ++m) {
    const uint32_t d0 = qt[m][0], d1 = qt[m][1], d2 = qt[m][2], d3 = qt[m][3];
    if constexpr (Tag::kId == QSDPA_F16 && BITS == 4) {
      qt[m][0] = perm(d2, d0, 0x05040100u);  // dims 0, 4
      qt[m][1] = perm(d2, d0, 0x07060302u);  // dims 1, 5
      qt[m][2] = perm(d3, d1, 0x05040100u);  // dims 2, 6
      qt[m][3] = perm(d3, d1, 0x07060302u);  // dims 3, 7
    }
  }

  const int64_t mrow = static_cast<int64_t>(b) * p.m_sb + static_cast<int64_t>(hq_lane) * p.m_sh +
                       static_cast<int64_t>(iq_lane) * p.m_sq;  // the lane's mask row
  f4 acc[G::NB];
#pragma unroll
  for (int i = 0; i < G::NB; ++i) acc[i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun = kNegBig;
  float lrun = 0.0f;

  while (j < J) {
    const int nj = next_pos(j);
    const int nrow = row_of(nj);
    auto ik = [&](typename K::Regs& X) { K::load_k(X, rs, L, nrow); };
    auto iv = [&](typename K::Regs& X) { K::load_v(X, rs, L, nrow); };
    K::compute_tile(R, p, qt, acc, mrun, lrun, s0 + row_of(j), n_lane, quad, mrow, vm, ik, iv);
    j = nj;
  }

  // ---- per-head totals over the four quads ----
  lrun += shfl_xor_f32(lrun, 16);
  lrun += shfl_xor_f32(lrun, 32);

  // ---- merge the waves through LDS: raw rows plus each wave's (m, l) ----
  if (quad == 0) {
    s_ml[wave][r][0] = mrun;
    s_ml[wave][r][1] = lrun;
  }
  // acc[nb][i] is out^T[dim (4*quad + i)*NB + nb][head r]: 4 runs of NB dims.
  float* row = s_acc + (wave * 16 + r) * kRowF;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float* dst = row + (4 * quad + i) * G::NB;
#pragma unroll
    for (int nb = 0; nb < G::NB; nb += 4)
      *reinterpret_cast<f4*>(dst + nb) = f4{acc[nb][i], acc[nb + 1][i], acc[nb + 2][i], acc[nb + 3][i]};
  }
  __syncthreads();

  // 16 heads x D dims; thread -> (head, 8 consecutive dims).
  constexpr int kPer = 8;
  for (int idx = threadIdx.x; idx < 16 * (D / kPer); idx += kThreads) {
    const int h = idx / (D / kPer);
    const int d = (idx % (D / kPer)) * kPer;
    if (h >= nh) continue;
    float Mh = s_ml[0][h][0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) Mh = fmaxf(Mh, s_ml[w][h][0]);
    float L = 0.0f;
    float v[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) v[e] = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = fast_exp2(s_ml[w][h][0] - Mh);
      L = fmaf(s_ml[w][h][1], f, L);
      const float* src = s_acc + (w * 16 + h) * kRowF + d;
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
    if (p.num_splits == 1) {
      const float inv = L > 0.0f ? 1.0f / L : 0.0f;
      uint32_t pk[kPer / 2];
#pragma unroll
      for (int e = 0; e < kPer / 2; ++e) pk[e] = pack_T2<Tag>(v[2 * e] * inv, v[2 * e + 1] * inv);
      uint16_t* dst = p.out + static_cast<int64_t>(b) * p.o_sb + static_cast<int64_t>(hh) * p.o_sh +
                      static_cast<int64_t>(iq) * p.o_sq + d;
      // out rows are only 2-byte aligned in general: store pairs.
#pragma unroll
      for (int e = 0; e < kPer / 2; ++e) {
        dst[2 * e] = static_cast<uint16_t>(pk[e]);
        dst[2 * e + 1] = static_cast<uint16_t>(pk[e] >> 16);
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

// SK: the stream-K schedule of a left-padded batch (a loop over segments);
// otherwise one uniform split (a separate instantiation, so the loop's
// register pressure stays out of the common case).
template <typename Tag, int D, int BITS, int GS, bool SK>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_mfma_kernel(MfmaParams p) {
  constexpr int kRowF = D + 4;  // LDS floats per (wave, head) row
  __shared__ __attribute__((aligned(16))) float s_acc[kWaves * 16 * kRowF];
  __shared__ float s_ml[kWaves][16][2];
  constexpr int kQRow = D * 2 + 16;  // bytes per staged Q row
  __shared__ __attribute__((aligned(16))) uint8_t s_q[16 * kQRow];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quad = lane >> 4;
  const int r = lane & 15;
  const int hblk = blockIdx.y % p.hb_count;
  const int kvh = blockIdx.y / p.hb_count;
  if constexpr (!SK) {
    // Uniform splits: grid (S, H_kv * row blocks, B); split x of sequence z.
    decode_segment<Tag, D, BITS, GS>(p, s_acc, s_ml, s_q, lane, wave, quad, r, hblk, kvh, blockIdx.z, blockIdx.x,
                                     p.num_splits, 0x7FFFFFFF, blockIdx.x);
  } else {
    // Left-padded batch: grid (U, H_kv * row blocks, 1), unit x of the
    // stream-K schedule (common.h) owns global tiles [x * C, (x + 1) * C) of
    // the sequences laid end to end, one segment per sequence it touches.
    const int total = streamk_total(p.kv_start, p.B, p.N);
    const int C = max(1, (total + p.units - 1) / p.units);
    if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0) streamk_write_sched(p.kv_start, p.B, p.N, C, p.sched);
    int g = static_cast<int>(blockIdx.x) * C;
    const int g_end = min(g + C, total);
    if (g >= g_end) return;  // the whole workgroup: no work, nothing to store
    int b, P;
    streamk_find(p.kv_start, p.B, p.N, g, b, P);
    while (g < g_end && b < p.B) {
      const int Tb = seq_tiles(p.kv_start, b, p.N);
      const int hi = min(g_end, P + Tb);
      if (hi > g) {
        decode_segment<Tag, D, BITS, GS>(p, s_acc, s_ml, s_q, lane, wave, quad, r, hblk, kvh, b, g - P, 1, hi - g,
                                         static_cast<int>(blockIdx.x) + b);
        __syncthreads();  // the next segment reuses the LDS
        g = hi;
      }
      P += Tb;
      ++b;
    }
  }
}

template <typename Tag, int D, int BITS>
void launch_gs(const MfmaParams& p, int gs, hipStream_t stream, const qsdpa_decode_args* a) {
  const dim3 grid(p.units ? p.units : p.num_splits, p.Hkv * p.hb_count, p.units ? 1 : p.B);
  void (*k)(MfmaParams);
  if (p.units)
    k = gs == 32 ? decode_mfma_kernel<Tag, D, BITS, 32, true>
      : gs == 64 ? decode_mfma_kernel<Tag, D, BITS, 64, true>
                 : decode_mfma_kernel<Tag, D, BITS, 128, true>;
  else
    k = gs == 32 ? decode_mfma_kernel<Tag, D, BITS, 32, false>
      : gs == 64 ? decode_mfma_kernel<Tag, D, BITS, 64, false>
                 : decode_mfma_kernel<Tag, D, BITS, 128, false>;
  launch_profiled(k, grid, dim3(kThreads), stream, a->prof_begin, a->prof_end, p);
}

template <typename Tag, int D>
void launch_bits(const MfmaParams& p, int bits, int gs, hipStream_t stream, const qsdpa_decode_args* a) {
  if (bits == 4) launch_gs<Tag, D, 4>(p, gs, stream, a);
  else launch_gs<Tag, D, 8>(p, gs, stream, a);
}

}  // namespace

// The MFMA path covers D in {128, 256} for any GQA factor (heads padded to
// blocks of 16).  Its vector loads need: q rows 4-byte aligned; K / V rows
// aligned to the per-lane piece (16 B for the K quarter when it is >= 16 B,
// the V piece size otherwise); scale / bias rows 4-byte aligned when a K
// quarter spans two groups (D = 256, group_size = 32).
bool mfma_supports(const qsdpa_decode_args* a) {
  if (a->D != 128 && a->D != 256) return false;
  if (a->group_size != 32 && a->group_size != 64 && a->group_size != 128) return false;
  if (!aligned_view(a->q, 4, 2)) return false;
  const int kq_bytes = a->D / 4 * a->bits / 8;             // K quarter row
  const int vp_bytes = a->D / 16 * a->bits / 8;            // V piece per token
  if (!aligned_view(a->k_packed, std::min(kq_bytes, 16), 4)) return false;
  if (!aligned_view(a->v_packed, std::min(vp_bytes, 16), 4)) return false;
  if (a->D / 4 / a->group_size == 2) {
    if (!aligned_view(a->k_scales, 4, 2) || !aligned_view(a->k_biases, 4, 2)) return false;
  }
  // V scales / biases are read as 32-bit words when a row holds >= 2 groups.
  if (a->D / a->group_size >= 2) {
    if (!aligned_view(a->v_scales, 4, 2) || !aligned_view(a->v_biases, 4, 2)) return false;
  }
  // Byte offsets of rows within the sequence (up to two tiles past its end)
  // are 32-bit.
  const int64_t max_sn = std::max({a->k_packed.stride_n * 4, a->v_packed.stride_n * 4,
                                   a->k_scales.stride_n * 2, a->v_scales.stride_n * 2,
                                   a->k_biases.stride_n * 2, a->v_biases.stride_n * 2});
  if (max_sn < 0 || max_sn * (static_cast<int64_t>(a->N) + 3 * kTile) >= (int64_t(1) << 31)) return false;
  // Q of a kv head (G heads x q_len positions) is read through one
  // descriptor with 32-bit byte offsets.
  const int64_t qL = std::max(a->q_len, 1);
  const int64_t q_sn = qL > 1 ? a->q.stride_n : 0;
  if (a->q.stride_h < 0 || q_sn < 0 ||
      ((a->H_q / a->H_kv - 1) * a->q.stride_h + (qL - 1) * q_sn) * 2 + a->D * 2 >= (int64_t(1) << 31))
    return false;
  return true;
}

// Splits per (batch, kv head, head block): one workgroup per CU in total
// (LDS and registers allow one 8-wave group per CU), each split at least
// four tiles (half the waves busy: at C1, N=4096, 32 splits give 9.56 us per
// step against 10.35 with 16; at C3, N=16K, 128 splits 13.6 against 14.95
// with 64).  A left-padded batch (kv_start, B > 1) runs the stream-K
// schedule over splits * B units, which also sizes for one round: measured
// at C4 (B=16, H_kv=8, lengths U[1K, 32K]) the decode takes 60.0 us with 2
// splits (32 units per kv head, one round), 69.6 us with 4 (two rounds) and
// 79.1 us with 3 (one and a half); uniform splits took 66.1 us at best.
int mfma_num_splits(const qsdpa_decode_args* a, int cus) {
  const int hb = (a->H_q / a->H_kv * std::max(a->q_len, 1) + 15) / 16;
  const int64_t units = static_cast<int64_t>(a->B) * a->H_kv * hb;
  int64_t s = (cus + units - 1) / units;
  s = std::min<int64_t>(s, std::max<int64_t>(1, a->N / (4 * kTile)));
  s = std::min<int64_t>(s, 1024);
  return static_cast<int>(std::max<int64_t>(s, 1));
}

int launch_decode_mfma(const qsdpa_decode_args* a, int num_splits, float* part_acc, float* part_ml,
                       int units, int* sched, hipStream_t stream) {
  MfmaParams p = mfma_params(a, num_splits, part_acc, part_ml);
  p.units = units;
  p.sched = sched;
  const bool f16 = a->dtype == QSDPA_F16;
  if (a->D == 128) {
    if (f16) launch_bits<F16, 128>(p, a->bits, a->group_size, stream, a);
    else launch_bits<BF16, 128>(p, a->bits, a->group_size, stream, a);
  } else {
    if (f16) launch_bits<F16, 256>(p, a->bits, a->group_size, stream, a);
    else launch_bits<BF16, 256>(p, a->bits, a->group_size, stream, a);
  }
  return check_launch("decode_mfma");
}

}  // namespace qsdpa
