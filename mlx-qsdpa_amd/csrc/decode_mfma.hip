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
// rows).  The sequence is cut into 32-token tiles, grouped in super-tiles of
// up to 8 consecutive tiles; split s of S owns super-tiles s, s + S, s + 2S,
// ..., so the whole grid streams one compact window of the cache at a time
// and a workgroup's waves start on consecutive tiles.  Each wave streams its
// share of the split's tiles with
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
#include "mfma_tile.h"
#include "quant_group.h"
#include "wave_split.h"

namespace qsdpa {

namespace {

// The folded append of sequence b, kv head kvh (one wave): K and V rows of
// p.knew / p.vnew quantized into key N - 1 of the caches, by the quantizer
// of qsdpa_quantize (quant_group.h) with its one-row layout -- GS / 8 lanes
// per group, 8 values each: lanes [0, D / 8) the K row, [D / 8, D / 4) the
// V row -- so the cache holds the same bits either way.  append_load
// issues the lane's 16-byte load of the new row; append_store quantizes
// and stores.
template <int D>
__device__ __forceinline__ uint4 append_load(const MfmaParams& p, int b, int kvh, int lane) {
  constexpr int kRowLanes = D / 8;
  if (lane >= 2 * kRowLanes) return uint4{0u, 0u, 0u, 0u};
  const bool isv = lane >= kRowLanes;
  const int l = isv ? lane - kRowLanes : lane;
  const uint16_t* src = isv ? p.vnew + b * p.vnew_sb + kvh * p.vnew_sh : p.knew + b * p.knew_sb + kvh * p.knew_sh;
  return *reinterpret_cast<const uint4*>(src + 8 * l);
}

template <typename Tag, int D, int BITS, int GS>
__device__ __forceinline__ void append_store(const MfmaParams& p, int b, int kvh, int lane, uint4 w) {
  constexpr int L = GS / 8;         // lanes per group
  constexpr int kRowLanes = D / 8;  // lanes per row
  constexpr int PER = 32 / BITS;
  if (lane >= 2 * kRowLanes) return;
  const bool isv = lane >= kRowLanes;
  const int l = isv ? lane - kRowLanes : lane;
  const int g = l / L, part = l % L;
  const int64_t t = p.N - 1;
  const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
  uint16_t raw[8];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    raw[2 * k] = static_cast<uint16_t>(wv[k]);
    raw[2 * k + 1] = static_cast<uint16_t>(wv[k] >> 16);
  }
  auto val = [&](int i) { return to_f32<Tag>(raw[i]); };
  float lo, hi;
  lane_minmax<8>(val, lo, hi);
  uint32_t* dp = const_cast<uint32_t*>(isv ? p.vp + b * p.vp_sb + kvh * p.vp_sh + t * p.vp_sn
                                           : p.kp + b * p.kp_sb + kvh * p.kp_sh + t * p.kp_sn);
  uint16_t* ds = const_cast<uint16_t*>(isv ? p.vs + b * p.vs_sb + kvh * p.vs_sh + t * p.vs_sn
                                           : p.ks + b * p.ks_sb + kvh * p.ks_sh + t * p.ks_sn);
  uint16_t* db = const_cast<uint16_t*>(isv ? p.vb + b * p.vb_sb + kvh * p.vb_sh + t * p.vb_sn
                                           : p.kb + b * p.kb_sb + kvh * p.kb_sh + t * p.kb_sn);
  quantize_group<Tag, BITS, GS, L>(val, lo, hi, part, dp + 8 * l / PER, ds + g, db + g);
}

template <typename Tag, int D, int BITS, int GS>
__device__ __forceinline__ void append_row(const MfmaParams& p, int b, int kvh, int lane) {
  append_store<Tag, D, BITS, GS>(p, b, kvh, lane, append_load<D>(p, b, kvh, lane));
}

// One segment of a workgroup's work: tiles t_lo, t_lo + stride, ... (at
// most jmax of them) of sequence b for the block's 16 query rows.  Writes the
// normalised output (one split) or the partials at column `col` of the rows'
// partial slots.  Called by the whole workgroup.
template <typename Tag, int D, int BITS, int GS, bool MASK, bool SK, bool FUSED, bool APPEND>
__device__ __forceinline__ void decode_segment(const MfmaParams& p, float* s_acc, float (*s_ml)[16][2],
                                               uint8_t* s_q, int lane, int wave, int quad, int r, int hblk,
                                               int kvh, int b, int t_lo, int stride, int jmax, int col,
                                               bool direct = false) {
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

  // Keys [s0, n_end) of this sequence, in 32-token tiles from s0, taken in
  // super-tiles of 2^sh consecutive tiles (wave_split.h): the segment owns
  // super-tiles t_lo, t_lo + stride, ... (positions j = 0, 1, ..., J - 1).
  // Uniform splits: split s of S owns super-tiles s, s + S, ..., so at any
  // moment the grid streams one compact window of the cache, and each
  // workgroup's first loads cover 8 consecutive tiles (its waves' first
  // positions).  Measured on MI355X at C3 (128 splits): 21.2-21.4 us per
  // decode kernel against 22.2-22.5 with single tiles round-robin (4 tiles
  // per super-tile: 21.2).
  const int s0 = p.kv_start ? min(max(p.kv_start[b], 0), p.N) : 0;
  const int len = max(n_end - s0, 0);
  const int T = (len + kTile - 1) / kTile;
  // (Not for D = 256 with 8-bit codes, whose lanes read 64 contiguous bytes of
  // a K row: C2 took 30.4-30.7 us against 30.1-30.2 with super-tiles.)
  const int sh = D == 256 && BITS == 8 ? 0 : super_tile_shift(T, stride);
  const int J = super_tile_positions(T, t_lo, stride, jmax, sh);
  auto tile_of = [&](int j) -> int { return super_tile_tile(j, t_lo, stride, sh); };
  // The waves' shares of the J positions (wave_split.h).
  static_assert(kWaves == kSplitWaves, "the tile split is for 8 waves");
  const int J8 = wave_split_rr_end(J, D);
  auto next_pos = [&](int j) -> int { return wave_split_next(j, J, J8, wave); };
  // Rows of a position relative to s0; past the end, rows outside every
  // descriptor (the loads read zero without touching memory).  Every tile
  // issues the same loads, so the compiler's vmcnt waits stay exact.
  const int oob = len + kTile;
  auto row_of = [&](int j) -> int { return j < J ? tile_of(j) * kTile : oob; };

  // Buffer descriptors over rows [s0, N) of this (batch, kv head), the
  // lane's load offsets and V meta gather.
  const Rsrcs rs = tile_rsrcs<D, BITS, GS>(p, b, kvh, s0, len);
  constexpr bool kPairK = G::PairK && !MASK;  // whole-row K loads (Geo::PairK)
  LaneOffsets L;
  VMetaLane vm;
  lane_setup<D, BITS, GS, kPairK>(rs, quad, r, L, vm);

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
  // The folded append: the wave that visits the sequence's last tile (wave
  // 0 of split 0 when the sequence has no keys in range) writes key N - 1.
  // Its new-row loads go first; unless the last tile is its first, its
  // first tile's loads follow at once and the quantization and stores run
  // while they are in flight.  Either way the stores are complete (a wait
  // for every counter) before the wave issues another load, so before the
  // last tile's.
  bool appender = false;
  uint4 nw = uint4{0u, 0u, 0u, 0u};
  if constexpr (APPEND) {
    appender = J > 0 ? tile_of(J - 1) == T - 1 && wave == wave_split_last_owner(J, D)
                     : t_lo == 0 && wave == 0;
    if (appender) {
      nw = append_load<D>(p, b, kvh, lane);
      if (J == 0 || j == J - 1) {
        append_store<Tag, D, BITS, GS>(p, b, kvh, lane, nw);
        __builtin_amdgcn_s_waitcnt(0);
        appender = false;
      }
    }
  }
  K::template load_k<kPairK>(R, rs, L, row_of(j));
  __builtin_amdgcn_sched_barrier(0);
  K::load_v(R, rs, L, row_of(j));
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (APPEND) {
    if (appender) {
      append_store<Tag, D, BITS, GS>(p, b, kvh, lane, nw);
      __builtin_amdgcn_s_waitcnt(0);
    }
  }

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
    auto ik = [&](typename K::Regs& X) { K::template load_k<kPairK>(X, rs, L, nrow); };
    auto iv = [&](typename K::Regs& X) { K::load_v(X, rs, L, nrow); };
    K::template compute_tile<MASK>(R, p, qt, acc, mrun, lrun, s0 + row_of(j), s0, n_lane, quad, mrow, vm, ik, iv);
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

  merge_store<Tag, D, kWaves, FUSED>(
      p, [&](int w, int h) { return s_acc + (w * 16 + h) * kRowF; },
      [&](int w, int h) { return f32x2{s_ml[w][h][0], s_ml[w][h][1]}; }, nh, v0, kvh, b, col, kThreads, direct);
}

// The split merge inside the launch (the FUSED instantiations), after
// decode_segment stored this workgroup's partial rows of sequence b at
// column `col` of the block's rows.  The sequence's partials are the
// `count` consecutive columns from `first` (uniform splits: the block's
// num_splits columns; the stream-K schedule: the columns of the segments
// that cover sequence b).  Every workgroup waits until its partial stores
// are complete, then takes a ticket of its (sequence, kv head, row block):
// an agent-scope atomic increment that wraps to zero at `count`, so the
// counter is zero again after every call.  The workgroup that draws the
// last ticket merges the partials in column order, CHUNK at a time with the
// running rescale of the merge kernel, and writes the output; the others
// go on.  No workgroup waits for another, and the order of every sum is
// fixed, so repeated calls give identical bits whichever workgroup merges.
// The partials cross XCDs through agent-coherent loads and stores
// (kCoherent).  Thread t merges dims [8 (t % (D / 8)), +8) of row t / (D / 8).
//
// One level only: with more splits, a second level (the last of a group of
// 16 merging into a group sum, the last group merging the sums) puts two
// rounds of store, ticket and load on the path of the last workgroup, about
// 2.9 us each on MI355X; measured at C3 (128 uniform splits) that made the
// step 30.2 us against 25.2 us with the merge kernel, so uniform splits
// above kFusedSplits keep the merge kernel.
//
// CHUNK: partials in flight at once, 16 for uniform splits (count <= 16: one
// round trip), 8 under the stream-K schedule, whose sequences span few
// segments and whose kernels have less register room (16 spilled to
// scratch there).
template <typename Tag, int D, int CHUNK>
__device__ __forceinline__ void split_merge(const MfmaParams& p, int* s_flag, int b, int kvh, int hblk, int first,
                                            int count) {
  constexpr bool kHalf = Tag::kId == QSDPA_F16;  // float16 normalised partial rows
  constexpr int kPer = 8, kRowT = D / kPer;
  constexpr uint32_t kPast = 0x80000000u;  // an offset past every descriptor: reads zero
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  unsigned* tk = p.tickets + static_cast<int64_t>(b * gridDim.y + blockIdx.y) * kTicketWords;
  // Every partial store of this workgroup is complete before its ticket.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    *s_flag = __builtin_amdgcn_atomic_inc32(tk, static_cast<unsigned>(count - 1), __ATOMIC_RELAXED, "agent") ==
              static_cast<unsigned>(count - 1);
  __syncthreads();
  if (!*s_flag) return;

  const int v0 = hblk * 16, nh = min(16, p.G * p.qL - v0);
  const int t = threadIdx.x, h = t / kRowT, d = (t % kRowT) * kPer;
  if (t >= 16 * kRowT || h >= nh) return;
  const int v = v0 + h;
  const int hh = kvh * p.G + v % p.G, iq = v / p.G;
  const PartRows<Tag, D> pr(p, b, kvh);
  const uint32_t row0 = PartRows<Tag, D>::local(p, v) + static_cast<uint32_t>(first);
  float M = kNegBig, L = 0.0f, acc[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) acc[e] = 0.0f;
  for (int c0 = 0; c0 < count; c0 += CHUNK) {
    // The chunk's loads are issued before its first wait (columns past
    // `count` read zero through an offset past the descriptor).
    u2 m2[CHUNK];
    u4 w[CHUNK][kHalf ? 1 : 2];
#pragma unroll
    for (int k = 0; k < CHUNK; ++k) {
      const bool ok = c0 + k < count;
      const uint32_t slot = row0 + static_cast<uint32_t>(c0 + k);
      m2[k] = __builtin_amdgcn_raw_buffer_load_b64(pr.ml, ok ? slot * 8 : kPast, 0, kCoherent);
#pragma unroll
      for (int q = 0; q < (kHalf ? 1 : 2); ++q)
        w[k][q] = __builtin_amdgcn_raw_buffer_load_b128(
            pr.acc, ok ? (slot * D + d + 4 * q) * PartRows<Tag, D>::kEsz : kPast, 0, kCoherent);
    }
    // Whole-vector bit casts: this compiler reads element 0 for a bit cast
    // of any single element of a vector.
    f32x2 ml[CHUNK];
    float Mc = M;
#pragma unroll
    for (int k = 0; k < CHUNK; ++k) {
      ml[k] = c0 + k < count ? __builtin_bit_cast(f32x2, m2[k]) : f32x2{kNegBig, 0.0f};
      Mc = fmaxf(Mc, ml[k][0]);
    }
    // out = sum_s w_s x_s / sum_s l_s 2^(m_s - M), w_s = l_s 2^(m_s - M)
    // for normalised rows, 2^(m_s - M) for float32 sums (the merge kernel's
    // equations, merge.hip); earlier chunks rescaled to the new maximum.
    const float f = fast_exp2(M - Mc);
    L *= f;
#pragma unroll
    for (int e = 0; e < kPer; ++e) acc[e] *= f;
    M = Mc;
#pragma unroll
    for (int k = 0; k < CHUNK; ++k) {
      const float wk = fast_exp2(ml[k][0] - M);
      L = fmaf(ml[k][1], wk, L);
      const float we = kHalf ? ml[k][1] * wk : wk;
      float xv[kPer];
      if constexpr (kHalf) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t u = w[k][0][e];
          xv[2 * e] = f16_bits_to_f32(static_cast<uint16_t>(u));
          xv[2 * e + 1] = f16_bits_to_f32(static_cast<uint16_t>(u >> 16));
        }
      } else {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const f4 fv = __builtin_bit_cast(f4, w[k][q]);
#pragma unroll
          for (int e = 0; e < 4; ++e) xv[4 * q + e] = fv[e];
        }
      }
#pragma unroll
      for (int e = 0; e < kPer; ++e) acc[e] = fmaf(xv[e], we, acc[e]);
    }
  }
  store_out8<Tag>(p, b, hh, iq, d, acc, L);
}

// Zero output rows of the block's 16 query rows for every sequence of the
// stream-K schedule without keys (no segment covers them, so no merge
// writes them).  One workgroup per block.
template <typename Tag, int D>
__device__ __forceinline__ void zero_empty_sequences(const MfmaParams& p, int kvh, int hblk) {
  constexpr int kPer = 8, kRowT = D / kPer;
  const int v0 = hblk * 16, nh = min(16, p.G * p.qL - v0);
  const int t = threadIdx.x, h = t / kRowT, d = (t % kRowT) * kPer;
  if (t >= 16 * kRowT || h >= nh) return;
  const int v = v0 + h;
  const int hh = kvh * p.G + v % p.G, iq = v / p.G;
  float zero[kPer];
#pragma unroll
  for (int e = 0; e < kPer; ++e) zero[e] = 0.0f;
  for (int b = 0; b < p.B; ++b)
    if (seq_tiles(p.kv_start, b, p.N) == 0) store_out8<Tag>(p, b, hh, iq, d, zero, 0.0f);
}

// APPEND: the folded append (p.knew / p.vnew; its own instantiations, so the
// others carry none of its registers: with it as a run-time branch the C3
// kernel's SGPR spills doubled and the C5 kernel spilled to scratch).
// SK: the stream-K schedule of a left-padded batch (a loop over segments);
// otherwise one uniform split (a separate instantiation, so the loop's
// register pressure stays out of the common case).  MASK: a mask tensor
// (its own instantiation: with the mask code in the unmasked kernel, C3
// took 23.2 instead of 22.3 us).
template <typename Tag, int D, int BITS, int GS, bool SK, bool MASK, bool FUSED, bool APPEND>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_mfma_kernel(MfmaParams p) {
  constexpr int kRowF = D + 4;  // LDS floats per (wave, head) row
  __shared__ __attribute__((aligned(16))) float s_acc[kWaves * 16 * kRowF];
  __shared__ float s_ml[kWaves][16][2];
  constexpr int kQRow = D * 2 + 16;  // bytes per staged Q row
  __shared__ __attribute__((aligned(16))) uint8_t s_q[16 * kQRow];
  __shared__ int s_flag;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quad = lane >> 4;
  const int r = lane & 15;
  const int hblk = blockIdx.y % p.hb_count;
  const int kvh = blockIdx.y / p.hb_count;
  if constexpr (!SK) {
    // Uniform splits: grid (S, H_kv * row blocks, B); split x of sequence z.
    decode_segment<Tag, D, BITS, GS, MASK, false, FUSED, APPEND>(p, s_acc, s_ml, s_q, lane, wave, quad, r, hblk, kvh, blockIdx.z, blockIdx.x,
                                     p.num_splits, 0x7FFFFFFF, blockIdx.x);
    if constexpr (FUSED) split_merge<Tag, D, kFusedSplits>(p, &s_flag, blockIdx.z, kvh, hblk, 0, p.num_splits);
  } else {
    // Left-padded batch: grid (U, H_kv * row blocks, 1), unit x of the
    // stream-K schedule (common.h) owns global tiles [x * C, (x + 1) * C) of
    // the sequences laid end to end, one segment per sequence it touches.
    const int total = streamk_total(p.kv_start, p.B, p.N);
    const int C = max(1, (total + p.units - 1) / p.units);
    // Sequences without keys: no segment reads their key N - 1, so unit 0
    // writes the folded append's row for them.
    if constexpr (APPEND) {
      if (blockIdx.x == 0 && wave == 0)
        for (int b = 0; b < p.B; ++b)
          if (seq_tiles(p.kv_start, b, p.N) == 0) append_row<Tag, D, BITS, GS>(p, b, kvh, lane);
    }
    if constexpr (FUSED) {
      // Sequences without keys get zero rows here (the merge kernel's job
      // otherwise).
      if (blockIdx.x == 0) zero_empty_sequences<Tag, D>(p, kvh, hblk);
    } else {
      if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0) streamk_write_sched(p.kv_start, p.B, p.N, C, p.sched);
    }
    int g = static_cast<int>(blockIdx.x) * C;
    const int g_end = min(g + C, total);
    if (g >= g_end) return;  // the whole workgroup: no work, nothing to store
    int b, P;
    streamk_find(p.kv_start, p.B, p.N, g, b, P);
    while (g < g_end && b < p.B) {
      const int Tb = seq_tiles(p.kv_start, b, p.N);
      const int hi = min(g_end, P + Tb);
      if (hi > g) {
        // Sequence b's tiles [P, P + Tb) lie in units P / C .. (P + Tb - 1) / C:
        // its partials are those units' columns (unit + b).
        const int uf = P / C, count = (P + Tb - 1) / C - uf + 1;
        decode_segment<Tag, D, BITS, GS, MASK, true, FUSED, APPEND>(p, s_acc, s_ml, s_q, lane, wave, quad, r, hblk, kvh, b, g - P, 1, hi - g,
                                         static_cast<int>(blockIdx.x) + b, FUSED && count == 1);
        if constexpr (FUSED) {
          if (count > 1) split_merge<Tag, D, 8>(p, &s_flag, b, kvh, hblk, uf + b, count);
        }
        __syncthreads();  // the next segment reuses the LDS
        g = hi;
      }
      P += Tb;
      ++b;
    }
  }
}

using DecodeKernel = void (*)(MfmaParams);

template <typename Tag, int D, int BITS, bool SK, bool MASK, bool FUSED, bool APPEND>
DecodeKernel by_gs(int gs) {
  return gs == 32 ? decode_mfma_kernel<Tag, D, BITS, 32, SK, MASK, FUSED, APPEND>
       : gs == 64 ? decode_mfma_kernel<Tag, D, BITS, 64, SK, MASK, FUSED, APPEND>
                  : decode_mfma_kernel<Tag, D, BITS, 128, SK, MASK, FUSED, APPEND>;
}

// The instantiation for a launch; null where none is built (the launcher
// never asks for those: abi.hip streamk_units, fused_merge, fused_append).
template <typename Tag, int D, int BITS, bool MASK, bool APPEND>
DecodeKernel pick_kernel(const MfmaParams& p, int gs) {
  // No stream-K instantiation for D = 256, 8-bit codes with a mask tensor
  // (the launcher gives such calls uniform splits: abi.hip streamk_units),
  // nor with the split merge inside the launch at D = 256, 8-bit codes (its
  // registers spilled to scratch): such batches keep the merge kernel.
  constexpr bool kStreamK = !(MASK && D == 256 && BITS == 8);
  constexpr bool kStreamKFused = kStreamK && !(D == 256 && BITS == 8);
  if (p.units) {
    if constexpr (kStreamKFused)
      return p.tickets ? by_gs<Tag, D, BITS, true, MASK, true, APPEND>(gs)
                       : by_gs<Tag, D, BITS, true, MASK, false, APPEND>(gs);
    else if constexpr (kStreamK)
      return p.tickets ? nullptr : by_gs<Tag, D, BITS, true, MASK, false, APPEND>(gs);
    else
      return nullptr;
  }
  return p.tickets ? by_gs<Tag, D, BITS, false, MASK, true, APPEND>(gs)
                   : by_gs<Tag, D, BITS, false, MASK, false, APPEND>(gs);
}

template <typename Tag, int D, int BITS, bool MASK>
void launch_mask(const MfmaParams& p, int gs, hipStream_t stream, const qsdpa_decode_args* a) {
  const dim3 grid(p.units ? p.units : p.num_splits, p.Hkv * p.hb_count, p.units ? 1 : p.B);
  DecodeKernel k = nullptr;
  // The folded append is built for D = 128 without a mask tensor.
  if constexpr (D == 128 && !MASK) {
    k = p.knew ? pick_kernel<Tag, D, BITS, MASK, true>(p, gs) : pick_kernel<Tag, D, BITS, MASK, false>(p, gs);
  } else {
    k = p.knew ? nullptr : pick_kernel<Tag, D, BITS, MASK, false>(p, gs);
  }
  if (k) launch_profiled(k, grid, dim3(kThreads), stream, a->prof_begin, a->prof_end, p);
}

template <typename Tag, int D, int BITS>
void launch_gs(const MfmaParams& p, int gs, hipStream_t stream, const qsdpa_decode_args* a) {
  if (p.mask) launch_mask<Tag, D, BITS, true>(p, gs, stream, a);
  else launch_mask<Tag, D, BITS, false>(p, gs, stream, a);
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

// Splits per (batch, kv head, head block): at most one workgroup per CU in
// total (LDS and registers allow one 8-wave group per CU; rounded down, as a
// few workgroups past the CU count run as a second round: C3's heads at
// q_len = 3 and 7 over 128K keys, 6 and 14 units of 43 and 19 splits, took
// 258 and 266 workgroups), each split at least
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
  int64_t s = cus / units;
  s = std::min<int64_t>(s, std::max<int64_t>(1, a->N / (4 * kTile)));
  s = std::min<int64_t>(s, 1024);
  return static_cast<int>(std::max<int64_t>(s, 1));
}

int launch_decode_mfma(const qsdpa_decode_args* a, int num_splits, float* part_acc, float* part_ml,
                       int units, int* sched, unsigned* tickets, bool append, hipStream_t stream) {
  MfmaParams p = mfma_params(a, num_splits, part_acc, part_ml);
  p.units = units;
  p.sched = sched;
  p.tickets = tickets;
  if (append) {
    p.knew = static_cast<const uint16_t*>(a->k_new.ptr);
    p.knew_sb = a->k_new.stride_b; p.knew_sh = a->k_new.stride_h;
    p.vnew = static_cast<const uint16_t*>(a->v_new.ptr);
    p.vnew_sb = a->v_new.stride_b; p.vnew_sh = a->v_new.stride_h;
  }
  if (units && a->mask.ptr && a->D == 256 && a->bits == 8)
    return fail(QSDPA_ERR_UNSUPPORTED, "decode_mfma: no stream-K kernel for D=256 8-bit codes with a mask");
  if (units && tickets && a->D == 256 && a->bits == 8)
    return fail(QSDPA_ERR_UNSUPPORTED, "decode_mfma: no stream-K kernel with the merge inside for D=256 8-bit codes");
  if (append && (a->D != 128 || a->mask.ptr))
    return fail(QSDPA_ERR_UNSUPPORTED, "decode_mfma: the folded append is built for D=128 without a mask");
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

