// Decode of more than 16 query rows per kv head at D = 256 with 4-bit codes
// and at D = 128 (speculative decoding windows, short chunks; the prefill
// kernel takes the large calls): 32 query rows per workgroup, each wave
// computing both 16-row halves from one dequantized K / V tile.
//
// Reference: the path these calls take there is the dequantize + SDPA
// fallback (mlx_qsdpa/dispatch.py:68-83); the attention is the decode's
// (kernels.py:224-318 per split, merged as kernels.py:342-418).
//
// The 16-row decode kernel (decode_mfma.hip) gives every block of 16 rows
// its own workgroups, so each block streams the kv head and dequantizes it
// again: the exact dequantization is about half of that kernel's VALU work
// at D = 256 and two thirds at D = 128.  Here a block of 32 rows does it
// once.  At D = 256 the two halves' accumulators (128 VGPRs) leave no room
// for Q^T in registers, so each QK step reads its B operands from the
// staged Q rows in LDS (16 ds_read_b128 per wave and tile at D = 256, 8 at
// D = 128, which does the same).  Everything else
// -- tiles, super-tiles, the waves' shares, the whole-row K loads, the
// transposed V loads, the online softmax, the LDS merge of the 8 waves and
// the partial rows -- is the 16-row kernel's, with two running (m, l) per
// lane (row r of each half).  Uniform key splits, or for left-padded
// batches the 16-row kernel's stream-K schedule (SK); the merge kernel for
// the partials; a mask tensor (its own instantiation, MASK) only at D = 128.
#include "abi_internal.h"
#include "mfma_tile.h"
#include "wave_split.h"

namespace qsdpa {

namespace {

constexpr int kRows = 32;  // query rows per workgroup

template <int D>
constexpr int kRowFloats = D + 4;  // LDS floats per (wave, row) of the merge
template <int D>
constexpr int kQRowBytes = D * 2 + 16;  // bytes per staged Q row

// One segment of a block's keys (sequence b): the super-tiles t_lo,
// t_lo + stride, ... up to jmax positions (uniform splits: split x of S from
// x with stride S; the stream-K schedule: a unit's consecutive tiles of one
// sequence), merged over the waves and stored as the output (one split) or
// the partials at column `col`.  Called by the whole workgroup.
template <typename Tag, int D, int BITS, int GS, bool MASK>
__device__ __forceinline__ void rows32_segment(const MfmaParams& p, float* s_acc, float (*s_ml)[16][2],
                                               uint8_t* s_q, int hblk, int kvh, int b, int t_lo, int stride,
                                               int jmax, int col) {
  using G = Geo<D, BITS, GS>;
  using K = Kernel<Tag, D, BITS, GS>;
  constexpr int kRowF = kRowFloats<D>;
  constexpr int kQRow = kQRowBytes<D>;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quad = lane >> 4;
  const int r = lane & 15;

  // The block's rows v0 .. v0 + nh - 1 of the kv head's G * qL rows (row v:
  // position v / G of head kvh * G + v % G); lane r computes row r of each
  // half (clamped to the last real row).
  const int v0 = hblk * kRows;
  const int nh = min(kRows, p.G * p.qL - v0);
  const int n_end = p.causal ? min(p.N, max(0, p.N - p.qL + (v0 + nh - 1) / p.G + 1)) : p.N;
  int n_lane[2];
  int64_t mrow[2];  // the lane's mask rows (MASK)
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int v = v0 + min(16 * k + r, nh - 1);
    const int iq = v / p.G;
    n_lane[k] = p.causal ? min(n_end, max(0, p.N - p.qL + iq + 1)) : n_end;
    mrow[k] = static_cast<int64_t>(b) * p.m_sb + static_cast<int64_t>(kvh * p.G + v % p.G) * p.m_sh +
              static_cast<int64_t>(iq) * p.m_sq;
  }

  // Keys [s0, n_end), 32-token tiles in super-tiles (the 16-row kernel's).
  const int s0 = p.kv_start ? min(max(p.kv_start[b], 0), p.N) : 0;
  const int len = max(n_end - s0, 0);
  const int T = (len + kTile - 1) / kTile;
  const int sh = super_tile_shift(T, stride);
  const int J = super_tile_positions(T, t_lo, stride, jmax, sh);
  auto tile_of = [&](int j) -> int { return super_tile_tile(j, t_lo, stride, sh); };
  static_assert(kWaves == kSplitWaves, "the tile split is for 8 waves");
  const int J8 = wave_split_rr_end(J, D);
  auto next_pos = [&](int j) -> int { return wave_split_next(j, J, J8, wave); };
  const int oob = len + kTile;  // rows outside every descriptor: the loads read zero
  auto row_of = [&](int j) -> int { return j < J ? tile_of(j) * kTile : oob; };

  const Rsrcs rs = tile_rsrcs<D, BITS, GS>(p, b, kvh, s0, len);
  LaneOffsets L;
  VMetaLane vm;
  lane_setup<D, BITS, GS, G::PairK>(rs, quad, r, L, vm);

  // Stage the block's 32 Q rows (zero rows for padding), kThreads / (D / 8)
  // rows per round, each 16-byte piece already in the order the K
  // dequantizer produces the dims (float16 4-bit: 0, 4, 1, 5, 2, 6, 3, 7).
  {
    constexpr int kQChunks = D / 8;  // 16-byte pieces per row
    constexpr int kRounds = kRows * kQChunks / kThreads;
    static_assert(kRounds * kThreads == kRows * kQChunks, "whole staging rounds");
    const int qh = threadIdx.x / kQChunks, qc = threadIdx.x % kQChunks;
    const uint8_t* q0 = reinterpret_cast<const uint8_t*>(p.q) +
                        (static_cast<int64_t>(b) * p.q_sb + static_cast<int64_t>(kvh) * p.G * p.q_sh) * 2;
    const rsrc_t rq = make_rsrc(
        q0, static_cast<uint32_t>(((p.G - 1) * p.q_sh + static_cast<int64_t>(p.qL - 1) * p.q_sq) * 2 + D * 2));
    u4 qv[kRounds];
#pragma unroll
    for (int k = 0; k < kRounds; ++k) {
      const int row = qh + (kThreads / kQChunks) * k;
      const int v = v0 + min(row, nh - 1);
      const int64_t off = (static_cast<int64_t>(v % p.G) * p.q_sh + static_cast<int64_t>(v / p.G) * p.q_sq) * 2;
      qv[k] = __builtin_amdgcn_raw_buffer_load_b128(rq, static_cast<uint32_t>(off + qc * 16), 0, 0);
    }
#pragma unroll
    for (int k = 0; k < kRounds; ++k) {
      const int row = qh + (kThreads / kQChunks) * k;
      u4 w = row < nh ? qv[k] : u4{0u, 0u, 0u, 0u};
      if constexpr (Tag::kId == QSDPA_F16 && BITS == 4) {
        w = u4{perm(w[2], w[0], 0x05040100u), perm(w[2], w[0], 0x07060302u), perm(w[3], w[1], 0x05040100u),
               perm(w[3], w[1], 0x07060302u)};
      }
      *reinterpret_cast<u4*>(s_q + row * kQRow + qc * 16) = w;
    }
  }
  __syncthreads();

  typename K::Regs R;
  int j = wave;
  K::template load_k<G::PairK>(R, rs, L, row_of(j));
  __builtin_amdgcn_sched_barrier(0);
  K::load_v(R, rs, L, row_of(j));
  __builtin_amdgcn_sched_barrier(0);

  // The lane's Q^T pieces: row r of half 0, dims quad * QD + 8 m.
  const uint8_t* qlds = s_q + r * kQRow + quad * G::QD * 2;
  f4 acc[2][G::NB];
#pragma unroll
  for (int k = 0; k < 2; ++k)
#pragma unroll
    for (int i = 0; i < G::NB; ++i) acc[k][i] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float mrun[2] = {kNegBig, kNegBig};
  float lrun[2] = {0.0f, 0.0f};

  while (j < J) {
    const int nj = next_pos(j);
    const int nrow = row_of(nj);
    auto ik = [&](typename K::Regs& X) { K::template load_k<G::PairK>(X, rs, L, nrow); };
    auto iv = [&](typename K::Regs& X) { K::load_v(X, rs, L, nrow); };
    K::template compute_tile2<MASK>(R, p, qlds, 16 * kQRow, acc, mrun, lrun, s0 + row_of(j), s0, n_lane, quad, mrow,
                                    vm, ik, iv);
    j = nj;
  }

  // Merge the 8 waves through LDS, one half at a time, and store each half's
  // rows: the output (one split) or the split's partials (merge kernel).
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int nk = min(16, nh - 16 * k);  // real rows of the half (uniform)
    if (nk <= 0) break;
    float l = lrun[k];
    l += shfl_xor_f32(l, 16);
    l += shfl_xor_f32(l, 32);
    if (k == 1) __syncthreads();  // half 0's merge has read the LDS
    if (quad == 0) {
      s_ml[wave][r][0] = mrun[k];
      s_ml[wave][r][1] = l;
    }
    float* row = s_acc + (wave * 16 + r) * kRowF;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = row + (4 * quad + i) * G::NB;
#pragma unroll
      for (int nb = 0; nb < G::NB; nb += 4)
        *reinterpret_cast<f4*>(dst + nb) =
            f4{acc[k][nb][i], acc[k][nb + 1][i], acc[k][nb + 2][i], acc[k][nb + 3][i]};
    }
    __syncthreads();
    merge_store<Tag, D, kWaves, false>(
        p, [&](int w, int h) { return s_acc + (w * 16 + h) * kRowF; },
        [&](int w, int h) { return f32x2{s_ml[w][h][0], s_ml[w][h][1]}; }, nk, v0 + 16 * k, kvh, b, col,
        kThreads);
  }
}

// SK: a left-padded batch on the stream-K schedule of the 16-row kernel
// (common.h): grid (U, H_kv * row blocks, 1), unit x owning global tiles
// [x C, (x + 1) C) of the sequences laid end to end, one segment per
// sequence it touches, its partials at column x + b; workgroup (0, 0)
// writes the (first column, count) table for the merge kernel.
// Otherwise uniform splits: grid (S, H_kv * row blocks, B).
template <typename Tag, int D, int BITS, int GS, bool MASK, bool SK>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_rows32_kernel(
    MfmaParams p) {
  static_assert(!(D == 256 && BITS == 8), "D = 256 with 8-bit codes: no register room for two halves");
  static_assert(!(D == 256 && MASK), "D = 256: no register room for the mask values");
  __shared__ __attribute__((aligned(16))) float s_acc[kWaves * 16 * kRowFloats<D>];
  __shared__ float s_ml[kWaves][16][2];
  __shared__ __attribute__((aligned(16))) uint8_t s_q[kRows * kQRowBytes<D>];
  const int hblk = blockIdx.y % p.hb_count;
  const int kvh = blockIdx.y / p.hb_count;
  if constexpr (!SK) {
    rows32_segment<Tag, D, BITS, GS, MASK>(p, s_acc, s_ml, s_q, hblk, kvh, blockIdx.z, blockIdx.x, p.num_splits,
                                           0x7FFFFFFF, blockIdx.x);
  } else {
    const int total = streamk_total(p.kv_start, p.B, p.N);
    const int C = max(1, (total + p.units - 1) / p.units);
    if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 64) streamk_write_sched(p.kv_start, p.B, p.N, C, p.sched);
    int g = static_cast<int>(blockIdx.x) * C;
    const int g_end = min(g + C, total);
    if (g >= g_end) return;  // the whole workgroup: no work, nothing to store
    int b, P;
    streamk_find(p.kv_start, p.B, p.N, g, b, P);
    while (g < g_end && b < p.B) {
      const int Tb = seq_tiles(p.kv_start, b, p.N);
      const int hi = min(g_end, P + Tb);
      if (hi > g) {
        rows32_segment<Tag, D, BITS, GS, MASK>(p, s_acc, s_ml, s_q, hblk, kvh, b, g - P, 1, hi - g,
                                               static_cast<int>(blockIdx.x) + b);
        __syncthreads();  // the next segment reuses the LDS
        g = hi;
      }
      P += Tb;
      ++b;
    }
  }
}

using Rows32Kernel = void (*)(MfmaParams);

template <typename Tag, int D, int BITS, bool MASK, bool SK>
Rows32Kernel rows32_by_gs(int gs) {
  return gs == 32 ? decode_rows32_kernel<Tag, D, BITS, 32, MASK, SK>
       : gs == 64 ? decode_rows32_kernel<Tag, D, BITS, 64, MASK, SK>
                  : decode_rows32_kernel<Tag, D, BITS, 128, MASK, SK>;
}

template <typename Tag, bool MASK, bool SK>
Rows32Kernel rows32_d128(const qsdpa_decode_args* a) {
  return a->bits == 4 ? rows32_by_gs<Tag, 128, 4, MASK, SK>(a->group_size)
                      : rows32_by_gs<Tag, 128, 8, MASK, SK>(a->group_size);
}

// No stream-K instantiation at D = 256: it spilled (28-48 bytes of scratch
// per lane); rows32_supports keeps such batches on the 16-row kernel.
template <typename Tag, bool SK>
Rows32Kernel rows32_pick_sk(const qsdpa_decode_args* a) {
  if (a->D == 256) {
    if constexpr (SK) return nullptr;
    else return rows32_by_gs<Tag, 256, 4, false, false>(a->group_size);
  }
  return a->mask.ptr ? rows32_d128<Tag, true, SK>(a) : rows32_d128<Tag, false, SK>(a);
}

template <typename Tag>
Rows32Kernel rows32_pick(const qsdpa_decode_args* a, bool sk) {
  return sk ? rows32_pick_sk<Tag, true>(a) : rows32_pick_sk<Tag, false>(a);
}

}  // namespace

// Calls for the 32-row kernel (those the prefill kernel does not take):
// D = 256 with 4-bit codes or D = 128, several query positions with more
// than 16 rows per kv head, a mask tensor only at D = 128 (C5's heads with
// a bool mask at q_len = 8 over 16K / 64K keys 32.1-32.2 / 89.1-89.5
// against 34.1-34.3 / 113.9-114.9 us, with an additive one at q_len = 16
// over 32K 85.1-89.5 against 118.3-119.6; C1's heads with a bool mask at
// q_len = 16 over 128K 35.7-35.8 against 43.1-43.5), no folded append (a
// left-padded batch runs the 16-row kernel's stream-K schedule, at D = 128
// only; the others uniform splits); and enough work: at least 16K keys
// and, at D = 256, 3 * 2^20 (row, key) pairs in all (32 rows of one kv head
// over 64K keys were still faster on the 16-row kernel, 16.5 against 19.1
// us, over 128K the same).  Measured against the 16-row kernel, C3's
// heads, wall time per call on one box (both with splits rounded down to
// one round of workgroups), 32-row kernel against 16-row kernel, in us:
//   q_len = 2 over 16K / 32K / 64K keys   16.5 / 19.4-19.6 / 22.1-22.2
//                                         against 15.4 / 17.9-18.1 / 23.2-23.3
//   q_len = 3 over 16K / 32K / 64K / 128K 19.0-19.1 / 21.6 / 28.0-28.4 / 42.8-44.0
//                                         against 18.3-18.5 / 24.2-24.3 / 33.0-33.2 / 53.8-55.1
//   q_len = 4 over 16K / 32K / 64K        19.4-19.7 / 22.2-22.4 / 28.7-28.8
//                                         against 18.2 / 23.6-23.8 / 34.2-34.3
//   q_len = 6 over 16K / 32K / 64K        22.9 / 29.0-29.2 / 38.9-41.9
//                                         against 24.7-24.8 / 35.0-35.2 / 57.0-57.5
//   q_len = 7 over 128K                   80.1-81.6 against 118.8-119.3
//   q_len = 8 over 32K                    29.7 against 33.9-34.1
//   q_len = 12 / 16 over 16K              31.1 / 31.8-32.0 against 31.4 / 34.3-34.4
//   q_len = 16 over 8K                    25.1-25.2 against 23.8
//
// At D = 128 (4- or 8-bit codes) the call's (row, key) pairs in all decide:
// at least 2^23, and 16K keys.  C5's heads (B = 4, 8-bit bf16) at q_len = 8
// over 16K / 32K keys 28.3 / 42.2-43.1 against 31.1-31.3 / 49.7-49.8 us,
// q_len = 16 over 16K 39.8-40.4 against 53.1-53.7, q_len = 31 over 32K
// 129.5-133.3 against 204.8-206.3; C1's heads (B = 1, 4-bit f16) at
// q_len = 16 over 128K 27.9-28.2 against 34.9-35.0; but C5's heads at
// q_len = 8 / 16 over 4K 18.1 / 23.4-23.6 against 16.8 / 21.5, C1's heads at
// q_len = 5 over 64K 16.6-16.8 against 16.3-16.4 and q_len = 16 over 32K
// 16.9 against 16.6.
bool rows32_supports(const qsdpa_decode_args* a) {
  if (!(a->D == 128 || (a->D == 256 && a->bits == 4)) || a->q_len <= 1 || a->k_new.ptr) return false;
  if (a->mask.ptr && a->D != 128) return false;  // D = 256: no register room for the mask values
  if (a->kv_start && a->B > 1 && a->D != 128) return false;  // no stream-K instantiation at D = 256
  const int64_t rows = static_cast<int64_t>(a->H_q / a->H_kv) * a->q_len;
  if (rows <= 16 || a->N < 16384) return false;
  const int64_t pairs = static_cast<int64_t>(a->B) * a->H_q * a->q_len * a->N;
  return pairs >= (a->D == 128 ? int64_t(1) << 23 : int64_t(3) << 20);
}

// Splits: as the 16-row kernel's (at most one workgroup per CU), over 32-row
// blocks.
int rows32_num_splits(const qsdpa_decode_args* a, int cus) {
  const int hb = (a->H_q / a->H_kv * a->q_len + kRows - 1) / kRows;
  const int64_t units = static_cast<int64_t>(a->B) * a->H_kv * hb;
  int64_t s = cus / units;
  s = std::min<int64_t>(s, std::max<int64_t>(1, a->N / (4 * kTile)));
  s = std::min<int64_t>(s, 1024);
  return static_cast<int>(std::max<int64_t>(s, 1));
}

int launch_decode_rows32(const qsdpa_decode_args* a, int num_splits, float* part_acc, float* part_ml,
                         int units, int* sched, hipStream_t stream) {
  MfmaParams p = mfma_params(a, num_splits, part_acc, part_ml);
  p.hb_count = (p.G * p.qL + kRows - 1) / kRows;
  p.units = units;
  p.sched = sched;
  const dim3 grid(units ? units : num_splits, p.Hkv * p.hb_count, units ? 1 : p.B);
  const bool sk = units > 0;
  Rows32Kernel k = a->dtype == QSDPA_F16 ? rows32_pick<F16>(a, sk) : rows32_pick<BF16>(a, sk);
  if (!k) return fail(QSDPA_ERR_UNSUPPORTED, "decode_rows32: no stream-K kernel at D=256");
  launch_profiled(k, grid, dim3(kThreads), stream, a->prof_begin, a->prof_end, p);
  return check_launch("decode_rows32");
}

}  // namespace qsdpa
