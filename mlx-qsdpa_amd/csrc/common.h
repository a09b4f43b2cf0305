// Shared device helpers for the gfx950 quantized SDPA kernels.
//
// Storage types are handled as raw 16-bit patterns so the float16 and
// bfloat16 paths share one code shape: `Tag` selects the conversion.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qsdpa.h"

namespace qsdpa {

struct F16 {
  static constexpr int kId = QSDPA_F16;
};
struct BF16 {
  static constexpr int kId = QSDPA_BF16;
};

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, static_cast<uint32_t>(h) << 16);
}
// float -> float16, round to nearest even (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ uint16_t f32_to_f16_bits(float x) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
// float -> bfloat16, round to nearest even; NaN stays NaN (quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  uint32_t u = __builtin_bit_cast(uint32_t, x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

template <typename Tag>
__device__ __forceinline__ float to_f32(uint16_t h) {
  if constexpr (Tag::kId == QSDPA_F16) return f16_bits_to_f32(h);
  else return bf16_bits_to_f32(h);
}
template <typename Tag>
__device__ __forceinline__ uint16_t from_f32(float x) {
  if constexpr (Tag::kId == QSDPA_F16) return f32_to_f16_bits(x);
  else return f32_to_bf16_bits(x);
}
// Round a float to the nearest T value and return it as float.
template <typename Tag>
__device__ __forceinline__ float round_T(float x) {
  return to_f32<Tag>(from_f32<Tag>(x));
}

// ---------------------------------------------------------------------------
// Cross-lane helpers (wave64).
// DPP controls: quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float shfl_xor_f32(float x, int mask) {
  const int lane = __lane_id();
  return __builtin_bit_cast(
      float, __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __builtin_bit_cast(int, x)));
}

// Sum over aligned groups of G consecutive lanes; every lane of a group gets
// the bitwise-identical total (each step adds symmetric partners).
template <int G>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (G >= 2) x += dpp_f32<0xB1>(x);
  if constexpr (G >= 4) x += dpp_f32<0x4E>(x);
  if constexpr (G >= 8) x += dpp_f32<0x141>(x);
  if constexpr (G >= 16) x += dpp_f32<0x140>(x);
  if constexpr (G >= 32) x += shfl_xor_f32(x, 16);
  if constexpr (G >= 64) x += shfl_xor_f32(x, 32);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int shfl_xor_i32(int x, int mask) {
  return __builtin_amdgcn_ds_bpermute((__lane_id() ^ mask) << 2, x);
}

// ---------------------------------------------------------------------------
// Balanced split schedule of a left-padded batch (kv_start given, B > 1).
// Sequence b holds T_b = ceil((N - kv_start[b]) / 32) key tiles (kv_start
// clamped to [0, N]).  U units are shared out over the batch: every unit
// gets at most C tiles, C the smallest budget with sum_b ceil(T_b / C) <= U,
// and sequence b gets n_b = ceil(T_b / C) units, numbered from
// P_b = n_0 + ... + n_{b-1}; unit P_b + i owns the sequence's tiles
// i, i + n_b, i + 2 n_b, ...  The longest unit is then about total / U
// tiles instead of the longest sequence's T / splits.  Each wave computes
// the schedule on its own from the B values of kv_start (the results are
// identical in every wave and workgroup).  Requires U >= B and
// B * (N / 32 + 1) < 2^31.
// ---------------------------------------------------------------------------
constexpr int kSchedTile = 32;

__device__ __forceinline__ int seq_tiles(const int32_t* kv_start, int b, int N) {
  const int s0 = min(max(kv_start[b], 0), N);
  return (N - s0 + kSchedTile - 1) / kSchedTile;
}

// The tile budget C (wave-uniform).
__device__ __forceinline__ int ragged_budget(const int32_t* kv_start, int B, int N, int U) {
  const int lane = __lane_id();
  int tot = 0, mx = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int b = c0 + lane;
    const int t = b < B ? seq_tiles(kv_start, b, N) : 0;
    tot += t;
    mx = max(mx, t);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    tot += shfl_xor_i32(tot, o);
    mx = max(mx, shfl_xor_i32(mx, o));
  }
  tot = __builtin_amdgcn_readfirstlane(tot);
  mx = __builtin_amdgcn_readfirstlane(mx);
  if (tot == 0) return 1;
  // count(c) = sum_b ceil(T_b / c) falls as c grows; count(c) >= tot / c,
  // so count fails below ceil(tot / U); it holds at c = max_b T_b (count =
  // nonempty sequences <= B <= U) and at ceil(tot / (U - B)) (count <=
  // tot / c + B).  Invariant: lo fails (or is 0), hi holds.
  int lo = (tot + U - 1) / U - 1;
  int hi = mx;
  if (U > B) hi = min(hi, (tot + (U - B) - 1) / (U - B));
  while (hi - lo > 1) {
    // 64 candidates at once, lane i testing lo + (i + 1) * step.
    const int step = (hi - lo + 63) / 64;
    const int c = min(lo + (lane + 1) * step, hi);
    int cnt = 0;
    for (int b = 0; b < B; ++b) cnt += (seq_tiles(kv_start, b, N) + c - 1) / c;
    const uint64_t ok = __builtin_amdgcn_ballot_w64(cnt <= U);  // lane 63 tests hi: never 0
    const int first = __builtin_ctzll(ok);
    const int new_hi = min(lo + (first + 1) * step, hi);
    lo = first == 0 ? lo : lo + first * step;
    hi = new_hi;
  }
  return hi;
}

// The (sequence, split within it, splits of the sequence) of unit u under
// budget C; b = -1 when u is past the last unit with work.
struct RaggedUnit {
  int b, split, count;
};

__device__ __forceinline__ int wave_inclusive_scan(int x) {
  const int lane = __lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __builtin_amdgcn_ds_bpermute((lane - o) << 2, x);
    if (lane >= o) x += t;
  }
  return x;
}

__device__ __forceinline__ RaggedUnit ragged_unit(const int32_t* kv_start, int B, int N, int C, int u) {
  const int lane = __lane_id();
  int base = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int b = c0 + lane;
    const int n = b < B ? (seq_tiles(kv_start, b, N) + C - 1) / C : 0;
    const int incl = wave_inclusive_scan(n);
    const int first = base + incl - n;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(u >= first && u < first + n);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      return RaggedUnit{c0 + l, u - __builtin_amdgcn_readlane(first, l), __builtin_amdgcn_readlane(n, l)};
    }
    base += __builtin_amdgcn_readlane(incl, 63);
  }
  return RaggedUnit{-1, 0, 0};
}

// Writes (P_b, n_b) of every sequence to sched[2b], sched[2b + 1] (one wave).
__device__ __forceinline__ void ragged_write_sched(const int32_t* kv_start, int B, int N, int C,
                                                   int* sched) {
  const int lane = __lane_id();
  int base = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int b = c0 + lane;
    const int n = b < B ? (seq_tiles(kv_start, b, N) + C - 1) / C : 0;
    const int incl = wave_inclusive_scan(n);
    if (b < B) *reinterpret_cast<int2*>(sched + 2 * b) = int2{base + incl - n, n};
    base += __builtin_amdgcn_readlane(incl, 63);
  }
}

// ---------------------------------------------------------------------------
// Packed T pairs (two 16-bit values in one 32-bit register).
// ---------------------------------------------------------------------------
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Round two floats to T (nearest even) and pack: v_cvt_pk_{f16,bf16}_f32.
template <typename Tag>
__device__ __forceinline__ uint32_t pack_T2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  if constexpr (Tag::kId == QSDPA_F16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
template <typename Tag>
__device__ __forceinline__ float unpack_T2_lo(uint32_t p) {
  return to_f32<Tag>(static_cast<uint16_t>(p & 0xFFFFu));
}
template <typename Tag>
__device__ __forceinline__ float unpack_T2_hi(uint32_t p) {
  if constexpr (Tag::kId == QSDPA_F16) return f16_bits_to_f32(static_cast<uint16_t>(p >> 16));
  else return __builtin_bit_cast(float, p & 0xFFFF0000u);
}
// a.x*b.x + a.y*b.y + c with float accumulation (v_dot2c_f32_{f16,bf16}).
template <typename Tag>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (Tag::kId == QSDPA_F16)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
  else
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                           false);
}

// Strided 4-D addressing (element strides).
__device__ __forceinline__ int64_t off3(int b, int h, int n, int64_t sb, int64_t sh, int64_t sn) {
  return static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh + static_cast<int64_t>(n) * sn;
}

}  // namespace qsdpa
