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

// Max of x over lanes i, i ^ 16, i ^ 32 and i ^ 48 (the four 16-lane rows)
// with gfx950's row swaps: VALU instructions, where a ds_bpermute goes
// through the LDS and waits for it.  Inline assembly, because this compiler
// has folded both halves of its permlane swap builtin's result into one
// register when both inputs were one value.  The s_nops give each swap two wait states after a
// VALU write of its operands and each v_max two after the swap.
__device__ __forceinline__ float max_over_rows(float x) {
  float a = x, b = x;
  asm volatile(
      "s_nop 1\n\t"
      "v_permlane16_swap_b32 %0, %1\n\t"
      "s_nop 1\n\t"
      "v_max_f32 %0, %0, %1\n\t"
      "v_mov_b32 %1, %0\n\t"
      "s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %1\n\t"
      "s_nop 1\n\t"
      "v_max_f32 %0, %0, %1"
      : "+v"(a), "+v"(b));
  return a;
}

// Max of 8 floats in four instructions (three v_max3_f32, one v_max_f32).
// Inline assembly: in IEEE mode the compiler puts a canonicalizing v_max in
// front of fmaxf for every input it cannot prove canonical (MFMA results,
// selects), which more than doubles the count.
__device__ __forceinline__ float max8(const float (&x)[8]) {
  float a, b, c, m;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(a) : "v"(x[0]), "v"(x[1]), "v"(x[2]));
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(b) : "v"(x[3]), "v"(x[4]), "v"(x[5]));
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(c) : "v"(x[6]), "v"(x[7]), "v"(a));
  asm("v_max_f32 %0, %1, %2" : "=v"(m) : "v"(b), "v"(c));
  return m;
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
// Stream-K schedule of a left-padded batch (kv_start given, B > 1).
// Sequence b holds T_b = ceil((N - kv_start[b]) / 32) key tiles (kv_start
// clamped to [0, N]).  The sequences' tiles are laid end to end, sequence b
// from P_b = T_0 + ... + T_{b-1}, and unit u of U owns global tiles
// [u * C, (u + 1) * C), C = ceil(total / U): every unit gets the same work
// whatever the lengths.  A unit's part in sequence b is a segment with its
// own partial, at column u + b of the rows' U + B partial slots (distinct:
// when a unit u' > u also meets a sequence b' < b, sequence b' would have to
// end after unit u starts and sequence b start before unit u' ends, but b
// starts after b' ends).  Sequence b's partials are then the consecutive
// columns u_first + b .. u_last + b, u_first = P_b / C, u_last =
// (P_b + T_b - 1) / C.  Each wave computes what it needs from the B values
// of kv_start (identical results everywhere).  Requires B * (N / 32 + 1)
// < 2^31.
// ---------------------------------------------------------------------------
constexpr int kSchedTile = 32;

__device__ __forceinline__ int seq_tiles(const int32_t* kv_start, int b, int N) {
  const int s0 = min(max(kv_start[b], 0), N);
  return (N - s0 + kSchedTile - 1) / kSchedTile;
}

__device__ __forceinline__ int wave_inclusive_scan(int x) {
  const int lane = __lane_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __builtin_amdgcn_ds_bpermute((lane - o) << 2, x);
    if (lane >= o) x += t;
  }
  return x;
}

// Total tiles of the batch (wave-uniform).
__device__ __forceinline__ int streamk_total(const int32_t* kv_start, int B, int N) {
  const int lane = __lane_id();
  int tot = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int b = c0 + lane;
    tot += b < B ? seq_tiles(kv_start, b, N) : 0;
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) tot += shfl_xor_i32(tot, o);
  return __builtin_amdgcn_readfirstlane(tot);
}

// The sequence holding global tile g (g < total) and its first tile P_b
// (wave-uniform).
__device__ __forceinline__ void streamk_find(const int32_t* kv_start, int B, int N, int g, int& b_out,
                                             int& p_out) {
  const int lane = __lane_id();
  int base = 0;
  b_out = B;
  p_out = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int b = c0 + lane;
    const int t = b < B ? seq_tiles(kv_start, b, N) : 0;
    const int incl = wave_inclusive_scan(t);
    const int first = base + incl - t;
    const uint64_t hit = __builtin_amdgcn_ballot_w64(t > 0 && first <= g && g < first + t);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      b_out = c0 + l;
      p_out = __builtin_amdgcn_readlane(first, l);
      return;
    }
    base += __builtin_amdgcn_readlane(incl, 63);
  }
}

// Writes sequence b's (first partial column, partial count) to sched[2b],
// sched[2b + 1] for the merge; (0, 0) for a sequence with no keys.  One wave.
__device__ __forceinline__ void streamk_write_sched(const int32_t* kv_start, int B, int N, int C, int* sched) {
  const int lane = __lane_id();
  int base = 0;
  for (int c0 = 0; c0 < B; c0 += 64) {
    const int b = c0 + lane;
    const int t = b < B ? seq_tiles(kv_start, b, N) : 0;
    const int incl = wave_inclusive_scan(t);
    const int first = base + incl - t;
    if (b < B) {
      const int uf = first / C, ul = (first + t - 1) / C;
      *reinterpret_cast<int2*>(sched + 2 * b) = t > 0 ? int2{uf + b, ul - uf + 1} : int2{0, 0};
    }
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
