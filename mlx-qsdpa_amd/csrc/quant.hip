// Quantize-on-append and dequantize kernels (MLX affine format).
//
// quantize: GS / 8 lanes per (row, group) with 8 values each for small jobs,
// GS / 32 lanes with 32 values for large ones.  The per-group rule is the
// float32 edge-snapped affine quantizer (see oracle/affine.py for the written
// contract); every operation is spelled with an explicitly rounded intrinsic
// (the one fma is written out), and each code's division goes through the
// group's reciprocal with an exact fallback near ties, which keeps the output
// bit-identical to the numpy restatement.
//
// dequantize: one thread per packed word; value = round_T(fmaf(s, q, b)).
// Replaces mx.quantize + slice assignment (mlx_qsdpa/cache.py:186-192) and
// mx.dequantize (mlx_qsdpa/dispatch.py:69-78, cache.py:628-633).
#include <algorithm>

#include "abi_internal.h"
#include "common.h"
#include "quant_group.h"

namespace qsdpa {
namespace {

struct QuantParams {
  int B, H, S, D, gs, t0;
  const uint16_t* src;
  int64_t s_sb, s_sh, s_sn;
  uint32_t* dp;
  int64_t p_sb, p_sh, p_sn;
  uint16_t* ds;
  int64_t c_sb, c_sh, c_sn;
  uint16_t* db;
  int64_t z_sb, z_sh, z_sn;
};

// Up to kMaxJobs quantize jobs (the keys and values of one cache update)
// run in one launch, job = blockIdx.y; they share dtype, bits and
// group_size.
constexpr int kMaxJobs = 4;
struct QuantJobs {
  QuantParams p[kMaxJobs];
};

// One group of GS values is spread over L consecutive lanes, GS / L values
// per lane (16-byte pieces when VEC, i.e. the rows are 16-byte aligned); the
// group's min / max are reduced across the L lanes and every lane quantizes
// and packs its own values.  L = GS / 8 for small jobs (a one-row append:
// its latency is that of 8 values, not GS); L = GS / 32 for large ones,
// which fill the GPU anyway: a lane's group work (min / max reductions,
// scale divisions) is then shared by 32 values.  A group's lanes are all in range or all out of it, so the
// cross-lane steps never read an exited lane.  I is the index type: 32-bit
// whenever the launch's thread count fits.
template <typename Tag, int BITS, int GS, int L, bool VEC, typename I>
__global__ __launch_bounds__(256) void quantize_kernel(QuantJobs jobs) {
  constexpr int VALS = GS / L;  // values per lane, a multiple of 8
  constexpr int PER = 32 / BITS;
  const QuantParams& p = jobs.p[blockIdx.y];
  const int ng = p.D / GS;
  const I total = static_cast<I>(p.B) * p.H * p.S * ng;
  const I gid = static_cast<I>(blockIdx.x) * blockDim.x + threadIdx.x;
  const I grp = gid / L;
  const int part = static_cast<int>(gid % L);
  if (grp >= total) return;
  const int g = static_cast<int>(grp % ng);
  I row = grp / ng;
  const int s = static_cast<int>(row % p.S);
  row /= p.S;
  const int h = static_cast<int>(row % p.H);
  const int b = static_cast<int>(row / p.H);

  const uint16_t* src = p.src + off3(b, h, s, p.s_sb, p.s_sh, p.s_sn) + g * GS + part * VALS;
  uint16_t raw[VALS];
  if constexpr (VEC) {
#pragma unroll
    for (int i = 0; i < VALS / 8; ++i) {
      const uint4 v = reinterpret_cast<const uint4*>(src)[i];
      const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        raw[8 * i + 2 * k] = static_cast<uint16_t>(wv[k]);
        raw[8 * i + 2 * k + 1] = static_cast<uint16_t>(wv[k] >> 16);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < VALS; ++i) raw[i] = src[i];
  }

  auto val = [&](int i) { return to_f32<Tag>(raw[i]); };
  float lo, hi;
  lane_minmax<VALS>(val, lo, hi);
  const int t = p.t0 + s;
  quantize_group<Tag, BITS, GS, L>(val, lo, hi, part, p.dp + off3(b, h, t, p.p_sb, p.p_sh, p.p_sn) + (g * GS + part * VALS) / PER,
                                   p.ds + off3(b, h, t, p.c_sb, p.c_sh, p.c_sn) + g,
                                   p.db + off3(b, h, t, p.z_sb, p.z_sh, p.z_sn) + g);
}

// Jobs with at least this many groups take one lane per group.
constexpr int64_t kWideJobGroups = 1 << 18;

template <typename Tag, int BITS, int GS, int L>
void launch_quantize_l(const QuantJobs& j, bool vec, int64_t groups, int count, hipStream_t stream) {
  const int64_t blocks = (groups * L + 255) / 256;
  const dim3 grid(static_cast<unsigned>(blocks), static_cast<unsigned>(count));
  if (blocks * 256 >= (int64_t(1) << 32)) {
    if (vec) quantize_kernel<Tag, BITS, GS, L, true, int64_t><<<grid, dim3(256), 0, stream>>>(j);
    else quantize_kernel<Tag, BITS, GS, L, false, int64_t><<<grid, dim3(256), 0, stream>>>(j);
  } else {
    if (vec) quantize_kernel<Tag, BITS, GS, L, true, uint32_t><<<grid, dim3(256), 0, stream>>>(j);
    else quantize_kernel<Tag, BITS, GS, L, false, uint32_t><<<grid, dim3(256), 0, stream>>>(j);
  }
}

template <typename Tag, int BITS, int GS>
void launch_quantize_gs(const QuantJobs& j, bool vec, int64_t groups, int count, hipStream_t stream) {
  if (groups >= kWideJobGroups) launch_quantize_l<Tag, BITS, GS, GS / 32>(j, vec, groups, count, stream);
  else launch_quantize_l<Tag, BITS, GS, GS / 8>(j, vec, groups, count, stream);
}

template <typename Tag, int BITS>
void launch_quantize_bits(const QuantJobs& j, int gs, bool vec, int64_t groups, int count, hipStream_t stream) {
  if (gs == 32) launch_quantize_gs<Tag, BITS, 32>(j, vec, groups, count, stream);
  else if (gs == 64) launch_quantize_gs<Tag, BITS, 64>(j, vec, groups, count, stream);
  else launch_quantize_gs<Tag, BITS, 128>(j, vec, groups, count, stream);
}

struct DequantParams {
  int B, H, N, D, gs, keep, rot;
  const uint32_t* sp;
  int64_t p_sb, p_sh, p_sn;
  const uint16_t* ss;
  int64_t c_sb, c_sh, c_sn;
  const uint16_t* sbias;  // may be null
  int64_t z_sb, z_sh, z_sn;
  uint16_t* dst;
  int64_t d_sb, d_sh, d_sn;
};

template <typename Tag, int BITS>
__global__ __launch_bounds__(256) void dequantize_kernel(DequantParams p) {
  constexpr int PER = 32 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const int words = p.D / PER;
  const int64_t total = static_cast<int64_t>(p.B) * p.H * p.N * words;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= total) return;
  const int w = static_cast<int>(gid % words);
  int64_t row = gid / words;
  const int t = static_cast<int>(row % p.N);
  row /= p.N;
  const int h = static_cast<int>(row % p.H);
  const int b = static_cast<int>(row / p.H);
  const int u = (t < p.keep) ? t : p.keep + (t - p.keep + p.rot) % (p.N - p.keep);

  const uint32_t word = p.sp[off3(b, h, u, p.p_sb, p.p_sh, p.p_sn) + w];
  const int g = (w * PER) / p.gs;
  const float s = to_f32<Tag>(p.ss[off3(b, h, u, p.c_sb, p.c_sh, p.c_sn) + g]);
  const float bi = p.sbias ? to_f32<Tag>(p.sbias[off3(b, h, u, p.z_sb, p.z_sh, p.z_sn) + g]) : 0.0f;
  uint16_t* out = p.dst + off3(b, h, t, p.d_sb, p.d_sh, p.d_sn) + w * PER;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const float q = static_cast<float>((word >> (j * BITS)) & kMask);
    out[j] = from_f32<Tag>(__fmaf_rn(s, q, bi));
  }
}

// Rotating-window prefill in one pass (reference: mlx_qsdpa/cache.py:593-634
// and 813-857, dequantize the window in temporal order, append the chunk,
// keep the newest max_size tokens, quantize again; plus keep > 0 sinks).
// Output row t of the new window is combined token c = t (a sink, or no
// token dropped) or t + drop (drop = n_old + S - total tokens leave after
// the sinks).  Combined token c < n_old is old window row u(c) = c for
// c < keep, else keep + (c - keep + rot) % (n_old - keep): dequantized
// exactly as dequantize_kernel does, value = T(fmaf(s, q, b)); otherwise it
// is chunk row c - n_old.  The row is then quantized as quantize_kernel
// does (quantize_group), 32 values per lane, GS / 32 lanes per group (the
// group's min / max reductions and scale divisions shared by 32 values, not
// 8: the kernel was VALU-bound at 8), into the destination buffers, which
// must not alias the old window.
struct RequantParams {
  int B, H, D, n_old, keep, rot, total, drop;
  const uint32_t* op;
  int64_t op_sb, op_sh, op_sn;
  const uint16_t* os;
  int64_t os_sb, os_sh, os_sn;
  const uint16_t* ob;  // may be null (zero biases)
  int64_t ob_sb, ob_sh, ob_sn;
  const uint16_t* src;
  int64_t s_sb, s_sh, s_sn;
  uint32_t* dp;
  int64_t p_sb, p_sh, p_sn;
  uint16_t* ds;
  int64_t c_sb, c_sh, c_sn;
  uint16_t* db;
  int64_t z_sb, z_sh, z_sn;
};
struct RequantJobs {
  RequantParams p[2];
};

template <typename Tag, int BITS, int GS, bool DST16>
__global__ __launch_bounds__(256) void requant_kernel(RequantJobs jobs) {
  // Grid: x over the (row, lane) pairs of one group column of one (batch,
  // head), y = (batch * H + head) * ng + group, z = job: the group, batch and
  // head are uniform.  Within a (batch, head) every offset fits in 32 bits
  // (the launcher checks), so the lanes' row offsets are 32-bit products.
  constexpr int VALS = 32;         // values per lane
  constexpr int L = GS / VALS;     // lanes per group
  constexpr int PER = 32 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const RequantParams& p = jobs.p[blockIdx.z];
  // (The compiler divides in vector registers; readfirstlane keeps the
  // slice bases' 64-bit products scalar.)
  const int ng = p.D / GS;
  const int g = __builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.y) % ng);
  const int bh = static_cast<int>(blockIdx.y) / ng;
  const int b = __builtin_amdgcn_readfirstlane(bh / p.H), h = __builtin_amdgcn_readfirstlane(bh % p.H);
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const int t = static_cast<int>(gid / L);
  const int part = static_cast<int>(gid % L);
  if (t >= p.total) return;
  auto rows = [&](auto* base, int64_t sb, int64_t sh) {
    return base + (static_cast<int64_t>(b) * sb + static_cast<int64_t>(h) * sh);
  };
  uint32_t* const dst_p = rows(p.dp, p.p_sb, p.p_sh);
  uint16_t* const dst_s = rows(p.ds, p.c_sb, p.c_sh);
  uint16_t* const dst_b = rows(p.db, p.z_sb, p.z_sh);
  auto at = [](int row, int64_t sn) { return static_cast<uint32_t>(row) * static_cast<uint32_t>(sn); };
  const int c = t < p.keep ? t : t + p.drop;
  const int d0 = g * GS + part * VALS;  // the lane's first dim
  float val[VALS];  // T values as float
  float lo, hi;     // their min / max
  if (c < p.n_old) {
    // Ring row of combined token c: c - keep + rot < 2 (n_old - keep), so one
    // conditional subtraction is the modulo.
    int u = c;
    if (c >= p.keep && p.rot != 0) {
      u = c - p.keep + p.rot;
      if (u >= p.n_old - p.keep) u -= p.n_old - p.keep;
      u += p.keep;
    }
    const float sc = to_f32<Tag>(rows(p.os, p.os_sb, p.os_sh)[at(u, p.os_sn) + g]);
    const float bi = p.ob ? to_f32<Tag>(rows(p.ob, p.ob_sb, p.ob_sh)[at(u, p.ob_sn) + g]) : 0.0f;
    const uint32_t* words = rows(p.op, p.op_sb, p.op_sh) + (at(u, p.op_sn) + d0 / PER);
    // T(fmaf(s, q, b)) as dequantize_kernel stores it, rounded two values
    // at a time (v_cvt_pk_*_f32: the same rounding, and a NaN still reads
    // as NaN, which the quantizer maps to code 0 whatever its bits).
    float y[VALS];
#pragma unroll
    for (int w = 0; w < VALS / PER; ++w) {
      const uint32_t word = words[w];
#pragma unroll
      for (int j = 0; j < PER; ++j)
        y[w * PER + j] = __fmaf_rn(sc, static_cast<float>((word >> (j * BITS)) & kMask), bi);
    }
#pragma unroll
    for (int i = 0; i < VALS; i += 2) {
      const uint32_t pr = pack_T2<Tag>(y[i], y[i + 1]);
      val[i] = unpack_T2_lo<Tag>(pr);
      val[i + 1] = unpack_T2_hi<Tag>(pr);
    }
    // The min / max of the rounded values are the rounded min / max of the
    // fma results (rounding is monotone), which the compiler knows to be
    // canonical floats: no quieting v_max per value.
    lane_minmax<VALS>([&](int i) { return y[i]; }, lo, hi);
    const uint32_t m = pack_T2<Tag>(lo, hi);
    lo = unpack_T2_lo<Tag>(m);
    hi = unpack_T2_hi<Tag>(m);
  } else {
    const uint16_t* src = rows(p.src, p.s_sb, p.s_sh) + (at(c - p.n_old, p.s_sn) + d0);
#pragma unroll
    for (int i = 0; i < VALS; ++i) val[i] = to_f32<Tag>(src[i]);
    lane_minmax<VALS>([&](int i) { return val[i]; }, lo, hi);
  }
  quantize_group<Tag, BITS, GS, L, DST16>([&](int i) { return val[i]; }, lo, hi, part, dst_p + (at(t, p.p_sn) + d0 / PER),
                                          dst_s + (at(t, p.c_sn) + g), dst_b + (at(t, p.z_sn) + g));
}

}  // namespace

int launch_quantize(const qsdpa_quantize_args* const* jobs, int count, hipStream_t stream) {
  if (count < 1 || count > kMaxJobs) return fail(QSDPA_ERR_INVALID, "quantize: %d jobs (1..%d)", count, kMaxJobs);
  QuantJobs j{};
  int64_t most = 0;  // groups of the largest job
  bool vec = true;
  for (int i = 0; i < count; ++i) {
    const qsdpa_quantize_args* a = jobs[i];
    QuantParams& p = j.p[i];
    p.B = a->B; p.H = a->H; p.S = a->S; p.D = a->D; p.gs = a->group_size; p.t0 = a->t0;
    p.src = static_cast<const uint16_t*>(a->src.ptr);
    p.s_sb = a->src.stride_b; p.s_sh = a->src.stride_h; p.s_sn = a->src.stride_n;
    p.dp = static_cast<uint32_t*>(const_cast<void*>(a->dst_packed.ptr));
    p.p_sb = a->dst_packed.stride_b; p.p_sh = a->dst_packed.stride_h; p.p_sn = a->dst_packed.stride_n;
    p.ds = static_cast<uint16_t*>(const_cast<void*>(a->dst_scales.ptr));
    p.c_sb = a->dst_scales.stride_b; p.c_sh = a->dst_scales.stride_h; p.c_sn = a->dst_scales.stride_n;
    p.db = static_cast<uint16_t*>(const_cast<void*>(a->dst_biases.ptr));
    p.z_sb = a->dst_biases.stride_b; p.z_sh = a->dst_biases.stride_h; p.z_sn = a->dst_biases.stride_n;
    most = std::max<int64_t>(most, static_cast<int64_t>(a->B) * a->H * a->S * (a->D / a->group_size));
    // 16-byte loads need 16-byte aligned rows (a lane's offset in the row
    // is a multiple of 8 elements).
    vec = vec && aligned(a->src.ptr, 16) && a->src.stride_b % 8 == 0 && a->src.stride_h % 8 == 0 &&
          a->src.stride_n % 8 == 0;
  }
  if (most == 0) return QSDPA_OK;
  if (most * 16 / 256 >= (int64_t(1) << 31))
    return fail(QSDPA_ERR_UNSUPPORTED, "quantize: %lld groups too many", static_cast<long long>(most));
  const qsdpa_quantize_args* a = jobs[0];
  if (a->dtype == QSDPA_F16) {
    if (a->bits == 4) launch_quantize_bits<F16, 4>(j, a->group_size, vec, most, count, stream);
    else launch_quantize_bits<F16, 8>(j, a->group_size, vec, most, count, stream);
  } else {
    if (a->bits == 4) launch_quantize_bits<BF16, 4>(j, a->group_size, vec, most, count, stream);
    else launch_quantize_bits<BF16, 8>(j, a->group_size, vec, most, count, stream);
  }
  return check_launch("quantize");
}

int launch_dequantize(const qsdpa_dequantize_args* a, hipStream_t stream) {
  DequantParams p;
  p.B = a->B; p.H = a->H; p.N = a->N; p.D = a->D; p.gs = a->group_size;
  p.keep = a->keep; p.rot = a->rot;
  p.sp = static_cast<const uint32_t*>(a->src_packed.ptr);
  p.p_sb = a->src_packed.stride_b; p.p_sh = a->src_packed.stride_h; p.p_sn = a->src_packed.stride_n;
  p.ss = static_cast<const uint16_t*>(a->src_scales.ptr);
  p.c_sb = a->src_scales.stride_b; p.c_sh = a->src_scales.stride_h; p.c_sn = a->src_scales.stride_n;
  p.sbias = static_cast<const uint16_t*>(a->src_biases.ptr);
  p.z_sb = a->src_biases.stride_b; p.z_sh = a->src_biases.stride_h; p.z_sn = a->src_biases.stride_n;
  p.dst = static_cast<uint16_t*>(const_cast<void*>(a->dst.ptr));
  p.d_sb = a->dst.stride_b; p.d_sh = a->dst.stride_h; p.d_sn = a->dst.stride_n;
  const int per = 32 / a->bits;
  const int64_t total = static_cast<int64_t>(a->B) * a->H * a->N * (a->D / per);
  if (total == 0) return QSDPA_OK;
  const dim3 block(256);
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  if (a->dtype == QSDPA_F16) {
    if (a->bits == 4) dequantize_kernel<F16, 4><<<grid, block, 0, stream>>>(p);
    else dequantize_kernel<F16, 8><<<grid, block, 0, stream>>>(p);
  } else {
    if (a->bits == 4) dequantize_kernel<BF16, 4><<<grid, block, 0, stream>>>(p);
    else dequantize_kernel<BF16, 8><<<grid, block, 0, stream>>>(p);
  }
  return check_launch("dequantize");
}

int launch_requant(const qsdpa_requant_args* const* jobs, int count, hipStream_t stream) {
  RequantJobs j{};
  int64_t most = 0;
  bool dst16 = true;
  const qsdpa_requant_args* a0 = jobs[0];
  for (int i = 0; i < count; ++i) {
    const qsdpa_requant_args* a = jobs[i];
    RequantParams& p = j.p[i];
    p.B = a->B; p.H = a->H; p.D = a->D; p.n_old = a->n_old; p.keep = a->keep; p.rot = a->rot;
    p.total = std::min(a->n_old + a->S, a->max_size);
    p.drop = a->n_old + a->S - p.total;
    p.op = static_cast<const uint32_t*>(a->old_packed.ptr);
    p.op_sb = a->old_packed.stride_b; p.op_sh = a->old_packed.stride_h; p.op_sn = a->old_packed.stride_n;
    p.os = static_cast<const uint16_t*>(a->old_scales.ptr);
    p.os_sb = a->old_scales.stride_b; p.os_sh = a->old_scales.stride_h; p.os_sn = a->old_scales.stride_n;
    p.ob = static_cast<const uint16_t*>(a->old_biases.ptr);
    p.ob_sb = a->old_biases.stride_b; p.ob_sh = a->old_biases.stride_h; p.ob_sn = a->old_biases.stride_n;
    p.src = static_cast<const uint16_t*>(a->src.ptr);
    p.s_sb = a->src.stride_b; p.s_sh = a->src.stride_h; p.s_sn = a->src.stride_n;
    p.dp = static_cast<uint32_t*>(const_cast<void*>(a->dst_packed.ptr));
    p.p_sb = a->dst_packed.stride_b; p.p_sh = a->dst_packed.stride_h; p.p_sn = a->dst_packed.stride_n;
    p.ds = static_cast<uint16_t*>(const_cast<void*>(a->dst_scales.ptr));
    p.c_sb = a->dst_scales.stride_b; p.c_sh = a->dst_scales.stride_h; p.c_sn = a->dst_scales.stride_n;
    p.db = static_cast<uint16_t*>(const_cast<void*>(a->dst_biases.ptr));
    p.z_sb = a->dst_biases.stride_b; p.z_sh = a->dst_biases.stride_h; p.z_sn = a->dst_biases.stride_n;
    // A lane's first code word is a multiple of 4 words into its row.
    dst16 = dst16 && aligned(a->dst_packed.ptr, 16) && p.p_sb % 4 == 0 && p.p_sh % 4 == 0 && p.p_sn % 4 == 0;
    most = std::max<int64_t>(most, static_cast<int64_t>(p.total) * (a->D / a->group_size));
  }
  if (most == 0 || a0->B * a0->H == 0) return QSDPA_OK;
  // Lanes of one group column of one (batch, head): rows x GS / 32; one
  // grid row per (batch, head, group).
  const int64_t ng = a0->D / a0->group_size;
  const int64_t lanes = most / ng * (a0->group_size / 32);
  if (lanes + 255 >= (int64_t(1) << 32) || static_cast<int64_t>(a0->B) * a0->H * ng > 65535)
    return fail(QSDPA_ERR_UNSUPPORTED, "requant: window too large");
  // Offsets within a (batch, head) are 32-bit in the kernel: rows x row
  // stride plus the row's extent must stay below 2^31 elements.
  for (int i = 0; i < count; ++i) {
    const qsdpa_requant_args* a = jobs[i];
    const int per = 32 / a->bits;
    auto fits = [](int64_t rows, int64_t stride_n, int64_t extent) {
      return stride_n >= 0 && (rows <= 0 || (rows - 1) * stride_n + extent < (int64_t(1) << 31));
    };
    const int64_t total = j.p[i].total;
    if (!fits(a->n_old, a->old_packed.stride_n, a->D / per) || !fits(a->n_old, a->old_scales.stride_n, ng) ||
        (a->old_biases.ptr && !fits(a->n_old, a->old_biases.stride_n, ng)) ||
        !fits(a->S, a->src.stride_n, a->D) || !fits(total, a->dst_packed.stride_n, a->D / per) ||
        !fits(total, a->dst_scales.stride_n, ng) || !fits(total, a->dst_biases.stride_n, ng))
      return fail(QSDPA_ERR_UNSUPPORTED, "requant: a (batch, head) slice spans 2^31 elements or more");
  }
  const dim3 grid(static_cast<unsigned>((lanes + 255) / 256), static_cast<unsigned>(a0->B * a0->H * ng),
                  static_cast<unsigned>(count));
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(256), 0, stream, j); };
  const bool f16 = a0->dtype == QSDPA_F16;
  const int gs = a0->group_size, bits = a0->bits;
#define QSDPA_REQUANT_CASE(T, B_, G_)                \
  if (bits == B_ && gs == G_) {                       \
    if (dst16) go(requant_kernel<T, B_, G_, true>);   \
    else go(requant_kernel<T, B_, G_, false>);        \
  }
  if (f16) {
    QSDPA_REQUANT_CASE(F16, 4, 32) QSDPA_REQUANT_CASE(F16, 4, 64) QSDPA_REQUANT_CASE(F16, 4, 128)
    QSDPA_REQUANT_CASE(F16, 8, 32) QSDPA_REQUANT_CASE(F16, 8, 64) QSDPA_REQUANT_CASE(F16, 8, 128)
  } else {
    QSDPA_REQUANT_CASE(BF16, 4, 32) QSDPA_REQUANT_CASE(BF16, 4, 64) QSDPA_REQUANT_CASE(BF16, 4, 128)
    QSDPA_REQUANT_CASE(BF16, 8, 32) QSDPA_REQUANT_CASE(BF16, 8, 64) QSDPA_REQUANT_CASE(BF16, 8, 128)
  }
#undef QSDPA_REQUANT_CASE
  return check_launch("requant");
}

}  // namespace qsdpa
