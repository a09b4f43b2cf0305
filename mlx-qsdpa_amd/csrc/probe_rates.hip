// VALU issue-rate probe (a build with -DQSDPA_TIMELINE only; the default
// build has none of it).  Each kernel runs one instruction, through inline
// assembly so that it is exactly that instruction, in 8 independent chains
// per lane; with 8 waves per SIMD the launch time over the instructions
// issued per SIMD is the instruction's issue interval.  The instructions are
// those of the dequantization and the softmax of the attention kernels.
#ifdef QSDPA_TIMELINE
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qsdpa {
namespace {

#define QSDPA_RATE_KERNEL(NAME, ASM)                                                                  \
  __global__ __launch_bounds__(256) void NAME(uint32_t* sink, int iters, uint32_t a, uint32_t b) {     \
    uint32_t x[8];                                                                                  \
    for (int i = 0; i < 8; ++i) x[i] = 0x3f800000u + threadIdx.x * 8 + i;                          \
    for (int it = 0; it < iters; ++it) {                                                            \
      _Pragma("unroll") for (int i = 0; i < 8; ++i) asm volatile(ASM : "+v"(x[i]) : "v"(a), "v"(b)); \
    }                                                                                               \
    uint32_t s = 0;                                                                                 \
    for (int i = 0; i < 8; ++i) s ^= x[i];                                                          \
    sink[blockIdx.x * 256 + threadIdx.x] = s;                                                       \
  }

QSDPA_RATE_KERNEL(rate_fma, "v_fma_f32 %0, %0, %1, %2")
QSDPA_RATE_KERNEL(rate_mul, "v_mul_f32 %0, %0, %1")
QSDPA_RATE_KERNEL(rate_add_f32, "v_add_f32 %0, %0, %1")
QSDPA_RATE_KERNEL(rate_add_u32, "v_add_u32 %0, %0, %1")
QSDPA_RATE_KERNEL(rate_and, "v_and_b32 %0, %0, %1")
QSDPA_RATE_KERNEL(rate_bitop3, "v_bitop3_b32 %0, %0, %1, %2 bitop3:0xea")
QSDPA_RATE_KERNEL(rate_lshl, "v_lshlrev_b32 %0, 16, %0")
QSDPA_RATE_KERNEL(rate_perm, "v_perm_b32 %0, %0, %1, %2")
QSDPA_RATE_KERNEL(rate_cvt_ubyte, "v_cvt_f32_ubyte0 %0, %0")
QSDPA_RATE_KERNEL(rate_cvt_pk_bf16, "v_cvt_pk_bf16_f32 %0, %0, %1")
QSDPA_RATE_KERNEL(rate_cvt_pk_f16, "v_cvt_pk_f16_f32 %0, %0, %1")
QSDPA_RATE_KERNEL(rate_fma_mix, "v_fma_mix_f32 %0, %0, %1, %2 op_sel_hi:[1,0,0]")
QSDPA_RATE_KERNEL(rate_pk_fma_f16, "v_pk_fma_f16 %0, %0, %1, %2")
QSDPA_RATE_KERNEL(rate_pk_add_f16, "v_pk_add_f16 %0, %0, %1")
QSDPA_RATE_KERNEL(rate_max3, "v_max3_f32 %0, %0, %1, %2")
QSDPA_RATE_KERNEL(rate_dot2_bf16, "v_dot2c_f32_bf16 %0, %1, %2")
QSDPA_RATE_KERNEL(rate_mul_lo, "v_mul_lo_u32 %0, %0, %1")
QSDPA_RATE_KERNEL(rate_exp, "v_exp_f32 %0, %0")
QSDPA_RATE_KERNEL(rate_rcp, "v_rcp_f32 %0, %0")
#undef QSDPA_RATE_KERNEL

typedef void (*RateKernel)(uint32_t*, int, uint32_t, uint32_t);
struct RateEntry {
  const char* name;
  RateKernel fn;
};
const RateEntry kRates[] = {
    {"v_fma_f32", rate_fma},           {"v_mul_f32", rate_mul},
    {"v_add_f32", rate_add_f32},       {"v_add_u32", rate_add_u32},
    {"v_and_b32", rate_and},           {"v_bitop3_b32", rate_bitop3},
    {"v_lshlrev_b32", rate_lshl},      {"v_perm_b32", rate_perm},
    {"v_cvt_f32_ubyte0", rate_cvt_ubyte}, {"v_cvt_pk_bf16_f32", rate_cvt_pk_bf16},
    {"v_cvt_pk_f16_f32", rate_cvt_pk_f16}, {"v_fma_mix_f32", rate_fma_mix},
    {"v_pk_fma_f16", rate_pk_fma_f16}, {"v_pk_add_f16", rate_pk_add_f16},
    {"v_max3_f32", rate_max3},         {"v_dot2c_f32_bf16", rate_dot2_bf16},
    {"v_mul_lo_u32", rate_mul_lo},     {"v_exp_f32", rate_exp},
    {"v_rcp_f32", rate_rcp},
};
constexpr int kNumRates = sizeof(kRates) / sizeof(kRates[0]);

}  // namespace
}  // namespace qsdpa

// Number of probed instructions, and the name of probe `which` (null past the end).
extern "C" int qsdpa_debug_valu_rate_count() { return qsdpa::kNumRates; }
extern "C" const char* qsdpa_debug_valu_rate_name(int which) {
  return which >= 0 && which < qsdpa::kNumRates ? qsdpa::kRates[which].name : nullptr;
}

// Launch probe `which` on `blocks` workgroups of 256 threads (sink: blocks *
// 256 uint32), between the two events when given.
extern "C" int qsdpa_debug_valu_rate(int which, int blocks, int iters, void* sink, void* stream, void* ev_begin,
                                     void* ev_end) {
  if (which < 0 || which >= qsdpa::kNumRates || blocks < 1 || iters < 1 || !sink) return -1;
  hipExtLaunchKernelGGL(qsdpa::kRates[which].fn, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                        static_cast<hipEvent_t>(ev_begin), static_cast<hipEvent_t>(ev_end), 0,
                        static_cast<uint32_t*>(sink), iters, 0x3f000000u, 0x3e800000u);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
#endif
