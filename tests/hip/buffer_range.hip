// TEST INFRASTRUCTURE: a check of the hardware behaviour the decode and
// prefill kernels rely on, not product code.
//
// The kernels address the rows of a tile through a raw buffer load's scalar
// offset (soffset) and rely on the descriptor's range check to return zero
// for every row past the sequence (partial last tiles, the pipeline's
// prefetch past the end).  This kernel reads one buffer of num_records =
// 4096 bytes at offsets below, at and past its end, once with the offset in
// the per-lane voffset and once in the scalar soffset; every address it
// forms lies inside the caller's 64 KiB allocation, so no access can fault
// whether or not the range check includes soffset.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kRecords = 4096;  // bytes the descriptor covers

__global__ __launch_bounds__(64) void buffer_range_kernel(const uint32_t* base, uint32_t* out) {
  const int lane = threadIdx.x;
  __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(base), 0, kRecords, 0x00020000);
  const int offs[5] = {0, 2048, 3968, 4096, 8192};
  for (int i = 0; i < 5; ++i) {
    out[(2 * i) * 64 + lane] = __builtin_amdgcn_raw_buffer_load_b32(rs, lane * 4 + offs[i], 0, 0);
    out[(2 * i + 1) * 64 + lane] = __builtin_amdgcn_raw_buffer_load_b32(rs, lane * 4, offs[i], 0);
  }
}

}  // namespace

// base: >= 64 KiB of device memory; out: 10 x 64 words.  Row 2i holds the
// loads with offset offs[i] in voffset, row 2i + 1 the same with it in
// soffset.  Returns the launch's hipError_t.
extern "C" int buffer_range_probe(const uint32_t* base, uint32_t* out, void* stream) {
  hipLaunchKernelGGL(buffer_range_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), base, out);
  return static_cast<int>(hipGetLastError());
}
