// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/qsdpa.h"

namespace qsdpa {

// Record a thread-local error message and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Map hipGetLastError() after a launch to QSDPA_OK / QSDPA_ERR_LAUNCH.
int check_launch(const char* what);

// The decode workspace starts with the split merge's counters: kTicketWords
// uint32 per block of 16 query rows (batch, kv head, row block), for at
// most kTicketBlocks blocks.  They must be zero before a workspace's first
// use, and every call leaves them zero.
constexpr int kTicketWords = 32;
constexpr int kTicketBlocks = 512;
constexpr int64_t kTicketBytes = int64_t(kTicketWords) * kTicketBlocks * 4;
// Most splits a matrix-core decode launch merges itself (one level, the
// last workgroup of a block: decode_mfma.hip::split_merge); more splits go
// to the merge kernel.
constexpr int kFusedSplits = 16;

inline bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

// Launch a one-argument kernel.  With profiling events (either non-null) the
// launch goes through hipExtLaunchKernel, which attaches the events to the
// kernel's own dispatch: their elapsed time is the kernel's execution time,
// with no marker packets queued before or after it.
template <typename P>
void launch_profiled(void (*kernel)(P), dim3 grid, dim3 block, hipStream_t stream, void* ev_begin,
                     void* ev_end, const P& p) {
  if (ev_begin || ev_end)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, static_cast<hipEvent_t>(ev_begin),
                          static_cast<hipEvent_t>(ev_end), 0, p);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, p);
}

// Launch hooks implemented in the kernel translation units.
int launch_quantize(const qsdpa_quantize_args* const* jobs, int count, hipStream_t stream);
int launch_dequantize(const qsdpa_dequantize_args* a, hipStream_t stream);
int launch_requant(const qsdpa_requant_args* const* jobs, int count, hipStream_t stream);
int launch_move_rows(const qsdpa_row_move* moves, int count, hipStream_t stream);
int launch_decode(const qsdpa_decode_args* a, int num_splits, hipStream_t stream);
int decode_plan(const qsdpa_decode_args* a, int* num_splits, int64_t* workspace_bytes);
// Whether the 32-row decode kernel (decode_rows32.hip) takes a call; the
// prefill kernel's routing defers to it for single row groups.
bool rows32_supports(const qsdpa_decode_args* a);

}  // namespace qsdpa
