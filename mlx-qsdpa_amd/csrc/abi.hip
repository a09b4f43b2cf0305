// C-ABI entry points: argument validation (the reference's ValueError set,
// mlx_qsdpa/dispatch.py:42-65, re-checked here so a direct FFI caller gets
// an error code instead of a fault), the split-count heuristic, workspace
// sizing and kernel dispatch.  No entry point allocates, frees or
// synchronizes.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>

#include "abi_internal.h"
#include "common.h"

namespace qsdpa {

static thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(QSDPA_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return QSDPA_OK;
}

// Defined in decode_valu.hip / decode_mfma.hip.
int valu_heads_per_block(int G);
int launch_decode_valu(const qsdpa_decode_args* a, int num_splits, float* part_acc, float* part_ml,
                       hipStream_t stream);
int launch_merge(const qsdpa_decode_args* a, int num_splits, const float* part_acc,
                 const float* part_ml, bool half_parts, const int* sched, int units, hipStream_t stream);
bool mfma_supports(const qsdpa_decode_args* a);
int mfma_num_splits(const qsdpa_decode_args* a, int cus);
int launch_decode_mfma(const qsdpa_decode_args* a, int num_splits, float* part_acc, float* part_ml,
                       int units, int* sched, unsigned* tickets, bool append, hipStream_t stream);
// Defined in prefill_mfma.hip.
bool prefill_supports(const qsdpa_decode_args* a);
int prefill_num_splits(const qsdpa_decode_args* a, int cus);
int launch_prefill_mfma(const qsdpa_decode_args* a, int splits, float* part_acc, float* part_ml,
                        hipStream_t stream);
// Defined in decode_rows32.hip (rows32_supports: abi_internal.h).
int rows32_num_splits(const qsdpa_decode_args* a, int cus);
int launch_decode_rows32(const qsdpa_decode_args* a, int num_splits, float* part_acc, float* part_ml,
                         int units, int* sched, hipStream_t stream);


namespace {

constexpr int kMaxSplits = 1024;

int compute_units() {
  static int cus = 0;
  static std::once_flag once;
  std::call_once(once, [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  });
  return cus;
}

bool valid_dtype(int d) { return d == QSDPA_F16 || d == QSDPA_BF16; }

int check_view(const qsdpa_view& v, const char* name, int align_bytes, int64_t stride_mult,
               bool required) {
  if (!v.ptr) {
    if (required) return fail(QSDPA_ERR_INVALID, "%s: null pointer", name);
    return QSDPA_OK;
  }
  if (!aligned(v.ptr, align_bytes))
    return fail(QSDPA_ERR_INVALID, "%s: pointer not %d-byte aligned", name, align_bytes);
  if (v.stride_b % stride_mult || v.stride_h % stride_mult || v.stride_n % stride_mult)
    return fail(QSDPA_ERR_INVALID, "%s: strides must be multiples of %lld elements", name,
                static_cast<long long>(stride_mult));
  return QSDPA_OK;
}

int validate_decode(const qsdpa_decode_args* a) {
  if (!a) return fail(QSDPA_ERR_INVALID, "null args");
  if (a->B < 1 || a->H_q < 1 || a->H_kv < 1 || a->N < 1)
    return fail(QSDPA_ERR_INVALID, "B, H_q, H_kv, N must be >= 1 (got %d, %d, %d, %d)", a->B,
                a->H_q, a->H_kv, a->N);
  if (a->bits != 4 && a->bits != 8) return fail(QSDPA_ERR_INVALID, "bits must be 4 or 8, got %d", a->bits);
  if (a->D % 32 != 0) return fail(QSDPA_ERR_INVALID, "D must be multiple of 32, got %d", a->D);
  if (a->D != 64 && a->D != 128 && a->D != 256)
    return fail(QSDPA_ERR_UNSUPPORTED, "D=%d not compiled (64, 128, 256)", a->D);
  if (a->group_size != 32 && a->group_size != 64 && a->group_size != 128)
    return fail(QSDPA_ERR_UNSUPPORTED, "group_size=%d not supported (32, 64, 128)", a->group_size);
  if (a->D % a->group_size != 0)
    return fail(QSDPA_ERR_INVALID, "D=%d not a multiple of group_size=%d", a->D, a->group_size);
  if (a->H_q % a->H_kv != 0)
    return fail(QSDPA_ERR_INVALID, "H_q (%d) must be divisible by H_kv (%d)", a->H_q, a->H_kv);
  if (!valid_dtype(a->dtype)) return fail(QSDPA_ERR_INVALID, "dtype must be F16 or BF16");
  if (a->num_splits < 0 || a->num_splits > kMaxSplits)
    return fail(QSDPA_ERR_INVALID, "num_splits must be in [0, %d]", kMaxSplits);
  int rc;
  if ((rc = check_view(a->q, "q", 2, 1, true))) return rc;
  if ((rc = check_view(a->out, "out", 2, 1, true))) return rc;
  if ((rc = check_view(a->k_packed, "k_packed", 16, 4, true))) return rc;
  if ((rc = check_view(a->v_packed, "v_packed", 16, 4, true))) return rc;
  if ((rc = check_view(a->k_scales, "k_scales", 2, 1, true))) return rc;
  if ((rc = check_view(a->v_scales, "v_scales", 2, 1, true))) return rc;
  if ((rc = check_view(a->k_biases, "k_biases", 2, 1, false))) return rc;
  if ((rc = check_view(a->v_biases, "v_biases", 2, 1, false))) return rc;
  if ((a->k_biases.ptr == nullptr) != (a->v_biases.ptr == nullptr))
    return fail(QSDPA_ERR_INVALID, "k_biases and v_biases must both be given or both be NULL");
  if (a->q_len < 0) return fail(QSDPA_ERR_INVALID, "q_len must be >= 0, got %d", a->q_len);
  if (a->q_len > 1 && !mfma_supports(a))
    return fail(QSDPA_ERR_UNSUPPORTED,
                "q_len=%d needs the matrix-core path (D 128 or 256, aligned views); use dequantize + attention",
                a->q_len);
  if (a->mask.ptr) {
    const int md = a->mask_dtype;
    if (md != QSDPA_F16 && md != QSDPA_BF16 && md != QSDPA_F32 && md != QSDPA_BOOL)
      return fail(QSDPA_ERR_INVALID, "mask_dtype %d invalid", md);
    const int al = md == QSDPA_F32 ? 4 : (md == QSDPA_BOOL ? 1 : 2);
    if ((rc = check_view(a->mask, "mask", al, 1, true))) return rc;
  }
  if ((a->k_new.ptr == nullptr) != (a->v_new.ptr == nullptr))
    return fail(QSDPA_ERR_INVALID, "k_new and v_new must both be given or both be NULL");
  if (a->k_new.ptr) {
    if (!a->k_biases.ptr) return fail(QSDPA_ERR_INVALID, "an append writes biases: k_biases / v_biases needed");
    if ((rc = check_view(a->k_new, "k_new", 2, 1, true))) return rc;
    if ((rc = check_view(a->v_new, "v_new", 2, 1, true))) return rc;
  }
  return QSDPA_OK;
}

}  // namespace

namespace {

// Where a split-K call keeps its scratch in the workspace, in bytes from
// its start: the split merge's counters (kTicketBytes, zero between calls),
// the partial rows, their (m, l), and the stream-K schedule.
struct WorkspaceLayout {
  int64_t acc, ml, sched, total;
};

WorkspaceLayout workspace_layout(const qsdpa_decode_args* a, int splits) {
  const int64_t rows = static_cast<int64_t>(a->B) * a->H_q * std::max(a->q_len, 1);
  WorkspaceLayout w;
  w.acc = kTicketBytes;
  w.ml = w.acc + rows * (splits + 1) * a->D * 4;
  w.sched = w.ml + rows * (splits + 1) * 2 * 4;
  w.total = w.sched + ((8LL * a->B + 255) / 256) * 256;
  return w;
}

}  // namespace

// A left-padded batch on the MFMA path runs splits * B equal units of the
// stream-K schedule (common.h) over its sequences laid end to end, instead
// of giving every sequence `splits`; 0 = uniform splits.
int streamk_units(const qsdpa_decode_args* a, int splits) {
  if (!a->kv_start || a->B < 2 || splits < 2 || !mfma_supports(a)) return 0;
  // D = 256, 8-bit codes with a mask tensor: the stream-K instantiation
  // would need more than 256 VGPRs (it spilled to scratch); uniform splits
  // handle kv_start as well.
  if (a->mask.ptr && a->D == 256 && a->bits == 8) return 0;
  const int64_t units = static_cast<int64_t>(splits) * a->B;
  if (units >= (int64_t(1) << 31) / 2) return 0;
  if (static_cast<int64_t>(a->B) * (a->N / kSchedTile + 1) >= (int64_t(1) << 31)) return 0;
  return static_cast<int>(units);
}

// The folded append (k_new / v_new) runs inside the matrix-core decode when
// one block of query rows covers a kv head (so one workgroup reads a
// sequence's key N - 1), the new rows are 16-byte aligned, D = 128 and
// there is no mask tensor (the instantiations built with it); otherwise
// the two rows are quantized by a launch of their own before the decode.
bool fused_append(const qsdpa_decode_args* a, bool prefill, bool mfma) {
  if (!a->k_new.ptr || prefill || !mfma || a->D != 128 || a->mask.ptr) return false;
  const int64_t G = a->H_q / a->H_kv, qL = std::max(a->q_len, 1);
  if (G * qL > 16) return false;
  for (const qsdpa_view* v : {&a->k_new, &a->v_new})
    if (!aligned(v->ptr, 16) || v->stride_b % 8 != 0 || v->stride_h % 8 != 0) return false;
  return true;
}

int launch_append_quantize(const qsdpa_decode_args* a, hipStream_t s) {
  qsdpa_quantize_args j[2] = {};
  for (int i = 0; i < 2; ++i) {
    j[i].B = a->B; j[i].H = a->H_kv; j[i].S = 1; j[i].D = a->D;
    j[i].bits = a->bits; j[i].group_size = a->group_size; j[i].dtype = a->dtype; j[i].t0 = a->N - 1;
    j[i].src = i ? a->v_new : a->k_new;
    j[i].dst_packed = i ? a->v_packed : a->k_packed;
    j[i].dst_scales = i ? a->v_scales : a->k_scales;
    j[i].dst_biases = i ? a->v_biases : a->k_biases;
  }
  const qsdpa_quantize_args* ptrs[2] = {&j[0], &j[1]};
  return launch_quantize(ptrs, 2, s);
}

// A split-K decode on the matrix-core kernel merges its partials inside the
// launch (decode_mfma.hip::split_merge) when its (sequence, kv head, row
// block) units have counters (at most kTicketBlocks of them) and a kv head's
// (stream-K) or a block's (uniform) partial rows span less than 2^31 bytes;
// with uniform splits only up to kFusedSplits of them (above that the merge
// kernel is faster: the last workgroup would read every split alone).  The
// stream-K schedule merges per sequence, over the few segments that cover
// it.  Otherwise the merge kernel combines the partials.
bool fused_merge(const qsdpa_decode_args* a, int splits, bool prefill, bool mfma, int units) {
  if (prefill || !mfma || splits < 2) return false;
  if (rows32_supports(a)) return false;  // the 32-row kernel: the merge kernel
  if (units == 0 && splits > kFusedSplits) return false;
  // D = 256 with 8-bit codes under the stream-K schedule has no such kernel
  // (its registers spilled to scratch).
  if (units > 0 && a->D == 256 && a->bits == 8) return false;
  const int64_t qL = std::max(a->q_len, 1);
  const int64_t G = a->H_q / a->H_kv;
  const int64_t blocks = static_cast<int64_t>(a->B) * a->H_kv * ((G * qL + 15) / 16);
  const int64_t cols = units > 0 ? static_cast<int64_t>(units) + a->B : splits;
  return blocks <= kTicketBlocks && G * qL * cols * a->D * 4 < (int64_t(1) << 31);
}

// Split count: enough workgroups to cover every CU twice, but never fewer
// than 64 keys per split, and no more than kMaxSplits.
int decode_plan(const qsdpa_decode_args* a, int* num_splits, int64_t* workspace_bytes) {
  // Many query positions per kv head: the prefill kernel, with key splits
  // where its row groups alone would leave CUs idle.
  const bool prefill = prefill_supports(a);
  int splits = prefill ? prefill_num_splits(a, compute_units()) : a->num_splits;
  const bool mfma = mfma_supports(a);
  if (splits == 0 && !prefill) {
    if (mfma) {
      splits = rows32_supports(a) ? rows32_num_splits(a, compute_units()) : mfma_num_splits(a, compute_units());
    } else {
      const int G = a->H_q / a->H_kv;
      const int64_t units = static_cast<int64_t>(a->B) * a->H_kv * (G / valu_heads_per_block(G));
      const int64_t target = 2LL * compute_units();
      int64_t s = (target + units - 1) / units;
      const int64_t max_by_len = std::max<int64_t>(1, a->N / 64);
      s = std::min<int64_t>(std::min<int64_t>(s, max_by_len), kMaxSplits);
      splits = static_cast<int>(std::max<int64_t>(s, 1));
    }
  }
  splits = std::min(splits, std::max(1, a->N));
  *num_splits = splits;
  // Partial slots per query row: splits, or splits + 1 columns per sequence
  // (U + B, U = splits * B) under the stream-K schedule of a left-padded
  // batch; then that schedule's (first column, count) per sequence.
  *workspace_bytes = splits > 1 ? workspace_layout(a, splits).total : 0;
  return QSDPA_OK;
}

// Launch the decode for validated arguments: the main kernel, then (split-K)
// the merge, with the partials in `workspace` (decode_plan's layout).
int run_decode(const qsdpa_decode_args* args, int splits, void* workspace, hipStream_t s) {
  // (prof_begin / prof_end ride on the main kernel's own dispatch)
  const bool prefill = prefill_supports(args);
  const bool mfma = mfma_supports(args);
  const int units = prefill ? 0 : streamk_units(args, splits);
  const bool fused = fused_merge(args, splits, prefill, mfma, units);
  float* part_acc = nullptr;
  float* part_ml = nullptr;
  int* sched = nullptr;
  if (splits > 1) {
    const WorkspaceLayout w = workspace_layout(args, splits);
    uint8_t* base = static_cast<uint8_t*>(workspace);
    part_acc = reinterpret_cast<float*>(base + w.acc);
    part_ml = reinterpret_cast<float*>(base + w.ml);
    sched = reinterpret_cast<int*>(base + w.sched);
  }
  int rc;
  const bool append_inside = fused_append(args, prefill, mfma);
  if (args->k_new.ptr && !append_inside && (rc = launch_append_quantize(args, s))) return rc;
  if (prefill) rc = launch_prefill_mfma(args, splits, part_acc, part_ml, s);
  else if (mfma && rows32_supports(args)) rc = launch_decode_rows32(args, splits, part_acc, part_ml, units, sched, s);
  else if (mfma)
    rc = launch_decode_mfma(args, splits, part_acc, part_ml, units, sched,
                            fused ? static_cast<unsigned*>(workspace) : nullptr, append_inside, s);
  else rc = launch_decode_valu(args, splits, part_acc, part_ml, s);
  if (rc) return rc;
  // The MFMA kernels store float16 inputs' partials as normalised float16
  // rows (in the first half of the float32 area).
  if (splits > 1 && !fused)
    rc = launch_merge(args, splits, part_acc, part_ml, mfma && args->dtype == QSDPA_F16, units ? sched : nullptr,
                      units + args->B, s);
  return rc;
}

// Split-K scratch of qsdpa_decode_noalloc: a static device array, one copy
// per GPU, alive until the process ends.  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in): each device's address
// comes from hipGetSymbolAddress on the first call on that device.  Every
// call on one GPU shares that GPU's array, so calls that overlap on one GPU
// (two streams, or two host threads) race on it.  Its first kTicketBytes
// hold the split merge's counters: zero when the code object is loaded (a
// static array without initializer is zero-filled) and zero again after
// every call; every partial a merge reads is written by the same call.
constexpr size_t kScratchBytes = QSDPA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

int scratch_address(void** out) {
  constexpr int kMaxDevices = 64;
  static void* addr[kMaxDevices] = {};
  static std::mutex mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(QSDPA_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(QSDPA_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(QSDPA_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    addr[dev] = p;
  }
  *out = addr[dev];
  return QSDPA_OK;
}

}  // namespace qsdpa

using namespace qsdpa;

extern "C" {

int qsdpa_abi_version(void) { return QSDPA_ABI_VERSION; }

const char* qsdpa_last_error(void) { return g_err; }

int64_t qsdpa_decode_workspace_size(const qsdpa_decode_args* args, int32_t* num_splits_out) {
  clear_error();
  int rc = validate_decode(args);
  if (rc) return rc;
  int splits = 1;
  int64_t ws = 0;
  rc = decode_plan(args, &splits, &ws);
  if (rc) return rc;
  if (num_splits_out) *num_splits_out = splits;
  return ws;
}

int qsdpa_decode(const qsdpa_decode_args* args, void* stream) {
  clear_error();
  int rc = validate_decode(args);
  if (rc) return rc;
  int splits = 1;
  int64_t ws = 0;
  rc = decode_plan(args, &splits, &ws);
  if (rc) return rc;
  if (splits > 1) {
    if (!args->workspace || static_cast<int64_t>(args->workspace_bytes) < ws)
      return fail(QSDPA_ERR_WORKSPACE, "workspace of %lld bytes required, got %lld",
                  static_cast<long long>(ws), static_cast<long long>(args->workspace_bytes));
    if (!aligned(args->workspace, 16)) return fail(QSDPA_ERR_INVALID, "workspace not 16-byte aligned");
  }
  return run_decode(args, splits, args->workspace, static_cast<hipStream_t>(stream));
}

int qsdpa_decode_noalloc(const qsdpa_decode_args* args, void* stream) {
  clear_error();
  int rc = validate_decode(args);
  if (rc) return rc;
  int splits = 1;
  int64_t ws = 0;
  rc = decode_plan(args, &splits, &ws);
  if (rc) return rc;
  void* scratch_ptr = nullptr;
  if (splits > 1) {
    if (ws > static_cast<int64_t>(kScratchBytes))
      return fail(QSDPA_ERR_WORKSPACE,
                  "these arguments need %lld bytes of split-K scratch; the static scratch holds %lld "
                  "(use qsdpa_decode with a workspace, or fewer splits / query rows)",
                  static_cast<long long>(ws), static_cast<long long>(kScratchBytes));
    if ((rc = scratch_address(&scratch_ptr))) return rc;
  }
  return run_decode(args, splits, scratch_ptr, static_cast<hipStream_t>(stream));
}

int qsdpa_quantize(const qsdpa_quantize_args* a, void* stream) {
  return qsdpa_quantize_batch(a, 1, stream);
}

int qsdpa_quantize_batch(const qsdpa_quantize_args* jobs, int32_t count, void* stream) {
  clear_error();
  if (!jobs) return fail(QSDPA_ERR_INVALID, "null args");
  if (count < 1 || count > 4) return fail(QSDPA_ERR_INVALID, "count must be in [1, 4], got %d", count);
  for (int i = 1; i < count; ++i)
    if (jobs[i].bits != jobs[0].bits || jobs[i].group_size != jobs[0].group_size || jobs[i].dtype != jobs[0].dtype)
      return fail(QSDPA_ERR_INVALID, "quantize jobs of one call must share bits, group_size and dtype");
  const qsdpa_quantize_args* ptrs[4];
  for (int i = 0; i < count; ++i) {
    const qsdpa_quantize_args* a = jobs + i;
    if (a->bits != 4 && a->bits != 8) return fail(QSDPA_ERR_INVALID, "bits must be 4 or 8, got %d", a->bits);
    if (a->group_size != 32 && a->group_size != 64 && a->group_size != 128)
      return fail(QSDPA_ERR_UNSUPPORTED, "group_size=%d not supported (32, 64, 128)", a->group_size);
    if (a->B < 0 || a->H < 0 || a->S < 0 || a->D <= 0 || a->D % a->group_size != 0)
      return fail(QSDPA_ERR_INVALID, "bad shape B=%d H=%d S=%d D=%d gs=%d", a->B, a->H, a->S, a->D,
                  a->group_size);
    if (a->t0 < 0) return fail(QSDPA_ERR_INVALID, "t0 must be >= 0");
    if (!valid_dtype(a->dtype)) return fail(QSDPA_ERR_INVALID, "dtype must be F16 or BF16");
    int rc;
    if ((rc = check_view(a->src, "src", 2, 1, true))) return rc;
    if ((rc = check_view(a->dst_packed, "dst_packed", 4, 1, true))) return rc;
    if ((rc = check_view(a->dst_scales, "dst_scales", 2, 1, true))) return rc;
    if ((rc = check_view(a->dst_biases, "dst_biases", 2, 1, true))) return rc;
    ptrs[i] = a;
  }
  return launch_quantize(ptrs, count, static_cast<hipStream_t>(stream));
}

int qsdpa_requant_window(const qsdpa_requant_args* jobs, int32_t count, void* stream) {
  clear_error();
  if (!jobs) return fail(QSDPA_ERR_INVALID, "null args");
  if (count < 1 || count > 2) return fail(QSDPA_ERR_INVALID, "count must be 1 or 2, got %d", count);
  for (int i = 1; i < count; ++i)
    if (jobs[i].bits != jobs[0].bits || jobs[i].group_size != jobs[0].group_size || jobs[i].dtype != jobs[0].dtype ||
        jobs[i].B != jobs[0].B || jobs[i].H != jobs[0].H)
      return fail(QSDPA_ERR_INVALID, "requant jobs of one call must share B, H, bits, group_size and dtype");
  const qsdpa_requant_args* ptrs[2];
  for (int i = 0; i < count; ++i) {
    const qsdpa_requant_args* a = jobs + i;
    if (a->bits != 4 && a->bits != 8) return fail(QSDPA_ERR_INVALID, "bits must be 4 or 8, got %d", a->bits);
    if (a->group_size != 32 && a->group_size != 64 && a->group_size != 128)
      return fail(QSDPA_ERR_UNSUPPORTED, "group_size=%d not supported (32, 64, 128)", a->group_size);
    if (!valid_dtype(a->dtype)) return fail(QSDPA_ERR_INVALID, "dtype must be F16 or BF16");
    if (a->B < 0 || a->H < 0 || a->D <= 0 || a->D % a->group_size != 0)
      return fail(QSDPA_ERR_INVALID, "bad shape B=%d H=%d D=%d gs=%d", a->B, a->H, a->D, a->group_size);
    if (a->max_size < 1 || a->keep < 0 || a->keep >= a->max_size || a->n_old < 0 || a->n_old > a->max_size ||
        a->S < 0 || a->rot < 0 || (a->rot > 0 && a->n_old <= a->keep))
      return fail(QSDPA_ERR_INVALID, "bad window (max_size=%d keep=%d n_old=%d S=%d rot=%d)", a->max_size,
                  a->keep, a->n_old, a->S, a->rot);
    int rc;
    const bool old = a->n_old > 0, add = a->S > 0;
    if ((rc = check_view(a->old_packed, "old_packed", 4, 1, old))) return rc;
    if ((rc = check_view(a->old_scales, "old_scales", 2, 1, old))) return rc;
    if ((rc = check_view(a->old_biases, "old_biases", 2, 1, false))) return rc;
    if ((rc = check_view(a->src, "src", 2, 1, add))) return rc;
    if ((rc = check_view(a->dst_packed, "dst_packed", 4, 1, true))) return rc;
    if ((rc = check_view(a->dst_scales, "dst_scales", 2, 1, true))) return rc;
    if ((rc = check_view(a->dst_biases, "dst_biases", 2, 1, true))) return rc;
    if (a->old_packed.ptr && a->old_packed.ptr == a->dst_packed.ptr)
      return fail(QSDPA_ERR_INVALID, "the destination must not be the old window");
    ptrs[i] = a;
  }
  return launch_requant(ptrs, count, static_cast<hipStream_t>(stream));
}

int qsdpa_move_rows(const qsdpa_row_move* moves, int32_t count, void* stream) {
  clear_error();
  if (count < 0) return fail(QSDPA_ERR_INVALID, "count must be >= 0, got %d", count);
  if (count > 0 && !moves) return fail(QSDPA_ERR_INVALID, "null moves");
  for (int i = 0; i < count; ++i) {
    const qsdpa_row_move& m = moves[i];
    if (m.heads < 0 || m.tokens < 0 || m.row_bytes < 1)
      return fail(QSDPA_ERR_INVALID, "move %d: heads=%d tokens=%d row_bytes=%d", i, m.heads, m.tokens,
                  m.row_bytes);
    if (m.src_head_stride < 0 || m.src_token_stride < 0 || m.dst_head_stride < 0 || m.dst_token_stride < 0)
      return fail(QSDPA_ERR_INVALID, "move %d: negative stride", i);
    if (m.src && (m.copy_begin < 0 || m.copy_begin > m.copy_end || m.copy_end > m.tokens))
      return fail(QSDPA_ERR_INVALID, "move %d: copy range [%d, %d) outside [0, %d)", i, m.copy_begin,
                  m.copy_end, m.tokens);
    if (m.heads > 0 && m.tokens > 0 && !m.dst) return fail(QSDPA_ERR_INVALID, "move %d: null dst", i);
  }
  return launch_move_rows(moves, count, static_cast<hipStream_t>(stream));
}

int qsdpa_dequantize(const qsdpa_dequantize_args* a, void* stream) {
  clear_error();
  if (!a) return fail(QSDPA_ERR_INVALID, "null args");
  if (a->bits != 4 && a->bits != 8) return fail(QSDPA_ERR_INVALID, "bits must be 4 or 8, got %d", a->bits);
  if (a->group_size != 32 && a->group_size != 64 && a->group_size != 128)
    return fail(QSDPA_ERR_UNSUPPORTED, "group_size=%d not supported (32, 64, 128)", a->group_size);
  if (a->B < 0 || a->H < 0 || a->N < 0 || a->D <= 0 || a->D % a->group_size != 0)
    return fail(QSDPA_ERR_INVALID, "bad shape B=%d H=%d N=%d D=%d gs=%d", a->B, a->H, a->N, a->D,
                a->group_size);
  if (a->keep < 0 || a->rot < 0 || (a->N > 0 && a->keep >= a->N && a->rot > 0))
    return fail(QSDPA_ERR_INVALID, "bad keep/rot (keep=%d rot=%d N=%d)", a->keep, a->rot, a->N);
  if (!valid_dtype(a->dtype)) return fail(QSDPA_ERR_INVALID, "dtype must be F16 or BF16");
  int rc;
  if ((rc = check_view(a->src_packed, "src_packed", 4, 1, true))) return rc;
  if ((rc = check_view(a->src_scales, "src_scales", 2, 1, true))) return rc;
  if ((rc = check_view(a->src_biases, "src_biases", 2, 1, false))) return rc;
  if ((rc = check_view(a->dst, "dst", 2, 1, true))) return rc;
  return launch_dequantize(a, static_cast<hipStream_t>(stream));
}

}  // extern "C"
