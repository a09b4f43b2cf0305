/*
 * qsdpa.h -- C ABI of the MI355X (gfx950) fused quantized SDPA decode library.
 *
 * Everything crossing this boundary is a plain C type: device pointers,
 * 64-bit element strides, int32 shape fields and an opaque stream handle
 * (a hipStream_t passed as void*; NULL = the null stream).  The library never
 * allocates or frees caller memory, keeps no pointer after a call returns and
 * never throws.  Every entry point returns QSDPA_OK (0) or a negative
 * QSDPA_ERR_* code; qsdpa_last_error() then holds a thread-local message.
 * All launches are stream-ordered; no entry point synchronizes the device.
 *
 * Data format (the MLX affine format of mx.quantize, bits in {4, 8}):
 *   packed : uint32 [.., N, D*bits/32]; element j of a word occupies bits
 *            [j*bits, (j+1)*bits), element index d = word*(32/bits) + j
 *            (reference: mlx_qsdpa/kernels.py:101-105).
 *   scales, biases : T [.., N, D/group_size], T in {fp16, bf16}; the value
 *            of element d of a token is scale[g]*q[d] + bias[g], g=d/group_size.
 *
 * Reference interfaces replaced (paths relative to the mlx-qsdpa repo):
 *   qsdpa_decode     <- the three mx.fast.metal_kernel launches of
 *                       mlx_qsdpa/dispatch.py:158-171 (single pass, kernel
 *                       built at kernels.py:182-191) and dispatch.py:225-265
 *                       (split-K pass 1 + pass 2, kernels.py:452-473).
 *   qsdpa_quantize   <- mx.quantize(keys, group_size, bits) followed by the
 *                       slice assignment into the cache buffers
 *                       (mlx_qsdpa/cache.py:186-192, 314-318, 576-581,
 *                       610-614, 798-804, 830-834).
 *   qsdpa_quantize_batch <- the key and value mx.quantize pair of one
 *                       update_and_fetch (same call sites), in one launch.
 *   qsdpa_dequantize <- mx.dequantize(...) (mlx_qsdpa/dispatch.py:69-78,
 *                       mlx_qsdpa/__init__.py:50-57) and the dequantize +
 *                       temporal reorder of cache.py:622-634, 842-857.
 *   qsdpa_requant_window <- the rotating prefill's dequantize + concatenate
 *                       + trim + quantize (cache.py:593-634, 813-857).
 *   qsdpa_move_rows  <- the batch caches' slicing / padding / concatenation
 *                       (cache.py:46-51, 337-348, 378-492, 868-1010).
 */
#ifndef QSDPA_H_
#define QSDPA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QSDPA_ABI_VERSION 6

enum {
  QSDPA_OK = 0,
  QSDPA_ERR_INVALID = -1,     /* bad argument (shape, stride, pointer) */
  QSDPA_ERR_UNSUPPORTED = -2, /* valid but not compiled (e.g. D=96)    */
  QSDPA_ERR_WORKSPACE = -3,   /* workspace missing or too small        */
  QSDPA_ERR_LAUNCH = -4       /* HIP launch error                      */
};

/* Element types. */
enum {
  QSDPA_F16 = 0,
  QSDPA_BF16 = 1,
  QSDPA_F32 = 2,
  QSDPA_BOOL = 3 /* one byte per element, nonzero = attend */
};

/*
 * A strided view of a 4-D tensor [B, H, N, inner] whose innermost dimension
 * is contiguous.  Strides are in ELEMENTS of the tensor's own type.  A stride
 * of 0 broadcasts that dimension.  ptr == NULL means "absent".
 */
typedef struct {
  const void* ptr;
  int64_t stride_b;
  int64_t stride_h;
  int64_t stride_n;
} qsdpa_view;

/*
 * Decode attention: out[b, h, i, :] = softmax(scale * q[b,h,i] . K[b, h/G]^T
 * + mask) V[b, h/G] with G = H_q / H_kv, K/V dequantized on the fly, for
 * the q_len query positions i (1 for a decode step; more for speculative
 * or chunked decoding and prefill).
 */
typedef struct {
  int32_t B, H_q, H_kv, N, D;
  int32_t bits;       /* 4 or 8 */
  int32_t group_size; /* 32, 64 or 128 */
  int32_t dtype;      /* QSDPA_F16 or QSDPA_BF16: q, scales, biases, out */
  float scale;        /* softmax scale applied to q.k */

  qsdpa_view q;        /* [B, H_q, q_len, D]  (stride_n: query position) */
  qsdpa_view k_packed; /* [B, H_kv, N, D*bits/32] uint32                 */
  qsdpa_view v_packed;
  qsdpa_view k_scales; /* [B, H_kv, N, D/group_size] dtype               */
  qsdpa_view v_scales;
  qsdpa_view k_biases; /* ptr NULL => zero biases (symmetric format)     */
  qsdpa_view v_biases;
  qsdpa_view out;      /* [B, H_q, q_len, D] dtype (stride_n: position)  */

  /* Optional mask over keys, broadcastable [B|1, H_q|1, q_len|1, N]: a
   * stride of 0 broadcasts; stride_n is the KEY stride and mask_stride_q
   * (below) the query-position stride.  QSDPA_BOOL: nonzero keeps the key;
   * QSDPA_F16/BF16/F32: additive (added to the scaled score).  ptr NULL =
   * no mask.                                                              */
  qsdpa_view mask;
  int32_t mask_dtype;

  /* Optional int32 [B]: keys with index < kv_start[b] are skipped (never
   * read).  Expresses left padding without a mask.  NULL = all keys.      */
  const int32_t* kv_start;

  /* 0 = choose automatically, 1 = single pass, >1 = split-K with this many
   * splits per (batch, kv head).  With kv_start and B > 1 (D in {128, 256})
   * the count is an average: the batch's keys per kv head are cut into
   * num_splits * B equal runs of tiles over the sequences laid end to end
   * (a run may cross sequences; a sequence with no keys gets none).       */
  int32_t num_splits;

  /* Scratch for split-K partials, from qsdpa_decode_workspace_size().
   * Its first 64 KiB hold the counters of the split merge that runs inside
   * the decode launch: zero-fill a workspace before its first use; every
   * call leaves them zero again, so a workspace can be re-used by later
   * calls (in stream order) of any shape.                                 */
  void* workspace;
  size_t workspace_bytes;

  /* Optional profiling hook: two hipEvent_t handles (or NULL).  When set,
   * the main decode kernel is launched with hipExtLaunchKernel carrying
   * them as its start / stop events, so hipEventElapsedTime(prof_begin,
   * prof_end) is that kernel's own execution time (any merge kernel runs
   * after prof_end).                                                     */
  void* prof_begin;
  void* prof_end;

  /* Query positions per (batch, head); 0 or 1 = one (a decode step).
   * q_len > 1 needs D in {128, 256} and the alignment of the matrix-core
   * path (else QSDPA_ERR_UNSUPPORTED); mlx_qsdpa's dispatch.py:68-83 sends
   * such calls through dequantize + attention instead.                    */
  int32_t q_len;
  /* Nonzero: causal, aligned to the last key (mask="causal" of the
   * reference): query i sees keys t <= N - q_len + i.  Combines with mask
   * and kv_start.                                                         */
  int32_t causal;
  int64_t mask_stride_q; /* mask stride over query positions (0 = broadcast) */

  /* Optional quantize-on-append folded into the decode: the one-token
   * update of a cache (update_and_fetch, mlx_qsdpa/cache.py:279-322, whose
   * mx.quantize + slice assignment qsdpa_quantize replaces) and the decode
   * over the updated cache in one call.  k_new / v_new: [B, H_kv, 1, D]
   * dtype.  When set (both), the call first quantizes k_new[b, h, 0] and
   * v_new[b, h, 0] into key N - 1 of the K / V views -- codes, scales and
   * biases, exactly as qsdpa_quantize with t0 = N - 1 would; the views must
   * be writable and carry biases -- then attends over all N keys.  On the
   * matrix-core path with one block of query rows per kv head (H_q / H_kv *
   * q_len <= 16) the workgroup that reads key N - 1 writes it first (no
   * extra launch); otherwise a quantize launch precedes the decode.  ptr
   * NULL (both) = no append.                                              */
  qsdpa_view k_new;
  qsdpa_view v_new;
} qsdpa_decode_args;

/* Bytes of workspace qsdpa_decode needs for these args (0 for a single
 * pass).  If num_splits_out is not NULL it receives the split count that
 * qsdpa_decode will use.  Returns a negative QSDPA_ERR_* on bad args.     */
int64_t qsdpa_decode_workspace_size(const qsdpa_decode_args* args,
                                    int32_t* num_splits_out);

/* Launch the decode on `stream`. */
int qsdpa_decode(const qsdpa_decode_args* args, void* stream);

/*
 * qsdpa_decode without a caller workspace: no counterpart in the reference.
 * For callers that cannot allocate -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Same arguments and
 * results as qsdpa_decode, except that args->workspace / workspace_bytes are
 * ignored: the split-K partials live in a static device array of
 * QSDPA_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends.
 * Arguments whose partials need more (qsdpa_decode_workspace_size) return
 * QSDPA_ERR_WORKSPACE.  The call allocates and frees nothing (the first
 * call on a device looks the array's address up).  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two
 * host threads) race and must be serialised by the caller.
 */
#define QSDPA_NOALLOC_SCRATCH_BYTES (16u << 20)
int qsdpa_decode_noalloc(const qsdpa_decode_args* args, void* stream);

/*
 * Quantize rows of T values into the affine format and store them at token
 * positions [t0, t0 + S) of the destination buffers:
 *   dst[b, h, t0 + s, :] = quantize(src[b, h, s, :]).
 * The per-group rule is the contract restated in oracle/affine.py.
 */
typedef struct {
  int32_t B, H, S, D;
  int32_t bits, group_size, dtype;
  int32_t t0;              /* first destination token index            */
  qsdpa_view src;          /* [B, H, S, D] dtype                        */
  qsdpa_view dst_packed;   /* [B, H, cap, D*bits/32] uint32 (writable)  */
  qsdpa_view dst_scales;   /* [B, H, cap, D/group_size] dtype           */
  qsdpa_view dst_biases;   /* [B, H, cap, D/group_size] dtype           */
} qsdpa_quantize_args;

int qsdpa_quantize(const qsdpa_quantize_args* args, void* stream);

/*
 * `count` (1..4) quantize jobs in one launch, e.g. the keys and the values
 * of one cache update (the mx.quantize pair of update_and_fetch,
 * mlx_qsdpa/cache.py:186-192, 314-318, 576-581, 610-614).  The jobs share
 * bits, group_size and dtype; shapes and destinations are their own.
 * qsdpa_quantize(args, s) is qsdpa_quantize_batch(args, 1, s).
 */
int qsdpa_quantize_batch(const qsdpa_quantize_args* jobs, int32_t count, void* stream);

/*
 * Dequantize N tokens to T:  dst[b, h, t, :] = dequant(src[b, h, u(t), :])
 * with u(t) = t for t < keep, else keep + (t - keep + rot) % (N - keep).
 * rot = 0 is a plain dequantize; rot > 0 turns a ring buffer whose oldest
 * ring slot is keep + rot into temporal order.  Each element is
 * round_to_T(fmaf(scale, q, bias)).  Biases may be absent (zero).
 */
typedef struct {
  int32_t B, H, N, D;
  int32_t bits, group_size, dtype;
  int32_t keep, rot;
  qsdpa_view src_packed;
  qsdpa_view src_scales;
  qsdpa_view src_biases;
  qsdpa_view dst;          /* [B, H, N, D] dtype (writable) */
} qsdpa_dequantize_args;

int qsdpa_dequantize(const qsdpa_dequantize_args* args, void* stream);

/*
 * Rotating-window prefill in one launch per call (K and V: count = 2):
 * the window's old tokens in temporal order, then the S new tokens; when
 * there are more than max_size, the first `keep` and the newest
 * max_size - keep are kept; all of them are quantized again into rows
 * [0, total) of the destination, total = min(n_old + S, max_size).
 *   old token c (temporal position c < n_old) is old row u(c) = c for
 *   c < keep or rot == 0, else keep + (c - keep + rot) % (n_old - keep),
 *   dequantized as qsdpa_dequantize does (T(fmaf(scale, q, bias)));
 *   new token i is src row i;
 *   each kept row is quantized as qsdpa_quantize does.
 * The destination must not overlap the old window.  The jobs of one call
 * share B, H, bits, group_size and dtype.  Every view's rows within one
 * (batch, head) must span fewer than 2^31 elements (offsets there are
 * 32-bit; QSDPA_ERR_UNSUPPORTED otherwise), and its strides must not be
 * negative.
 * Replaces the dequantize + concatenate + trim + quantize of
 * mlx_qsdpa/cache.py:593-634 (QuantizedRotatingSDPACache._update_prefill,
 * _dequant_temporal) and cache.py:813-857 (the batched cache's).
 */
typedef struct {
  int32_t B, H, D;
  int32_t bits, group_size, dtype;
  int32_t n_old;            /* tokens in the old window (may be 0)        */
  int32_t keep, rot;        /* the old window's ring order (see above)    */
  int32_t S;                /* new tokens                                 */
  int32_t max_size;         /* window size                                */
  qsdpa_view old_packed;    /* [B, H, >= n_old, D*bits/32] uint32         */
  qsdpa_view old_scales;    /* [B, H, >= n_old, D/group_size] dtype       */
  qsdpa_view old_biases;    /* ptr NULL => zero biases                    */
  qsdpa_view src;           /* [B, H, S, D] dtype                         */
  qsdpa_view dst_packed;    /* [B, H, >= total, D*bits/32] (writable)     */
  qsdpa_view dst_scales;
  qsdpa_view dst_biases;
} qsdpa_requant_args;

int qsdpa_requant_window(const qsdpa_requant_args* jobs, int32_t count, void* stream);

/*
 * Token-row block moves, the device side of the batch caches'
 * administration (filter, extend, extract, merge, the finalize roll).
 * One move fills `tokens` token rows of row_bytes bytes for every head
 * h < heads: row t (dst + h*dst_head_stride + t*dst_token_stride) receives
 *     src + h*src_head_stride + (t - copy_begin)*src_token_stride
 * for copy_begin <= t < copy_end, and zero bytes otherwise (all rows when
 * src is NULL).  Strides are in bytes.  The moves of one call go to
 * the device in kernel arguments (48 per launch): no device memory, no copy
 * before the launch, no synchronization.  Moves of one call may run in any
 * order and concurrently: no destination may overlap another destination
 * or any source of the same call.
 * Replaces the MLX gathers, slices, mx.pad / mx.concatenate and
 * _dynamic_roll of mlx_qsdpa/cache.py:46-51, 337-348 (finalize), 378-492
 * (filter, extend, extract, merge) and 868-1010 (the rotating batch's).
 */
typedef struct {
  const void* src;          /* row of token copy_begin, head 0; NULL => zeros */
  void* dst;                /* row of token 0, head 0                         */
  int64_t src_head_stride, src_token_stride;   /* bytes, >= 0                 */
  int64_t dst_head_stride, dst_token_stride;   /* bytes, >= 0                 */
  int32_t heads, tokens;    /* >= 0                                           */
  int32_t row_bytes;        /* >= 1                                           */
  int32_t copy_begin, copy_end; /* 0 <= copy_begin <= copy_end <= tokens      */
} qsdpa_row_move;

int qsdpa_move_rows(const qsdpa_row_move* moves, int32_t count, void* stream);

/* Thread-local message describing the last error ("" if none). */
const char* qsdpa_last_error(void);

/* QSDPA_ABI_VERSION of the loaded library. */
int qsdpa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* QSDPA_H_ */
