// Token-row block moves: the device side of the batch caches' administration.
//
// A batch cache holds each sequence as one batch row of (B, H, N, W)
// buffers (packed codes, scales, biases for keys and values).  Filtering,
// stacking, extracting, merging and the right-to-left padding roll only
// relocate whole token rows of those buffers: every operation is a list of
// moves "fill `tokens` rows of row_bytes bytes per head at dst, the rows
// [lo, hi) from src and the others with zeros".  One launch runs up to
// kMovesPerLaunch of them, described in the kernel arguments, so an
// administration step issues no host-to-device copy, no index tensor and no
// synchronization: it is a stream-ordered byte copy.
//
// Mapping: blockIdx.y picks the move, the x dimension strides over its
// heads * tokens * units copy units (unit = the widest of 16/8/4/2/1 bytes
// that every address of the move is aligned to).  Consecutive threads take
// consecutive units of a row and then the next row, so a contiguous token
// range is read and written as one contiguous stream.  HBM-bound: each moved
// byte is read once and written once.
#include "abi_internal.h"

namespace qsdpa {
namespace {

struct Move {
  const unsigned char* src;  // row of token `lo` (null: every row is zeroed)
  unsigned char* dst;        // row of token 0
  long long src_hs, src_ts, dst_hs, dst_ts;  // bytes
  unsigned rows;    // heads * tokens
  unsigned tokens;  // >= 1
  unsigned units;   // units per row
  unsigned shift;   // log2 of the unit size
  unsigned lo, hi;  // tokens [lo, hi) are copied, the others zeroed
};
static_assert(sizeof(Move) == 72, "Move is one 72-byte kernel-argument record");

constexpr int kMovesPerLaunch = 48;
constexpr int kThreads = 256;
constexpr unsigned kMaxUnits = 0x7fffffffu;  // per move and launch: keeps the 32-bit index from wrapping

struct MoveSet {
  Move m[kMovesPerLaunch];
};

template <int SHIFT>
struct Unit;
template <> struct Unit<4> { using T = uint4; };
template <> struct Unit<3> { using T = uint2; };
template <> struct Unit<2> { using T = unsigned; };
template <> struct Unit<1> { using T = unsigned short; };
template <> struct Unit<0> { using T = unsigned char; };

template <int SHIFT>
__device__ __forceinline__ void run_move(const Move& m) {
  using T = typename Unit<SHIFT>::T;
  const unsigned total = m.rows * m.units;
  const unsigned step = gridDim.x * kThreads;
  for (unsigned i = blockIdx.x * kThreads + threadIdx.x; i < total; i += step) {
    const unsigned r = i / m.units, u = i - r * m.units;
    const unsigned h = r / m.tokens, t = r - h * m.tokens;
    T* d = reinterpret_cast<T*>(m.dst + h * m.dst_hs + t * m.dst_ts) + u;
    if (t >= m.lo && t < m.hi) {
      *d = reinterpret_cast<const T*>(m.src + h * m.src_hs + (t - m.lo) * m.src_ts)[u];
    } else {
      T z;
      __builtin_memset(&z, 0, sizeof(T));
      *d = z;
    }
  }
}

__global__ __launch_bounds__(kThreads) void move_rows_kernel(MoveSet s) {
  const Move& m = s.m[blockIdx.y];
  switch (m.shift) {
    case 4: run_move<4>(m); break;
    case 3: run_move<3>(m); break;
    case 2: run_move<2>(m); break;
    case 1: run_move<1>(m); break;
    default: run_move<0>(m); break;
  }
}

// Widest unit (as log2 bytes) that the row size, both base addresses and the
// strides that are actually stepped are multiples of.
unsigned unit_shift(const qsdpa_row_move& mv) {
  for (unsigned sh = 4; sh > 0; --sh) {
    const long long u = 1ll << sh;
    bool ok = mv.row_bytes % u == 0 && reinterpret_cast<uintptr_t>(mv.dst) % u == 0;
    if (mv.heads > 1) ok = ok && mv.dst_head_stride % u == 0;
    if (mv.tokens > 1) ok = ok && mv.dst_token_stride % u == 0;
    if (mv.src) {
      ok = ok && reinterpret_cast<uintptr_t>(mv.src) % u == 0;
      if (mv.heads > 1) ok = ok && mv.src_head_stride % u == 0;
      if (mv.tokens > 1) ok = ok && mv.src_token_stride % u == 0;
    }
    if (ok) return sh;
  }
  return 0;
}

}  // namespace

int launch_move_rows(const qsdpa_row_move* moves, int count, hipStream_t stream) {
  MoveSet set;
  int n = 0;
  unsigned widest = 0;
  auto flush = [&]() -> int {
    if (n == 0) return QSDPA_OK;
    const unsigned blocks = (widest + kThreads - 1) / kThreads;
    const dim3 grid(blocks < 1024 ? blocks : 1024, n);
    hipLaunchKernelGGL(move_rows_kernel, grid, dim3(kThreads), 0, stream, set);
    n = 0;
    widest = 0;
    return check_launch("move_rows");
  };
  for (int i = 0; i < count; ++i) {
    const qsdpa_row_move& mv = moves[i];
    if (mv.heads == 0 || mv.tokens == 0) continue;
    const unsigned sh = unit_shift(mv);
    const unsigned units = static_cast<unsigned>(mv.row_bytes) >> sh;
    // Split a move whose unit count would not fit the kernel's 32-bit index
    // into token ranges that do.
    const unsigned long long per_token = static_cast<unsigned long long>(mv.heads) * units;
    if (per_token > kMaxUnits)
      return fail(QSDPA_ERR_INVALID, "move %d: %d heads x %d bytes per row is too large", i, mv.heads,
                  mv.row_bytes);
    const int chunk = static_cast<int>(kMaxUnits / per_token);
    const int lo = mv.src ? mv.copy_begin : 0, hi = mv.src ? mv.copy_end : 0;
    for (int t0 = 0; t0 < mv.tokens; t0 += chunk) {
      const int tk = mv.tokens - t0 < chunk ? mv.tokens - t0 : chunk;
      // This chunk's tokens [t0, t0 + tk) copy [max(lo, t0), min(hi, t0 + tk)).
      const int clo = lo > t0 ? lo : t0;
      const int chi = hi < t0 + tk ? hi : t0 + tk;
      Move& m = set.m[n];
      m.src = clo < chi ? static_cast<const unsigned char*>(mv.src) + (clo - lo) * mv.src_token_stride
                        : nullptr;
      m.lo = clo < chi ? static_cast<unsigned>(clo - t0) : 0u;
      m.hi = clo < chi ? static_cast<unsigned>(chi - t0) : 0u;
      m.dst = static_cast<unsigned char*>(mv.dst) + t0 * mv.dst_token_stride;
      m.src_hs = mv.src_head_stride;
      m.src_ts = mv.src_token_stride;
      m.dst_hs = mv.dst_head_stride;
      m.dst_ts = mv.dst_token_stride;
      m.rows = static_cast<unsigned>(mv.heads) * static_cast<unsigned>(tk);
      m.tokens = static_cast<unsigned>(tk);
      m.units = units;
      m.shift = sh;
      const unsigned total = m.rows * units;
      if (total > widest) widest = total;
      if (++n == kMovesPerLaunch) {
        const int rc = flush();
        if (rc) return rc;
      }
    }
  }
  return flush();
}

}  // namespace qsdpa
