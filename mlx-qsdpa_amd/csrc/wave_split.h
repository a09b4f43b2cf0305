// How a decode split's key tiles are laid out (super-tiles) and how the 8
// waves of a decode workgroup share the split's J tile positions
// (decode_mfma.hip).  Plain C++ as well as device code, so that a host
// program can check the invariants the kernel relies on: every tile of a
// sequence belongs to exactly one split position, and every position in
// [0, J) is visited by exactly one wave.
//
// Positions below J - E go round-robin to the 8 waves; the last E go to
// waves 0-3 only.  Waves 4-7 share their SIMDs with waves 0-3, and the older
// waves' loads are served first, so equal shares would leave 0-3 idle at the
// end.  D = 256 (HBM-bound): E = 8 (J / 16), three tiles for waves 0-3 for
// every one of 4-7; D = 128 (VALU-bound): E = 8 (J / 32), five for three.
// Every wave's first position (its index) must lie in the round-robin part
// (J - E >= 8 whenever E > 0), or the waves' position sequences would
// overlap; E is 0 otherwise.
#pragma once

#if defined(__HIPCC__)
#define QSDPA_HD __host__ __device__ __forceinline__
#else
#define QSDPA_HD inline
#endif

namespace qsdpa {

constexpr int kSplitWaves = 8;

// Positions [0, J8) are round-robin; [J8, J) belong to waves 0-3.
QSDPA_HD int wave_split_rr_end(int J, int D) {
  const int E0 = D == 256 ? 8 * (J / 16) : 8 * (J / 32);
  const int E = J - E0 >= kSplitWaves ? E0 : 0;
  return J - E;
}

// The position wave `wave` takes after position j (J or more: none).  A
// wave starts at position `wave`.
QSDPA_HD int wave_split_next(int j, int J, int J8, int wave) {
  if (j + kSplitWaves < J8) return j + kSplitWaves;
  if (wave >= 4) return J;
  return j < J8 ? J8 + wave : j + 4;
}

// The wave that visits the last position J - 1 (J >= 1).
QSDPA_HD int wave_split_last_owner(int J, int D) {
  const int J8 = wave_split_rr_end(J, D);
  return J8 < J ? (J - 1 - J8) % 4 : (J - 1) % kSplitWaves;
}

// Super-tiles: a segment of a sequence's T key tiles owns super-tiles of
// 2^sh consecutive tiles, t_lo, t_lo + stride, ... (at most jmax of them).
// Uniform splits (stride = S > 1) use 8-tile super-tiles where every split
// still gets one (T / S >= 8), else 4, 2 or 1; stream-K segments (stride 1)
// take single tiles.
QSDPA_HD int super_tile_shift(int T, int stride) {
  const int per = stride > 1 ? T / stride : 0;
  return per >= 8 ? 3 : per >= 4 ? 2 : per >= 2 ? 1 : 0;
}

// Positions of the segment: whole super-tiles, the sequence's last one
// possibly short.
QSDPA_HD int super_tile_positions(int T, int t_lo, int stride, int jmax, int sh) {
  const int TS = (T + (1 << sh) - 1) >> sh;
  const int cnt = TS > t_lo ? (jmax < (TS - t_lo + stride - 1) / stride ? jmax : (TS - t_lo + stride - 1) / stride) : 0;
  if (cnt <= 0) return 0;
  const int rest = T - ((t_lo + (cnt - 1) * stride) << sh);
  return ((cnt - 1) << sh) + (rest < (1 << sh) ? rest : (1 << sh));
}

// The tile of position j.
QSDPA_HD int super_tile_tile(int j, int t_lo, int stride, int sh) {
  return ((t_lo + (j >> sh) * stride) << sh) + (j & ((1 << sh) - 1));
}

}  // namespace qsdpa
