// MFMA head-grouped split-K decode (placeholder until the gfx950 MFMA kernel
// lands; every shape currently routes to the VALU kernel).
#include "abi_internal.h"
#include "common.h"

namespace qsdpa {

bool mfma_supports(const qsdpa_decode_args*) { return false; }

int mfma_num_splits(const qsdpa_decode_args*, int) { return 1; }

int launch_decode_mfma(const qsdpa_decode_args*, int, float*, float*, hipStream_t) {
  return fail(QSDPA_ERR_UNSUPPORTED, "MFMA decode not built");
}

}  // namespace qsdpa
