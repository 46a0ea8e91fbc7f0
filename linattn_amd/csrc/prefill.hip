// Block-sparse prefill (MFMA).
#include "common.h"

extern "C" int la_block_sparse_prefill(const la_prefill_args *, void *) {
  return la::fail(LA_ERR_UNSUPPORTED, "la_block_sparse_prefill: not built yet");
}
