// Block selection for block-sparse prefill.
#include "common.h"

extern "C" size_t la_block_select_workspace(const la_block_select_args *) { return 0; }
extern "C" int la_block_select(const la_block_select_args *, void *) {
  return la::fail(LA_ERR_UNSUPPORTED, "la_block_select: not built yet");
}
