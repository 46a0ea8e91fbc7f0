// Lightning-indexer top-k (filled in below the stub line once implemented).
#include "common.h"

extern "C" size_t la_indexer_topk_workspace(const la_indexer_args *) { return 0; }
extern "C" int la_indexer_topk(const la_indexer_args *, void *) {
  return la::fail(LA_ERR_UNSUPPORTED, "la_indexer_topk: not built yet");
}
