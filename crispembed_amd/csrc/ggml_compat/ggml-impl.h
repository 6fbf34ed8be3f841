// ggml-impl.h (compat subset) -- STANDALONE-BUILD STAND-IN for the graph query
// a backend's fusion pass uses from ggml's internal header; see ggml.h in this
// directory for the provenance and limits.
#pragma once
#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

// How many nodes of the graph read node `node_idx`'s result (ggml counts the uses
// over the whole graph, so a node read by a later split is never fused away).
GGML_API int ggml_node_get_use_count(const struct ggml_cgraph *cgraph, int node_idx);

#ifdef __cplusplus
}
#endif
