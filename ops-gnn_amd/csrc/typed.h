// Exact-dtype (integer, float64) segment and scatter reductions: internal
// entry points that ogn_segment_reduce / ogn_scatter_atomic dispatch to.
#pragma once

#include "ogn_device.h"

namespace ogn {

// int8, uint8, int16, int32, int64, float64
bool is_exact_dtype(int dt);

// Workspace for the piece records of long integer segments (0: none used).
size_t exact_segment_workspace_size(int64_t batch, int64_t length, int64_t k, int dtype, int reduce);

// Arguments as ogn_segment_reduce (validated by the caller).  A workspace
// smaller than exact_segment_workspace_size, or the short-segments hint,
// folds every segment serially.
int exact_segment_reduce(const int64_t* indptr, int64_t ptr_batches, const void* src, int dtype, int64_t batch,
                         int64_t length, int64_t segments, int64_t k, void* out, int64_t* arg, int reduce,
                         int semantics, int has_out, bool short_segments, void* workspace, size_t workspace_bytes,
                         hipStream_t stream);

size_t exact_scatter_workspace_size(int64_t cells, int reduce);

// Arguments as ogn_scatter_atomic (validated by the caller).
int exact_scatter_atomic(const void* src, int dtype, const int64_t* index, int64_t isb, int64_t isl, int64_t isf,
                         int64_t before, int64_t len, int64_t after, int64_t size, void* out, int64_t* arg,
                         int reduce, int has_out, void* workspace, hipStream_t stream);

}  // namespace ogn
