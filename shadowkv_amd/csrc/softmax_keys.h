// The few-row selection's key producer (score.hip), called from select.hip: the softmax + GQA-max
// kernel writing the selection keys (bf16 GQA-max probabilities) and, per workgroup, the
// histogram of the keys' high order-key bytes, so that the selection starts from the summed
// histogram instead of counting every key again on one workgroup per row.
#pragma once

#include "skv_common.h"

namespace skv {

// Workgroups per row of softmax_keys_hist for `rows` rows of n landmarks (n % 8 == 0), i.e. the
// number of partial histograms per row it writes; 0 when the shape cannot take that path.
int softmax_hist_parts(int rows, int n);

// out_max[z][j] = bf16 max_i softmax_i(D[z][i][:])[j] (bit-identical to skv_softmax_gqa_max) and
// hist[z][part][b] = number of keys of workgroup `part` of row z whose order key's high byte is b,
// for softmax_hist_parts(rows, n) parts per row. Needs n % 8 == 0 and 16-byte aligned D/out_max.
int softmax_keys_hist(const uint16_t* D, const float* norm, const float* sum, uint16_t* out_max, uint32_t* hist,
                      int rows, int m, int n, hipStream_t stream);

}  // namespace skv
