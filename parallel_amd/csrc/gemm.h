// Internal launchers shared between the GEMM and router translation units.
#pragma once

#include "common.h"

namespace moe {

// partials[s][T][E] (f32) = x[T, s-th K range] . wr[E, s-th K range]^T.
int router_logits_partials(const bf16_t* x, const bf16_t* wr, float* partials, int T, int H, int E, int splits,
                           int k_chunk, hipStream_t stream);

// partials[c][E][H] (f32) = dl[rows of chunk c, E]^T . x[rows of chunk c, H].
int router_wgrad_partials(const bf16_t* dl, const bf16_t* x, float* partials, int T, int H, int E, int chunks,
                          int chunk_rows, hipStream_t stream);

// dx[T,H] (bf16) = dl[T,E] . wr[E,H].
int router_dgrad(const bf16_t* dl, const bf16_t* wr, bf16_t* dx, int T, int H, int E, hipStream_t stream);

}  // namespace moe
