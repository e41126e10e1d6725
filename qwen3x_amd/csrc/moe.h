// moe.h -- library-internal entry of the MoE layer for the decode engine.
#pragma once

#include "common.h"

namespace q3x {

// One token of the MoE layer of q3x_hip_moe_layer (engine.cpp:406-430), its
// result added to Y: Y += routed sum + gated shared expert, the layer output
// formed in full first and added once, as the reference adds the layer's
// output to its residual (engine.cpp:240-242).  With norm_w, X is the raw
// residual and the layer's input RMSNorm(X) * (1 + norm_w) (engine.cpp:
// 228-233, the post-attention norm) is formed inside the router and expert
// launches; X may then be Y itself.  Q3X_HIP_ENOTSUP (and Y left unchanged)
// where the shape or alignment needs the grouped path; the caller then
// normalises X, runs q3x_hip_moe_layer and adds its output itself.
int moe_layer_decode_add(const q3x_hip_moe_layer_weights& layer, const float* X, const uint16_t* norm_w, float* Y,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

// h[count, I] = silu(X G^T) * (X U^T) for X[count, H] and gate / up
// matrices [I, H] of one type: a prefill FFN's gate and up GEMMs with the
// SwiGLU (engine.cpp:371-376) in their epilogue -- gate row q and up row q in
// one 32-column tile -- each product summed as the GEMM launches sum it
// (K in block order within one half), then silu(g) * u as swiglu_kernel.
// Q3X_HIP_ENOTSUP (nothing enqueued) where I % 64 != 0 or an operand is
// unaligned (weights 2, X 16, h 4 bytes).
int gate_up_swiglu(const void* gate, const void* up, uint32_t type, int I, int H, const float* X, int count,
                   float* h, hipStream_t stream);

}  // namespace q3x
