/*
 * q3x_oracle.h -- CPU restatement of qwen3x's quantized matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * backend.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it; the product library never links or calls it.
 *
 * Every function restates the reference's own algorithm, with the loop order
 * and fused multiply-adds of the reference build (g++ -O3 -march=native
 * contracts `a += b * c` into one FMA), so results are bit-identical to the
 * reference CPU path.  Sources followed (paths inside the reference tree):
 *   f16 decode                arch/cpu.cpp:31-52
 *   embed_q8_0 / embed_q4_0   arch/cpu.cpp:55-63, 81-90 (q4.h:19-23)
 *   dot/mv Q8_0, Q4_0         arch/cpu.cpp:64-78, 91-106
 *   quantized_bytes           arch/cpu.cpp:161-179
 *   sigmoid / silu            engine.cpp:187-191
 *   router_top_k              engine.cpp:377-405
 *   routed part of moe()      engine.cpp:406-420, expert_mv engine.cpp:214-224
 *   per-token prefill         engine.cpp:580-583 (N independent mv calls)
 *   quantize_q8_0 / _q4_0     scripts/pack_weights.py:299-343
 */
#ifndef Q3X_ORACLE_H
#define Q3X_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { Q3XO_BF16 = 0, Q3XO_Q8_0 = 1, Q3XO_Q4_0 = 2 };

float q3xo_f16(uint16_t value);
/* 1 = ok (bytes written), 0 = rejected (bytes untouched). */
int q3xo_quantized_bytes(uint32_t type, int rows, int cols, size_t* bytes);
/* Dequantize one row (arch/cpu.cpp try_embed).  1 = handled, 0 = not. */
int q3xo_embed(const void* weights, uint32_t type, int cols, int row, float* out);
/* Rows [row0, row1) of y = W x, serial, reference order.  1 = handled. */
int q3xo_mv_rows(const void* weights, uint32_t type, int row0, int row1, int cols,
                 const float* x, float* y);
/* y = W x split over `threads` row ranges (bit-identical to serial). */
int q3xo_mv(const void* weights, uint32_t type, int rows, int cols,
            const float* x, float* y, int threads);
/* Y[t] = W X[t] for t < count: the reference's prefill is one mv per token. */
int q3xo_gemm(const void* weights, uint32_t type, int rows, int cols,
              const float* X, int count, float* Y, int threads);

float q3xo_sigmoid(float x);
float q3xo_silu(float x);
/* Router of one token: ids[slot], weights[slot] = renormalised probability.
 * probabilities: scratch of `experts` floats (softmax output).  0 on bad args. */
int q3xo_router_top_k(const float* logits, int experts, int top_k, int* ids,
                      float* weights, float* probabilities);
/* Routed experts for `tokens` tokens (engine.cpp moe() minus router/shared):
 * Y[t] = sum_slot weights[t,slot] * Down_e * (silu(G_e x) * U_e x), slot order,
 * starting from 0.  gate_up: [E, 2I, H], down: [E, H, I].  1 = ok. */
int q3xo_moe_routed(const void* gate_up, const void* down, uint32_t type,
                    int experts, int H, int I, const float* X, int tokens,
                    const int* ids, const float* weights, int top_k, float* Y,
                    int threads);
/* y[r] = BF16 row r . x for r < rows (engine.cpp:181-212: f32(bf16) is the
 * value's bits shifted up 16, the dot a sequential FMA chain).  1 = ok. */
int q3xo_mv_bf16(const uint16_t* weights, int rows, int cols, const float* x, float* y);
/* The whole MoE layer of engine.cpp:406-430 for `tokens` tokens: BF16 router
 * [E, H] -> top_k -> routed experts (as q3xo_moe_routed) -> shared expert
 * (shared_gate/up [shared_I, H], shared_down [H, shared_I], same type as the
 * experts) scaled by sigmoid(BF16 shared_scale [1, H] . x) and added last.
 * ids/weights (optional, [tokens, top_k]) receive the routing.  Requires
 * shared_I <= I (the reference reuses its 2I gate_up buffer).  1 = ok. */
int q3xo_moe_layer(const uint16_t* router, const void* gate_up, const void* down,
                   const void* shared_gate, const void* shared_up, const void* shared_down,
                   const uint16_t* shared_scale, uint32_t type, int experts, int H, int I,
                   int shared_I, int top_k, const float* X, int tokens, float* Y, int* ids,
                   float* weights, int threads);
/* The BF16 dot of q3xo_mv_bf16 and q3xo_moe_layer: lanes 1 = the reference's
 * portable loop (engine.cpp:200-205), 16 = its AVX-512 kernel
 * (arch/x86/kernels.h:21-37), as a reference built with AVX-512 takes.
 * Process-wide; 1 = ok, 0 = other values. */
int q3xo_set_bf16_lanes(int lanes);
/* pack_weights.py quantizers applied to float32 values (n % 32 == 0).
 * 1 = ok, 0 = partial block or non-finite input. */
int q3xo_quantize(uint32_t type, const float* values, size_t n, void* out);

#ifdef __cplusplus
}
#endif
#endif
