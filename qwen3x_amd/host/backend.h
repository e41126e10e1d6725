// backend.h -- the backend operations the reference's runtime calls
// (q3x_backend::*, internal.h:11-34), implemented on the HIP library: a
// model is a loaded model.bin (q3x_hip_model_load), a state a decode engine
// over it (q3x_hip_engine_*).  Same names, arguments and behaviour as the
// reference's CPU and CUDA backends (engine.cpp:561-613, arch/cuda/
// engine.cu:2196-2370): model_create reports a load failure in `err` and
// returns null; every other failure aborts, as the reference's Q3X_ASSERT
// and CUDA_OK do.  Q8_0 and Q4_0 models (Qwen3.5-9B, Qwen3.6-35B-A3B,
// Qwen3.8-27B) run here; the BF16 ones (0.8B, 4B) are refused at
// state_create, the matmul path being quantized.
#pragma once

#include <cstddef>
#include <cstdint>

namespace q3x_backend {

struct Model;
struct State;

Model* model_create(const char* path, char* err, size_t errlen);
void model_destroy(Model* model);

State* state_create(Model* model, int context_size);
void state_destroy(State* state);
void state_reset(State* state);
void state_forward(Model* model, State* state, const int* tokens, int count, bool compute_logits);
void state_checkpoint_save(State* state);
void state_checkpoint_restore(State* state);
int state_argmax(const State* state);
void state_copy_logits(const State* state, float* output);
uint32_t model_id(const Model* model);

int vocab_size();
int max_context();
bool token_is_stop(int token);

}  // namespace q3x_backend
