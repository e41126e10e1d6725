// backend.cpp -- see backend.h.
#include "backend.h"

#include <cstdio>
#include <cstdlib>
#include <new>

#include "q3x_hip.h"

namespace {

void fail(const char* what, const char* file, int line, int code) {
    std::fprintf(stderr, "%s:%d: %s failed: %s (%d)\n", file, line, what, q3x_hip_strerror(code), code);
    std::abort();
}

#define BACKEND_CHECK(call)                                   \
    do {                                                      \
        const int code_ = (call);                             \
        if (code_ != Q3X_HIP_OK) fail(#call, __FILE__, __LINE__, code_); \
    } while (0)
#define BACKEND_ASSERT(cond) \
    do {                     \
        if (!(cond)) fail(#cond, __FILE__, __LINE__, Q3X_HIP_EINVAL); \
    } while (0)

constexpr int kVocabulary = 248320;       // model_config.h:61 (every supported model)
constexpr int kMaxContext = 262144;       // model_config.h:13
constexpr int kEndOfText = 248044;        // engine.cpp:28
constexpr int kImEnd = 248046;

}  // namespace

namespace q3x_backend {

struct Model {
    q3x_hip_model* handle = nullptr;
    q3x_hip_model_config config{};
    const void* weights = nullptr;
};

struct State {
    q3x_hip_engine* engine = nullptr;
    int vocabulary = 0;
};

Model* model_create(const char* path, char* err, size_t errlen) {
    BACKEND_ASSERT(path);
    Model* model = new (std::nothrow) Model();
    const char* message = nullptr;
    if (!model || q3x_hip_model_load(path, &model->handle, &message) != Q3X_HIP_OK) {
        if (err && errlen) std::snprintf(err, errlen, "%s", message ? message : "allocation failed");
        delete model;
        return nullptr;
    }
    BACKEND_CHECK(q3x_hip_model_info(model->handle, &model->config, nullptr, nullptr, &model->weights, nullptr));
    if (err && errlen) err[0] = '\0';
    return model;
}

void model_destroy(Model* model) {
    if (!model) return;
    q3x_hip_model_free(model->handle);
    delete model;
}

State* state_create(Model* model, int context_size) {
    BACKEND_ASSERT(model && context_size > 0 && context_size <= kMaxContext);
    State* state = new (std::nothrow) State();
    BACKEND_ASSERT(state);
    const char* message = nullptr;
    const int code =
        q3x_hip_engine_create(&model->config, model->weights, context_size, 0, &state->engine, &message);
    if (code != Q3X_HIP_OK) {
        std::fprintf(stderr, "state_create: %s\n", message ? message : q3x_hip_strerror(code));
        fail("q3x_hip_engine_create", __FILE__, __LINE__, code);
    }
    state->vocabulary = model->config.V;
    return state;
}

void state_destroy(State* state) {
    if (!state) return;
    q3x_hip_engine_destroy(state->engine);
    delete state;
}

void state_reset(State* state) {
    BACKEND_ASSERT(state);
    BACKEND_CHECK(q3x_hip_engine_reset(state->engine));
}

void state_forward(Model* model, State* state, const int* tokens, int count, bool compute_logits) {
    BACKEND_ASSERT(model && state && tokens && count > 0);
    BACKEND_CHECK(q3x_hip_engine_forward(state->engine, tokens, count, compute_logits ? 1 : 0));
}

void state_checkpoint_save(State* state) {
    BACKEND_ASSERT(state);
    BACKEND_CHECK(q3x_hip_engine_checkpoint_save(state->engine));
}

void state_checkpoint_restore(State* state) {
    BACKEND_ASSERT(state);
    BACKEND_CHECK(q3x_hip_engine_checkpoint_restore(state->engine));
}

int state_argmax(const State* state) {
    if (!state) return -1;
    int token = -1;
    BACKEND_CHECK(q3x_hip_engine_argmax(state->engine, &token));
    return token;
}

void state_copy_logits(const State* state, float* output) {
    BACKEND_ASSERT(state && output);
    BACKEND_CHECK(q3x_hip_engine_logits(state->engine, output));
}

uint32_t model_id(const Model* model) { return model->config.id; }

int vocab_size() { return kVocabulary; }
int max_context() { return kMaxContext; }
bool token_is_stop(int token) { return token == kEndOfText || token == kImEnd; }

}  // namespace q3x_backend
