// model.cpp -- model.bin: header check, tensor schema and device upload.
//
// The format is the reference's (model_config.h; engine.cpp:455-559;
// arch/cuda/engine.cu:2007-2188; written by scripts/pack_weights.py): a
// 72-byte header, then the tensors of one fixed configuration in one fixed
// order, each at the next multiple of 64 bytes, the file ending at the last
// tensor.  The schema depends on nothing but the header, so the whole file is
// validated from the header and its size before any device work; the upload
// then streams the file through pinned staging buffers on several reader
// threads, overlapping reads with host-to-device copies, into one device
// buffer laid out exactly as the file (device address = base + file offset).
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cerrno>
#include <cstring>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include <hip/hip_runtime_api.h>

#include "q3x_hip.h"

struct q3x_hip_model {
    q3x_hip_model_config config{};
    std::vector<q3x_hip_tensor> tensors;
    uint8_t* base = nullptr;  // device buffer of `bytes`, the whole file
    uint64_t bytes = 0;
};

namespace {

constexpr uint64_t kPrefixBytes = 8;        // "Q3XMODL\0"
constexpr int kFieldCount = 16;             // ConfigField, model_config.h:22-39
constexpr uint64_t kAlignment = 64;         // take(), engine.cpp:464
constexpr uint32_t kMaxContext = 262144;    // model_config.h:13
static_assert(Q3X_HIP_MODEL_HEADER_BYTES == kPrefixBytes + 4 * kFieldCount, "header size");

// The five supported models, field for field as model_config.h:59-102 (the
// file format fixes every shape by model ID).
constexpr q3x_hip_model_config kConfigs[] = {
    {800, "Qwen3.5-0.8B", 248320, 1024, 3584, 24, 4, 8, 2, 256, 64, 16, 16, 128, 128, 4, 0, 0, 0,
     Q3X_HIP_MATRIX_BF16, 1},
    {4000, "Qwen3.5-4B", 248320, 2560, 9216, 32, 4, 16, 4, 256, 64, 16, 32, 128, 128, 4, 0, 0, 0,
     Q3X_HIP_MATRIX_BF16, 1},
    {9000, "Qwen3.5-9B", 248320, 4096, 12288, 32, 4, 16, 4, 256, 64, 16, 32, 128, 128, 4, 0, 0, 0,
     Q3X_HIP_MATRIX_Q8_0, 0},
    {36035, "Qwen3.6-35B-A3B", 248320, 2048, 512, 40, 4, 16, 2, 256, 64, 16, 32, 128, 128, 4, 256, 8, 512,
     Q3X_HIP_MATRIX_Q4_0, 0},
    {38027, "Qwen3.8-27B", 248320, 5120, 17408, 64, 4, 24, 4, 256, 64, 16, 48, 128, 128, 4, 0, 0, 0,
     Q3X_HIP_MATRIX_Q4_0, 0},
};

uint32_t read_u32(const uint8_t* p) {
    uint32_t v;
    std::memcpy(&v, p, sizeof(v));
    return v;  // little-endian host (x86-64), as the format
}

// The 16 header fields a file of `c` must carry, in ConfigField order
// (model_config.h:115-141).
void expected_fields(const q3x_hip_model_config& c, uint32_t (&f)[kFieldCount]) {
    const int values[kFieldCount - 1] = {static_cast<int>(c.id), c.V, c.H, c.I, c.N, c.AI, c.AH, c.KVH,
                                         c.AD, c.RD, c.KH, c.VH, c.KD, c.VD, c.CK};
    for (int i = 0; i < kFieldCount - 1; ++i) f[i] = static_cast<uint32_t>(values[i]);
    f[kFieldCount - 1] = kMaxContext;
}

uint64_t tensor_bytes(uint32_t type, int experts, int rows, int cols) {
    const uint64_t count = static_cast<uint64_t>(std::max(experts, 1)) * static_cast<uint64_t>(rows) *
                           static_cast<uint64_t>(cols);
    switch (type) {
    case Q3X_HIP_MATRIX_Q8_0: return count / 32 * 34;
    case Q3X_HIP_MATRIX_Q4_0: return count / 32 * 18;
    case Q3X_HIP_TENSOR_F32: return count * 4;
    default: return count * 2;  // BF16
    }
}

// The tensor list of configuration `c` in file order (engine.cpp:499-557),
// offsets not yet assigned.
std::vector<q3x_hip_tensor> schema(const q3x_hip_model_config& c) {
    std::vector<q3x_hip_tensor> list;
    auto add = [&](uint32_t role, int layer, uint32_t type, int rows, int cols, int experts = 0) {
        list.push_back(q3x_hip_tensor{role, layer, type, experts, rows, cols, 0,
                                      tensor_bytes(type, experts, rows, cols)});
    };
    const uint32_t M = c.matrix_type, BF = Q3X_HIP_MATRIX_BF16, F32 = Q3X_HIP_TENSOR_F32;
    const int AS = c.AH * c.AD, KVW = c.KVH * c.AD;
    const int DO = c.VH * c.VD, DQKV = 2 * c.KH * c.KD + DO;
    add(Q3X_HIP_EMBEDDING, -1, M, c.V, c.H);
    if (!c.tied_embeddings) add(Q3X_HIP_LM_HEAD, -1, M, c.V, c.H);
    add(Q3X_HIP_FINAL_NORM, -1, BF, 1, c.H);
    for (int l = 0; l < c.N; ++l) {
        add(Q3X_HIP_INPUT_NORM, l, BF, 1, c.H);
        if (l % c.AI != c.AI - 1) {  // DeltaNet layer
            add(Q3X_HIP_DELTA_QKV, l, M, DQKV, c.H);
            add(Q3X_HIP_DELTA_Z, l, M, DO, c.H);
            add(Q3X_HIP_DELTA_A, l, M, c.VH, c.H);
            add(Q3X_HIP_DELTA_B, l, M, c.VH, c.H);
            add(Q3X_HIP_DELTA_CONV, l, BF, DQKV, c.CK);
            add(Q3X_HIP_DELTA_ALOG, l, F32, 1, c.VH);
            add(Q3X_HIP_DELTA_DT, l, BF, 1, c.VH);
            add(Q3X_HIP_DELTA_NORM, l, F32, 1, c.VD);
            add(Q3X_HIP_DELTA_OUT, l, M, c.H, DO);
        } else {  // full attention layer
            add(Q3X_HIP_ATTN_Q, l, M, 2 * AS, c.H);
            add(Q3X_HIP_ATTN_K, l, M, KVW, c.H);
            add(Q3X_HIP_ATTN_V, l, M, KVW, c.H);
            add(Q3X_HIP_ATTN_QNORM, l, BF, 1, c.AD);
            add(Q3X_HIP_ATTN_KNORM, l, BF, 1, c.AD);
            add(Q3X_HIP_ATTN_OUT, l, M, c.H, AS);
        }
        add(Q3X_HIP_POST_NORM, l, BF, 1, c.H);
        if (c.experts) {
            add(Q3X_HIP_MOE_ROUTER, l, BF, c.experts, c.H);
            add(Q3X_HIP_MOE_GATE_UP, l, M, 2 * c.I, c.H, c.experts);
            add(Q3X_HIP_MOE_DOWN, l, M, c.H, c.I, c.experts);
            add(Q3X_HIP_MOE_SHARED_GATE, l, M, c.shared_I, c.H);
            add(Q3X_HIP_MOE_SHARED_UP, l, M, c.shared_I, c.H);
            add(Q3X_HIP_MOE_SHARED_DOWN, l, M, c.H, c.shared_I);
            add(Q3X_HIP_MOE_SHARED_SCALE, l, BF, 1, c.H);
        } else {
            add(Q3X_HIP_FFN_GATE, l, M, c.I, c.H);
            add(Q3X_HIP_FFN_UP, l, M, c.I, c.H);
            add(Q3X_HIP_FFN_DOWN, l, M, c.H, c.I);
        }
    }
    return list;
}

// Offsets in file order from the end of the header, each tensor at the next
// multiple of 64 bytes (take(), engine.cpp:461-478); returns the end.
uint64_t place(std::vector<q3x_hip_tensor>& list) {
    uint64_t cursor = Q3X_HIP_MODEL_HEADER_BYTES;
    for (auto& t : list) {
        cursor = (cursor + kAlignment - 1) / kAlignment * kAlignment;
        t.offset = cursor;
        cursor += t.bytes;
    }
    return cursor;
}

// Shapes the schema walk accepts for a configuration given by the caller
// (the five fixed ones pass): positive sizes, whole 32-element blocks in
// every quantized row, heads that divide evenly, and sizes whose products
// fit the int fields of the tensor table.
bool config_ok(const q3x_hip_model_config& c) {
    const long long dims[] = {c.V, c.H, c.I, c.N, c.AI, c.AH, c.KVH, c.AD, c.RD, c.KH, c.VH, c.KD, c.VD, c.CK};
    for (long long d : dims)
        if (d <= 0 || d > (1 << 24)) return false;
    if (c.matrix_type > Q3X_HIP_MATRIX_Q4_0 || c.AH % c.KVH != 0 || c.VH % c.KH != 0) return false;
    if (c.experts < 0 || c.top_k < 0 || c.shared_I < 0) return false;
    if (c.experts && (c.top_k < 1 || c.top_k > c.experts || c.shared_I < 1)) return false;
    const long long AS = 1ll * c.AH * c.AD, KVW = 1ll * c.KVH * c.AD, DO = 1ll * c.VH * c.VD;
    const long long DQKV = 2ll * c.KH * c.KD + DO;
    const long long rows[] = {2 * AS, KVW, DQKV, DO, 2ll * c.I * std::max(c.experts, 1), 1ll * c.H * std::max(c.experts, 1)};
    for (long long r : rows)
        if (r > INT32_MAX) return false;
    if (c.matrix_type != Q3X_HIP_MATRIX_BF16) {
        const long long cols[] = {c.H, AS, DO, c.I, c.experts ? c.shared_I : 32};
        for (long long k : cols)
            if (k % 32 != 0) return false;
    }
    return true;
}

// Header and size checks of Model::load (engine.cpp:485-496, 559) and the
// schema walk of take() (engine.cpp:461-478): the cursor only grows, so a
// tensor ends past the file exactly when the aligned schema end does.
int validate(const uint8_t* header, uint64_t file_size, const q3x_hip_model_config** config,
             std::vector<q3x_hip_tensor>* tensors, const char** message) {
    if (file_size < Q3X_HIP_MODEL_HEADER_BYTES) { *message = "bad model.bin"; return Q3X_HIP_EMODEL; }
    if (std::memcmp(header, "Q3XMODL\0", kPrefixBytes) != 0) {
        *message = "wrong model.bin magic";
        return Q3X_HIP_EMODEL;
    }
    const uint32_t id = read_u32(header + kPrefixBytes);
    const q3x_hip_model_config* found = nullptr;
    for (const auto& c : kConfigs)
        if (c.id == id) found = &c;
    if (!found) { *message = "unsupported Qwen model ID"; return Q3X_HIP_EMODEL; }
    uint32_t want[kFieldCount];
    expected_fields(*found, want);
    for (int i = 0; i < kFieldCount; ++i) {
        if (read_u32(header + kPrefixBytes + 4 * i) != want[i]) {
            *message = "Qwen model.bin header mismatch";
            return Q3X_HIP_EMODEL;
        }
    }
    std::vector<q3x_hip_tensor> list = schema(*found);
    const uint64_t cursor = place(list);
    if (cursor > file_size) { *message = "truncated model.bin"; return Q3X_HIP_EMODEL; }
    if (cursor != file_size) { *message = "model.bin size does not match schema"; return Q3X_HIP_EMODEL; }
    *config = found;
    *tensors = std::move(list);
    return Q3X_HIP_OK;
}

// pread until `len` bytes are in: false on an error or an early end of file.
bool read_exact(int fd, uint8_t* dst, uint64_t len, uint64_t offset) {
    while (len) {
        const ssize_t n = pread(fd, dst, static_cast<size_t>(std::min<uint64_t>(len, 1ull << 30)),
                                static_cast<off_t>(offset));
        if (n < 0 && errno == EINTR) continue;
        if (n <= 0) return false;
        dst += n;
        offset += static_cast<uint64_t>(n);
        len -= static_cast<uint64_t>(n);
    }
    return true;
}

// Four readers with 4 MiB staging buffers load a page-cached file at ~51 GB/s
// on MI355X (PCIe Gen5 x16); 32 MiB buffers fall to ~26 GB/s, 64 MiB to ~16,
// and the runtime's own pageable hipMemcpy from a mapping reaches ~31.
constexpr uint64_t kChunk = 4ull << 20;  // bytes per staging buffer
constexpr int kReaders = 4;              // reader threads, two staging buffers each

// Copies file bytes [0, size) to dst on `device`.  Reader r takes chunks r,
// r + R, ...: it reads chunk k into staging buffer k % 2 (after the copy that
// last used that buffer has finished) and queues the copy on its own stream,
// so one buffer is read while the other is in flight.
int upload(int fd, uint64_t size, uint8_t* dst, int device, const char** message) {
    const uint64_t chunks = (size + kChunk - 1) / kChunk;
    const int readers = static_cast<int>(std::min<uint64_t>(static_cast<uint64_t>(kReaders), chunks));
    std::atomic<int> failed{0};
    std::mutex lock;
    const char* first = nullptr;
    auto fail = [&](const char* m) {
        std::lock_guard<std::mutex> g(lock);
        if (!first) first = m;
        failed.store(1);
    };
    auto reader = [&](int r) {
        if (hipSetDevice(device) != hipSuccess) return fail("HIP model upload failed");
        hipStream_t stream = nullptr;
        void* staging[2] = {nullptr, nullptr};
        hipEvent_t done[2] = {nullptr, nullptr};
        bool ok = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) == hipSuccess;
        for (int b = 0; ok && b < 2; ++b)
            ok = hipHostMalloc(&staging[b], kChunk, hipHostMallocDefault) == hipSuccess &&
                 hipEventCreateWithFlags(&done[b], hipEventDisableTiming) == hipSuccess;
        if (!ok) fail("HIP model upload failed");
        uint64_t k = 0;
        for (uint64_t c = r; ok && c < chunks && !failed.load(); c += readers, ++k) {
            const int b = static_cast<int>(k & 1);
            if (k >= 2 && hipEventSynchronize(done[b]) != hipSuccess) { fail("HIP model upload failed"); break; }
            const uint64_t offset = c * kChunk, len = std::min(kChunk, size - offset);
            if (!read_exact(fd, static_cast<uint8_t*>(staging[b]), len, offset)) {
                fail("cannot read model.bin");
                break;
            }
            if (hipMemcpyAsync(dst + offset, staging[b], len, hipMemcpyHostToDevice, stream) != hipSuccess ||
                hipEventRecord(done[b], stream) != hipSuccess) {
                fail("HIP model upload failed");
                break;
            }
        }
        // Every queued copy ends before its staging buffer is freed.
        if (stream && hipStreamSynchronize(stream) != hipSuccess) fail("HIP model upload failed");
        for (int b = 0; b < 2; ++b) {
            if (done[b]) (void)hipEventDestroy(done[b]);
            if (staging[b]) (void)hipHostFree(staging[b]);
        }
        if (stream) (void)hipStreamDestroy(stream);
    };
    std::vector<std::thread> threads;
    for (int r = 1; r < readers; ++r) threads.emplace_back(reader, r);
    reader(0);
    for (auto& t : threads) t.join();
    if (failed.load()) {
        *message = first;
        return std::strcmp(first, "cannot read model.bin") == 0 ? static_cast<int>(Q3X_HIP_EMODEL)
                                                                 : static_cast<int>(Q3X_HIP_ERUNTIME);
    }
    return Q3X_HIP_OK;
}

void set(const char** error, const char* message) {
    if (error) *error = message;
}

}  // namespace

extern "C" int q3x_hip_model_layout(const void* header, size_t header_bytes, uint64_t file_size,
                                    q3x_hip_model_config* config, q3x_hip_tensor* tensors, size_t capacity,
                                    size_t* count, const char** error) {
    if (!header || !count) return Q3X_HIP_EINVAL;
    if (file_size >= Q3X_HIP_MODEL_HEADER_BYTES && header_bytes < Q3X_HIP_MODEL_HEADER_BYTES)
        return Q3X_HIP_EINVAL;
    const q3x_hip_model_config* found = nullptr;
    std::vector<q3x_hip_tensor> list;
    const char* message = nullptr;
    const int code = validate(static_cast<const uint8_t*>(header), file_size, &found, &list, &message);
    if (code != Q3X_HIP_OK) {
        set(error, message);
        return code;
    }
    *count = list.size();
    if (tensors && capacity < list.size()) return Q3X_HIP_EINVAL;
    if (tensors) std::copy(list.begin(), list.end(), tensors);
    if (config) *config = *found;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_model_schema(const q3x_hip_model_config* config, q3x_hip_tensor* tensors, size_t capacity,
                                    size_t* count, uint64_t* bytes) {
    if (!config || !count || !config_ok(*config)) return Q3X_HIP_EINVAL;
    std::vector<q3x_hip_tensor> list = schema(*config);
    const uint64_t end = place(list);
    *count = list.size();
    if (bytes) *bytes = end;
    if (tensors && capacity < list.size()) return Q3X_HIP_EINVAL;
    if (tensors) std::copy(list.begin(), list.end(), tensors);
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_model_load(const char* path, q3x_hip_model** model, const char** error) {
    if (!path || !model) return Q3X_HIP_EINVAL;
    *model = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        set(error, "cannot open model.bin");
        return Q3X_HIP_EMODEL;
    }
    struct Closer {
        int fd;
        ~Closer() { close(fd); }
    } closer{fd};
    struct stat info {};
    if (fstat(fd, &info) != 0 || info.st_size < static_cast<off_t>(Q3X_HIP_MODEL_HEADER_BYTES)) {
        set(error, "bad model.bin");
        return Q3X_HIP_EMODEL;
    }
    const uint64_t size = static_cast<uint64_t>(info.st_size);
    uint8_t header[Q3X_HIP_MODEL_HEADER_BYTES];
    if (!read_exact(fd, header, sizeof(header), 0)) {
        set(error, "cannot read model.bin");
        return Q3X_HIP_EMODEL;
    }
    const q3x_hip_model_config* config = nullptr;
    std::vector<q3x_hip_tensor> list;
    const char* message = nullptr;
    int code = validate(header, size, &config, &list, &message);
    if (code != Q3X_HIP_OK) {
        set(error, message);
        return code;
    }
    q3x_hip_model* m = new (std::nothrow) q3x_hip_model();
    if (!m) {
        set(error, "cannot allocate the model table");
        return Q3X_HIP_ERUNTIME;
    }
    m->config = *config;
    m->tensors = std::move(list);
    m->bytes = size;
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        delete m;
        set(error, "HIP model allocation failed");
        return Q3X_HIP_ERUNTIME;
    }
    void* base = nullptr;
    const hipError_t status = hipMalloc(&base, size);
    if (status != hipSuccess) {
        delete m;
        (void)hipGetLastError();
        set(error, status == hipErrorOutOfMemory ? "HIP model does not fit in device memory"
                                                 : "HIP model allocation failed");
        return Q3X_HIP_ERUNTIME;
    }
    m->base = static_cast<uint8_t*>(base);
    posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);
    code = upload(fd, size, m->base, device, &message);
    if (code != Q3X_HIP_OK) {
        q3x_hip_model_free(m);
        set(error, message);
        return code;
    }
    *model = m;
    return Q3X_HIP_OK;
}

extern "C" void q3x_hip_model_free(q3x_hip_model* model) {
    if (!model) return;
    if (model->base) (void)hipFree(model->base);
    delete model;
}

extern "C" int q3x_hip_model_info(const q3x_hip_model* model, q3x_hip_model_config* config,
                                  const q3x_hip_tensor** tensors, size_t* count, const void** base,
                                  uint64_t* bytes) {
    if (!model) return Q3X_HIP_EINVAL;
    if (config) *config = model->config;
    if (tensors) *tensors = model->tensors.data();
    if (count) *count = model->tensors.size();
    if (base) *base = model->base;
    if (bytes) *bytes = model->bytes;
    return Q3X_HIP_OK;
}

extern "C" int q3x_hip_model_tensor(const q3x_hip_model* model, uint32_t role, int layer,
                                    q3x_hip_tensor* tensor, const void** data) {
    if (!model || role >= Q3X_HIP_TENSOR_ROLES) return Q3X_HIP_EINVAL;
    if (role == Q3X_HIP_LM_HEAD && model->config.tied_embeddings) role = Q3X_HIP_EMBEDDING;
    for (const auto& t : model->tensors) {
        if (t.role == role && t.layer == layer) {
            if (tensor) *tensor = t;
            if (data) *data = model->base + t.offset;
            return Q3X_HIP_OK;
        }
    }
    return Q3X_HIP_EINVAL;
}

extern "C" int q3x_hip_model_moe_layer(const q3x_hip_model* model, int layer, q3x_hip_moe_layer_weights* weights) {
    if (!model || !weights || !model->config.experts || layer < 0 || layer >= model->config.N)
        return Q3X_HIP_EINVAL;
    const void* p[7];
    const uint32_t roles[7] = {Q3X_HIP_MOE_ROUTER, Q3X_HIP_MOE_GATE_UP, Q3X_HIP_MOE_DOWN,
                               Q3X_HIP_MOE_SHARED_GATE, Q3X_HIP_MOE_SHARED_UP, Q3X_HIP_MOE_SHARED_DOWN,
                               Q3X_HIP_MOE_SHARED_SCALE};
    for (int i = 0; i < 7; ++i)
        if (q3x_hip_model_tensor(model, roles[i], layer, nullptr, &p[i]) != Q3X_HIP_OK) return Q3X_HIP_EINVAL;
    const q3x_hip_model_config& c = model->config;
    *weights = q3x_hip_moe_layer_weights{p[0], p[1], p[2], p[3], p[4], p[5], p[6], c.matrix_type,
                                         c.experts, c.top_k, c.H, c.I, c.shared_I};
    return Q3X_HIP_OK;
}
