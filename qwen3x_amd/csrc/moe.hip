// moe.hip -- router top-k and the routed-expert matmul of the MoE layer.
//
// Reference: engine.cpp:377-420 (CPU router_top_k and routed loop of moe())
// and arch/cuda/engine.cu:1153-1250, 1709-1726 (router_top_k_kernel runs one
// thread for one token; expert_gate_up_q4_kernel / expert_swiglu_kernel /
// expert_down_weighted_q4_kernel run per token, so the reference has no
// grouped expert GEMM and its prefill is token by token).
//
// Here the router runs one wavefront per token, exchanging values by DPP.
// The routed matmul has two shapes:
//   decode (tokens == 1): the selected experts' gate and up rows go through
//     the pipelined matvec (matvec.h; its waves split evenly over the slots,
//     each step a gate row and its up row), which stores h = silu(g) * u;
//     then one kernel runs every slot's down row for each output row and
//     combines the slots in order (moe_down_combine_kernel);
//   prefill (tokens > 1): the (token, slot) pairs are grouped by expert with
//     a stable counting sort (deterministic positions), each expert's group is
//     cut into tiles of 80 pairs, and one grouped GEMM launch
//     (gemm_x3.h: bf16 matrix cores, three exact products per FP32 product)
//     runs gate_up for every tile of every expert with SwiGLU in its
//     epilogue, then one runs down; a combine sums the slots of each token
//     in slot order from zero.
// No atomics touch any accumulated value, so results are deterministic.
#include "moe.h"

#include "gemm.h"
#include "gemm_x3.h"
#include "libm_expf.h"
#include "matvec.h"

namespace q3x {

constexpr int kRouterMaxExperts = 1024;
constexpr int kRouterMaxTopK = 8;          // q3x_model::MAX_TOP_K (model_config.h:14)
constexpr int kGroupThreads = 1024;
constexpr int kChunk = 1024;               // pairs per grouping chunk
// Grouped GEMM tiles (gemm_x3_kernel): at least kGrpBM pairs, which bounds
// the tile count the workspace holds.
constexpr int kGrpBM = 64;
// The grouped GEMMs issue a stage's matrix instructions before the next
// stage's conversion (gemm_x3_kernel's CF), which keeps their 80x32 wave
// tiles at two workgroups per CU: in kernel traces of one box gate_up
// 327-330 us against 334-336, down 166-168 against 168-171 (config 4).
constexpr bool kGrpCF = true;

// ---------------------------------------------------------------- router ----

// One token's routing in one wavefront; lane l holds experts [PER*l, PER*l +
// PER), so lane order is expert order.  The softmax is the reference's
// operation for operation (engine.cpp:380-387): the maximum (exact in any
// order), e = exp(l - max) with libm's expf arithmetic (libm_expf.h), the
// total added in expert order from zero, and p = e / total correctly
// rounded.  The total's order is sequential, so the wave writes e to LDS and
// every lane runs the same chain of adds over it (broadcast reads).  Then
// top_k argmax passes, each over keys (0 for an expert already chosen or
// past the end, else the probability's bits + 1: probabilities are >= 0, so
// their bits order like the values).  A lane keeps its best key (lowest
// index among equal ones); the wave's largest key is found with DPP and
// readlanes, and the lowest lane holding it wins, i.e. the lowest expert
// index among equal probabilities, as the reference's strict '>' scan picks.
// Weights = p / (sum of the selected p, added in slot order), correctly
// rounded (engine.cpp:388-404).  The phases below are shared by the two
// routers: router_topk_wave (ids and weights) and router_select_by_exp (ids
// alone, without the total when that is provably safe).

// The token's logits, PER per lane (-inf past the end).
template <int PER>
__device__ __forceinline__ void router_load(const float* __restrict__ row, int experts, float (&l)[PER]) {
    const int first = PER * (threadIdx.x & (kWave - 1));
#pragma unroll
    for (int j = 0; j < PER; ++j) l[j] = first + j < experts ? row[first + j] : -INFINITY;
}

// e = exp(l - max) in registers and in mine_p (LDS, 64 * PER floats; zeros
// past the end pad the last group of four).
template <int PER>
__device__ __forceinline__ void router_exps(const float (&l)[PER], int experts, float* __restrict__ mine_p,
                                            float (&e)[PER]) {
    const int first = PER * (threadIdx.x & (kWave - 1));
    float local_max = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) local_max = local_max < l[j] ? l[j] : local_max;
    const float maximum = wave_max_f32(local_max);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        e[j] = first + j < experts ? libm_expf(l[j] - maximum) : 0.0f;
        mine_p[first + j] = e[j];
    }
    wave_lds_sync();
}

// The softmax total, added in expert order from zero (every lane the same).
// The padding zeros add nothing: total + 0 == total for total >= +0.
__device__ __forceinline__ float router_total(const float* __restrict__ mine_p, int experts) {
    float total = 0.0f;
    const int groups4 = (experts + 3) / 4;
#pragma unroll 4
    for (int q = 0; q < groups4; ++q) {
        const f32x4 v = reinterpret_cast<const f32x4*>(mine_p)[q];
        total += v.x;
        total += v.y;
        total += v.z;
        total += v.w;
    }
    return total;
}

// `passes` argmax passes over the keys (see above): chosen[s] = the value of
// the s-th key, chosen_id[s] its expert (uniform).
template <int PER>
__device__ __forceinline__ void router_passes(uint32_t (&key)[PER], int passes, float (&chosen)[kRouterMaxTopK + 1],
                                              int (&chosen_id)[kRouterMaxTopK + 1]) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int slot = 0; slot < kRouterMaxTopK + 1; ++slot) {
        chosen[slot] = 0.0f;
        chosen_id[slot] = 0;
        if (slot >= passes) continue;
        uint32_t best = 0;
        int best_j = 0;
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (key[j] > best) { best = key[j]; best_j = j; }
        const uint32_t top = wave_max_u32(best);
        const unsigned long long holders = __ballot(best == top);
        const int winner = __builtin_ctzll(holders);
        chosen[slot] = __uint_as_float(top - 1u);
        chosen_id[slot] = PER * winner + static_cast<int>(read_lane_u32(static_cast<uint32_t>(best_j), winner));
        if (lane == winner) {
#pragma unroll
            for (int j = 0; j < PER; ++j)
                if (j == best_j) key[j] = 0u;
        }
    }
}

// Weights of the selected probabilities: p_s / (sum of p in slot order),
// correctly rounded; lane s < top_k returns slot s's.
__device__ __forceinline__ float router_slot_weight(const float (&chosen)[kRouterMaxTopK + 1], int top_k) {
    const int lane = threadIdx.x & (kWave - 1);
    float selected_total = 0.0f;
#pragma unroll
    for (int slot = 0; slot < kRouterMaxTopK; ++slot)
        if (slot < top_k) selected_total += chosen[slot];
    float mine = 0.0f;
#pragma unroll
    for (int slot = 0; slot < kRouterMaxTopK; ++slot)
        if (slot == lane) mine = chosen[slot];
    return __fdiv_rn(mine, selected_total);
}

__device__ __forceinline__ int lane_slot_id(const int (&chosen_id)[kRouterMaxTopK + 1]) {
    const int lane = threadIdx.x & (kWave - 1);
    int mine = 0;
#pragma unroll
    for (int slot = 0; slot < kRouterMaxTopK; ++slot)
        if (slot == lane) mine = chosen_id[slot];
    return mine;
}

// The full router: lane s < top_k returns slot s's expert and weight.
template <int PER>
__device__ __forceinline__ void router_topk_wave(const float* __restrict__ row, int experts, int top_k,
                                                 float* __restrict__ mine_p, int& out_id, float& out_weight) {
    const int first = PER * (threadIdx.x & (kWave - 1));
    float l[PER], e[PER];
    router_load<PER>(row, experts, l);
    router_exps<PER>(l, experts, mine_p, e);
    const float total = router_total(mine_p, experts);
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) key[j] = first + j < experts ? __float_as_uint(__fdiv_rn(e[j], total)) + 1u : 0u;
    float chosen[kRouterMaxTopK + 1];
    int chosen_id[kRouterMaxTopK + 1];
    router_passes<PER>(key, top_k, chosen, chosen_id);
    out_id = lane_slot_id(chosen_id);
    out_weight = router_slot_weight(chosen, top_k);
}

// The experts alone, ordered by e instead of p = e / total where that order
// is provably p's: dividing by the same total is monotone, equal e give
// equal p (ties keep the lowest index in either order), and two e more than
// 2^-21 apart (relative) stay strictly ordered after the division's rounding
// (each rounding moves a normal quotient by at most 2^-24 of it).  The e
// order's first top_k are the reference's ids in the reference's order when
// every class of equal e that reaches into the first top_k is that far above
// the next smaller e, since only then can no expert from below share a p
// with it and win by a lower index.  The passes see the top_k + 1 largest e,
// so the rule is: neighbours among the first top_k equal or that far apart,
// the pair at the boundary (positions top_k - 1 and top_k) that far apart and
// never equal -- a tie there hides the next smaller e, which may sit one ulp
// below with a lower index and round to the same p -- and the smallest of
// them at least 2^-100 (its quotient by a total of at most 1024 stays
// normal).  The total's 256-add chain is then skipped.  Returns false (and no
// ids) otherwise.
template <int PER>
__device__ __forceinline__ bool router_select_by_exp(const float* __restrict__ row, int experts, int top_k,
                                                     float* __restrict__ mine_p, int& out_id) {
    const int first = PER * (threadIdx.x & (kWave - 1));
    float l[PER], e[PER];
    router_load<PER>(row, experts, l);
    router_exps<PER>(l, experts, mine_p, e);
    uint32_t key[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) key[j] = first + j < experts ? __float_as_uint(e[j]) + 1u : 0u;
    const int passes = min(top_k + 1, experts);
    float chosen[kRouterMaxTopK + 1];
    int chosen_id[kRouterMaxTopK + 1];
    router_passes<PER>(key, passes, chosen, chosen_id);
    bool apart = true;
#pragma unroll
    for (int s = 0; s + 1 < kRouterMaxTopK + 1; ++s)
        if (s + 1 < passes) {
            const double a = chosen[s], b = chosen[s + 1];
            const bool gap = a >= b * (1.0 + 0x1p-21);
            apart = apart && (gap || (a == b && s + 1 < top_k));
        }
    float smallest = chosen[0];
#pragma unroll
    for (int s = 1; s < kRouterMaxTopK + 1; ++s)
        if (s < passes) smallest = chosen[s];
    out_id = lane_slot_id(chosen_id);
    return apart && smallest >= 0x1p-100f;
}

// One wavefront per token (router_topk_wave); lane s < top_k writes slot s.
// With ext_ids, the token's pairs also go to ext_ids / ext_weights [tokens,
// top_k + 1], slot top_k being the shared expert: id `experts`, weight
// sigmoid(shared_logit[token]) (engine.cpp:427-429).
template <int PER>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int tokens,
                                                          int experts, int top_k, int* __restrict__ ids,
                                                          float* __restrict__ weights, int* __restrict__ ext_ids,
                                                          float* __restrict__ ext_weights,
                                                          const float* __restrict__ shared_logit) {
    __shared__ __attribute__((aligned(16))) float probs[4][kRouterMaxExperts];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int token = blockIdx.x * 4 + wave;
    if (token >= tokens) return;  // whole waves leave together; no block barrier below
    int id;
    float weight;
    router_topk_wave<PER>(logits + static_cast<size_t>(token) * experts, experts, top_k, probs[wave], id, weight);
    if (lane < top_k) {
        ids[static_cast<size_t>(token) * top_k + lane] = id;
        weights[static_cast<size_t>(token) * top_k + lane] = weight;
    }
    if (ext_ids && lane <= top_k) {
        const size_t at = static_cast<size_t>(token) * (top_k + 1) + lane;
        ext_ids[at] = lane < top_k ? id : experts;
        ext_weights[at] = lane < top_k ? weight : sigmoid_ref(shared_logit[token]);
    }
}

// The decode gate_up rows of ExpertGateUpRows, the experts chosen inside the
// launch: route() selects the token's experts from its logits in wave 0 of
// every workgroup -- a workgroup needs only the selection, and computing it
// where it is used spares the router its own launch -- and keeps the ids in
// LDS for for_wave.  Workgroup 0 runs the full router (router_topk_wave) and
// stores ids and weights to ids_out / weights_out for the down-and-combine
// launch and the caller; the others take router_select_by_exp's ids where it
// applies (no total: the 256-add chain off their critical path), else the
// full router's.  Every workgroup selects the same ids in the same order.
// Workgroup 0 starts first, so its longer routing rarely delays the launch.
struct RoutedGateUpRows : ExpertGateUpRows {
    static constexpr uint32_t kRouteLds = 64 + 4 * kRouterMaxExperts;  // ids, weights, probabilities
    const float* logits;
    int top_k;
    int* ids_out;
    float* weights_out;
    __device__ const int* route(uint8_t* lds) const {
        int* chosen = reinterpret_cast<int*>(lds);
        float* chosen_w = reinterpret_cast<float*>(lds + 32);
        float* probs = reinterpret_cast<float*>(lds + 64);
        if (threadIdx.x < kWave) {
            const int lane = threadIdx.x;
            int id = 0;
            float w = 0.0f;
            // Workgroup 0 needs the weights too; the others only the ids.
            const bool by_exp = blockIdx.x != 0 && experts <= 4 * kWave &&
                                router_select_by_exp<4>(logits, experts, top_k, probs, id);
            if (!by_exp) {
                if (experts <= 4 * kWave) router_topk_wave<4>(logits, experts, top_k, probs, id, w);
                else if (experts <= 8 * kWave) router_topk_wave<8>(logits, experts, top_k, probs, id, w);
                else router_topk_wave<16>(logits, experts, top_k, probs, id, w);
            }
            if (lane < top_k) {
                chosen[lane] = id;
                chosen_w[lane] = w;
                if (blockIdx.x == 0) {
                    ids_out[lane] = id;
                    weights_out[lane] = w;
                }
            }
        }
        __syncthreads();
        return chosen;
    }
};

// ------------------------------------------------------------ workspace ----

struct MoeLayout {
    size_t ntiles, nvalid, tile_expert, tile_start, tile_count, pos_of_pair, src_token;
    size_t chunk_counts;
    int chunks;
    size_t gu, h, d, total;
    int max_tiles;
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

inline MoeLayout moe_layout(int tokens, int experts, int top_k, int H, int I) {
    MoeLayout L{};
    const size_t P = static_cast<size_t>(tokens) * top_k;
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t at = off; off = align_up(off + bytes, 256); return at; };
    {  // grouping arrays (also for one token: the fallback of unaligned decode shapes)
        L.max_tiles = static_cast<int>(P / kGrpBM + std::min<size_t>(experts, P) + 1);
        L.ntiles = take(sizeof(int));
        L.nvalid = take(sizeof(int));
        L.tile_expert = take(sizeof(int) * L.max_tiles);
        L.tile_start = take(sizeof(int) * L.max_tiles);
        L.tile_count = take(sizeof(int) * L.max_tiles);
        L.pos_of_pair = take(sizeof(int) * P);
        L.src_token = take(sizeof(int) * P);
        L.chunks = static_cast<int>((P + kChunk - 1) / kChunk);
        L.chunk_counts = take(sizeof(int) * static_cast<size_t>(L.chunks) * experts);
    }
    L.gu = take(sizeof(float) * P * 2 * I);
    L.h = take(sizeof(float) * P * I);
    L.d = take(sizeof(float) * P * H);
    L.total = off;
    return L;
}

// ------------------------------------------------------------- grouping ----

// Exclusive scan of v over the kGroupThreads threads of the workgroup
// (integers, so exact in any order): a shuffle scan inside each wave, then
// each wave adds the totals of the waves before it (buf: kGroupThreads /
// kWave ints of LDS).  Two barriers; the second frees buf for the next call.
__device__ int block_exclusive_scan(int v, int* buf) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    int x = v;
#pragma unroll
    for (int offset = 1; offset < kWave; offset <<= 1) {
        const int y = __shfl_up(x, offset);
        if (lane >= offset) x += y;
    }
    if (lane == kWave - 1) buf[wave] = x;
    __syncthreads();
    int before = 0;
    for (int w = 0; w < wave; ++w) before += buf[w];
    __syncthreads();
    return before + x - v;
}

// Stable counting sort of the (token, slot) pairs by expert, in two
// launches: per chunk of kChunk pairs, the expert histogram and each pair's
// rank -- the number of earlier pairs of its chunk with the same expert:
// within a wave the lanes with the same id found by one ballot per distinct
// id, across the chunk's waves an exclusive sum of the waves' counts
// (moe_rank_kernel); then a workgroup per chunk that sums the histograms
// into its chunk's base for every expert (group start plus the expert's
// pairs in earlier chunks) and places its pairs at base + rank, workgroup 0
// also writing the tile table (moe_place_kernel).  Every expert's group
// therefore lists its pairs in (token, slot) order and positions are
// identical on every run.  Pairs with an id outside [0, experts) get
// position -1.
__global__ __launch_bounds__(kChunk) void moe_rank_kernel(const int* __restrict__ ids, int P, int experts,
                                                          int* __restrict__ chunk_counts, int* __restrict__ rank_of_pair) {
    constexpr int kWaves = kChunk / kWave;
    __shared__ int wave_count[kWaves][kRouterMaxExperts];  // per wave and expert: count, then exclusive base
    for (int i = threadIdx.x; i < kWaves * experts; i += kChunk) wave_count[i / experts][i % experts] = 0;
    __syncthreads();
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int p = blockIdx.x * kChunk + threadIdx.x;
    const int e = p < P ? ids[p] : -1;
    const bool valid = e >= 0 && e < experts;
    // Lanes of this wave with the same id: one ballot per distinct id.
    uint64_t same = 0;
    uint64_t open = __ballot(1);
    while (open) {
        const int v = __builtin_amdgcn_readlane(e, __builtin_ctzll(open));
        const uint64_t m = __ballot(e == v);
        if (e == v) same = m;
        open &= ~m;
    }
    const int rank_in_wave = __popcll(same & ((1ull << lane) - 1));
    if (valid && rank_in_wave == 0) wave_count[wave][e] = __popcll(same);
    __syncthreads();
    for (int x = threadIdx.x; x < experts; x += kChunk) {
        int run = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const int c = wave_count[w][x];
            wave_count[w][x] = run;
            run += c;
        }
        chunk_counts[static_cast<size_t>(blockIdx.x) * experts + x] = run;
    }
    __syncthreads();
    if (p < P) rank_of_pair[p] = valid ? wave_count[wave][e] + rank_in_wave : -1;
}

__global__ __launch_bounds__(kGroupThreads) void moe_place_kernel(
    const int* __restrict__ chunk_counts, int chunks, int experts, int bm, int* __restrict__ tile_expert,
    int* __restrict__ tile_start, int* __restrict__ tile_count, int* __restrict__ ntiles, int* __restrict__ nvalid,
    const int* __restrict__ ids, int P, int top_k, int* __restrict__ pos_of_pair, int* __restrict__ src_token) {
    static_assert(kChunk == kGroupThreads, "one workgroup per chunk, a pair per thread");
    __shared__ int buf[kGroupThreads];
    __shared__ int chunk_base[kRouterMaxExperts];
    const int e = threadIdx.x;
    const bool owner = e < experts;
    // Expert e's pairs in all chunks and in the chunks before this one.
    int total = 0, before = 0;
    if (owner) {
#pragma unroll 8
        for (int c = 0; c < chunks; ++c) {
            const int v = chunk_counts[static_cast<size_t>(c) * experts + e];
            before += c < static_cast<int>(blockIdx.x) ? v : 0;
            total += v;
        }
    }
    const int start = block_exclusive_scan(total, buf);
    if (owner) chunk_base[e] = start + before;
    if (blockIdx.x == 0) {
        const int tiles = owner ? (total + bm - 1) / bm : 0;
        const int tile0 = block_exclusive_scan(tiles, buf);
        for (int j = 0; j < tiles; ++j) {
            tile_expert[tile0 + j] = e;
            tile_start[tile0 + j] = start + j * bm;
            tile_count[tile0 + j] = min(bm, total - j * bm);
        }
        if (e == kGroupThreads - 1) { *ntiles = tile0 + tiles; *nvalid = start + total; }
    }
    __syncthreads();
    // This chunk's pairs at base + rank (moe_rank_kernel's rank, in place in
    // pos_of_pair).
    const int p = blockIdx.x * kChunk + threadIdx.x;
    if (p < P) {
        const int rank = pos_of_pair[p];
        if (rank >= 0) {
            const int pos = chunk_base[ids[p]] + rank;
            pos_of_pair[p] = pos;
            src_token[pos] = p / top_k;
        }
    }
}

// Grouped GEMM policy: tile ty is the tile table's entry; A rows are
// gathered (a_index[position] = source row) or taken in position order; the
// weights are expert tile_expert[ty] of the pool; out[position, n].
struct GroupedGemm {
    // A 1-D grid sized for the most tiles possible; the live ones, *ntiles
    // A-row tiles times tiles_x, are remapped so that the weight-row tiles of
    // one A-row tile (which read the same gathered A rows) share an XCD.
    static constexpr bool kLinearGrid = true;
    static constexpr bool kPairedColumns = false;
    static constexpr bool kPartialTiles = true;  // every expert's last tile is short
    static constexpr bool kMfma16 = true;        // skip 16-row halves past the valid pairs
    int tiles_x;  // weight-row tiles
    const float* A;
    int a_cols;
    const int* a_index;
    const uint8_t* pool;
    size_t expert_bytes;
    size_t row_bytes;
    const int* tile_expert;
    const int* tile_start;
    const int* tile_count;
    const int* ntiles;
    float* out;
    int out_cols;
    // A shared expert grouped as expert shared_group: its own matrix
    // (shared_rows; for the gate_up GEMM the gate, shared_up the up).
    int shared_group = -1;
    const uint8_t* shared_rows = nullptr;
    const uint8_t* shared_up = nullptr;
    __device__ int linear_total() const { return *ntiles * tiles_x; }
    __device__ bool tile(int ty, int, GemmTile& t) const {
        if (ty >= *ntiles) return false;
        t.group = tile_expert[ty];
        t.m0 = tile_start[ty];
        t.mcount = tile_count[ty];
        return true;
    }
    __device__ const float* a_row(const GemmTile& t, int m) const {
        const int pos = t.m0 + m;
        const int row = a_index ? a_index[pos] : pos;
        return A + static_cast<size_t>(row) * a_cols;
    }
    __device__ const uint8_t* b_row(const GemmTile& t, int n) const {
        if (t.group == shared_group) return shared_rows + static_cast<size_t>(n) * row_bytes;
        return pool + static_cast<size_t>(t.group) * expert_bytes + static_cast<size_t>(n) * row_bytes;
    }
    __device__ void store(const GemmTile& t, int m, int n, float v) const {
        out[static_cast<size_t>(t.m0 + m) * out_cols + n] = v;
    }
    __device__ void store_pair(const GemmTile&, int, int, float, float) const {}
};

// The gate_up grouped GEMM with SwiGLU in its epilogue.  Tile column block
// bx covers outputs j in [64 bx, 64 bx + 64): its 32-row subtile s holds the
// gate rows j = 64 bx + 16 s + q (q < 16) followed by the matching up rows
// I + j, so the kernel pairs column q with q + 16 and this policy stores
// h[pos, j] = silu(gate) * up (engine.cpp:415-416) instead of gate_up.
struct GroupedGateUp : GroupedGemm {
    static constexpr bool kPairedColumns = true;
    int I;
    float* h;
    __device__ static int out_col(int n) { return 64 * (n >> 7) + 16 * ((n >> 5) & 3) + (n & 15); }
    __device__ const uint8_t* b_row(const GemmTile& t, int n) const {
        const int j = out_col(n);
        if (t.group == shared_group) return ((n & 16) ? shared_up : shared_rows) + static_cast<size_t>(j) * row_bytes;
        const int row = (n & 16) ? I + j : j;
        return pool + static_cast<size_t>(t.group) * expert_bytes + static_cast<size_t>(row) * row_bytes;
    }
    __device__ void store_pair(const GemmTile& t, int m, int n, float gate, float up) const {
        h[static_cast<size_t>(t.m0 + m) * I + out_col(n)] = silu_ref(gate) * up;
    }
};

// h[pos, j] = silu(gu[pos, j]) * gu[pos, I + j] for pos < *count
// (engine.cpp:415-416).  count == nullptr: `limit` rows.
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gu, float* __restrict__ h,
                                                     int I, int limit, const int* __restrict__ count) {
    const int rows = count ? *count : limit;
    const size_t total = static_cast<size_t>(rows) * I;
    for (size_t idx = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; idx < total;
         idx += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t pos = idx / I, j = idx % I;
        const float g = gu[pos * 2 * I + j];
        const float u = gu[pos * 2 * I + I + j];
        h[idx] = silu_ref(g) * u;
    }
}

// Y[t, i] (+)= sum over slots, in slot order from zero, of
// weights[t, slot] * d[pos, i] (engine.cpp:411, 418-419: out = 0 then
// out += w * d per slot).  pos = pos_of_pair[t*top_k + slot] (grouped) or the
// slot itself (decode); slots with an out-of-range expert id are skipped.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ d, const int* __restrict__ pos_of_pair,
                                                      const int* __restrict__ ids, int experts,
                                                      const float* __restrict__ weights, int tokens, int top_k,
                                                      int H, float* __restrict__ Y, int accumulate) {
    const size_t idx = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    if (idx >= static_cast<size_t>(tokens) * H) return;
    const int t = static_cast<int>(idx / H), i = static_cast<int>(idx % H);
    float acc = 0.0f;
    for (int slot = 0; slot < top_k; ++slot) {
        const int pair = t * top_k + slot;
        int pos;
        if (pos_of_pair) {
            pos = pos_of_pair[pair];
        } else {
            const int e = ids[pair];
            pos = (e >= 0 && e < experts) ? slot : -1;
        }
        if (pos < 0) continue;
        acc = fmaf(weights[pair], d[static_cast<size_t>(pos) * H + i], acc);
    }
    if (accumulate) Y[idx] += acc;
    else Y[idx] = acc;
}

// combine_kernel over four consecutive outputs per thread (16-byte loads and
// stores; H % 4 == 0, d and Y 16-byte aligned), same arithmetic per element.
__global__ __launch_bounds__(256) void combine4_kernel(const float* __restrict__ d,
                                                       const int* __restrict__ pos_of_pair,
                                                       const float* __restrict__ weights, int tokens, int top_k,
                                                       int H, float* __restrict__ Y, int accumulate) {
    const size_t idx = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x;
    const int H4 = H / 4;
    if (idx >= static_cast<size_t>(tokens) * H4) return;
    const int t = static_cast<int>(idx / H4), i4 = static_cast<int>(idx % H4);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int slot = 0; slot < top_k; ++slot) {
        const int pair = t * top_k + slot;
        const int pos = pos_of_pair[pair];
        if (pos < 0) continue;
        const float w = weights[pair];
        const f32x4 v = reinterpret_cast<const f32x4*>(d + static_cast<size_t>(pos) * H)[i4];
        acc.x = fmaf(w, v.x, acc.x);
        acc.y = fmaf(w, v.y, acc.y);
        acc.z = fmaf(w, v.z, acc.z);
        acc.w = fmaf(w, v.w, acc.w);
    }
    f32x4* out = reinterpret_cast<f32x4*>(Y + static_cast<size_t>(t) * H) + i4;
    if (accumulate) {
        const f32x4 y = *out;
        acc.x += y.x; acc.y += y.y; acc.z += y.z; acc.w += y.w;
    }
    *out = acc;
}

// The MoE layer's shared expert (engine.cpp:422-429) as the decode kernels
// see it: gate / up [I, H], down [H, I], and the logit whose sigmoid weighs
// its output.  down == nullptr: routed experts only.
struct SharedExpert {
    const uint8_t* gate = nullptr;
    const uint8_t* up = nullptr;
    const uint8_t* down = nullptr;
    int I = 0;
    const float* logit = nullptr;
};

// Decode (one token): the down projection of every selected expert, its
// input h = silu(g) * u (engine.cpp:415-416, from the paired gate_up matvec)
// staged in LDS, and the slot-order combine (engine.cpp:411, 418-419:
// out = 0, then out += w * d per slot), in one kernel.  Wave gw computes the
// output rows i = gw, gw + GW, ...: for each, the rows (slot s, i) of the
// top_k experts, G = 64 / LPR slots at a time (one row group of LPR lanes per
// slot, one lane per 32-weight block of a pass), then lane 0 adds the slots'
// results in slot order from zero.  Slots whose id is out of range are
// skipped.  With a shared expert, it is one more slot after the routed ones
// (its h zero past shared.I), added last with weight sigmoid(*shared.logit)
// (engine.cpp:427-429).
template <uint32_t QT, int LPR, int MAXS>
__global__ __launch_bounds__(512) void moe_down_combine_kernel(
    const uint8_t* __restrict__ down, size_t expert_bytes, size_t row_bytes, int experts,
    const int* __restrict__ ids, const float* __restrict__ weights, int top_k, const float* __restrict__ h,
    int I, int H, float* __restrict__ Y, int accumulate, SharedExpert shared) {
    using S = PipeShape<QT, LPR>;
    constexpr int BB = S::BB, G = S::G, J = S::J;
    constexpr int IT = (MAXS + G - 1) / G;  // slot groups at most (MAXS: top_k, +1 with a shared expert)
    constexpr bool Q4 = QT == Q3X_HIP_MATRIX_Q4_0;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_dyn[];

    const int bpr = I / kBlock;
    const uint32_t xs_bytes = pipe_x_bytes(bpr);  // one slot's activations
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int wpb = blockDim.x / kWave;
    const int gw = blockIdx.x * wpb + wave;
    const int GW = gridDim.x * wpb;
    const int g = lane / LPR;
    const int li = lane % LPR;
    // Only the build with a slot to spare carries the shared expert's code.
    const bool has_shared = MAXS > kRouterMaxTopK && shared.down != nullptr;
    const int slots = top_k + (has_shared ? 1 : 0);
    uint8_t* const wl = lds_dyn + slots * xs_bytes + wave * S::WAVE_LDS;

    const int npass = (bpr + LPR - 1) / LPR;
    const int groups = (slots + G - 1) / G;
    const int my_steps = gw < H ? (H - gw + GW - 1) / GW * npass : 0;
    constexpr int kShared = -2;
    // The selected experts (uniform); an id out of range reads as zeros.
    int expert[IT * G];
#pragma unroll
    for (int slot = 0; slot < IT * G; ++slot) {
        const int e = slot < top_k ? __builtin_amdgcn_readfirstlane(ids[slot]) : -1;
        expert[slot] = slot == top_k && has_shared ? kShared : e >= 0 && e < experts ? e : -1;
    }
    const size_t shared_row_bytes = static_cast<size_t>(shared.I / kBlock) * BB;
    const int shared_bpr = shared.I / kBlock;
    // Weight segments of one step (output row i, pass) for every slot group;
    // `live` false gives zeros without touching memory.
    u32x4 pre[IT][G][J];
    auto issue = [&](int i, int pass, int it, bool live) {
        const int b0 = pass * LPR;
        const int nblk = min(LPR, bpr - b0);
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            const int e = expert[it * G + gg];
            const uint8_t* src = down;
            int bytes = 0;
            if (live && e >= 0) {
                src = down + static_cast<size_t>(e) * expert_bytes + static_cast<size_t>(i) * row_bytes +
                      static_cast<size_t>(b0) * BB;
                bytes = nblk * BB;
            } else if (live && e == kShared && b0 < shared_bpr) {
                src = shared.down + static_cast<size_t>(i) * shared_row_bytes + static_cast<size_t>(b0) * BB;
                bytes = min(LPR, shared_bpr - b0) * BB;
            }
            const __amdgpu_buffer_rsrc_t rsrc =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(src), 0, bytes, kBufferFlags);
#pragma unroll
            for (int j = 0; j < J; ++j)
                pre[it][gg][j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, 16 * lane + 1024 * j, 0, kNonTemporal);
        }
    };
    // h of every slot into the padded x layout: its loads go out first (they
    // return from L2), then the first step's weights, whose latency overlaps
    // the copy.
    constexpr int kHPerThread = 8;
    float hv[kHPerThread];
    const int hn = slots * I;
    // The shared slot's h holds shared.I values; the rest of its row is zero.
    auto h_at = [&](int c) { return c >= top_k * I + shared.I ? 0.0f : h[c]; };
#pragma unroll
    for (int k = 0; k < kHPerThread; ++k) {
        const int c = threadIdx.x + k * static_cast<int>(blockDim.x);
        hv[k] = c < hn ? h_at(c) : 0.0f;
    }
#pragma unroll
    for (int it = 0; it < IT; ++it)
        if (it < groups) issue(gw, 0, it, my_steps > 0);
    auto put_h = [&](int c, float v) {
        const int slot = c / I, j = c - slot * I;
        *reinterpret_cast<float*>(lds_dyn + slot * xs_bytes + x_block_offset(j >> 5) + 4 * (j & 31)) = v;
    };
#pragma unroll
    for (int k = 0; k < kHPerThread; ++k) {
        const int c = threadIdx.x + k * static_cast<int>(blockDim.x);
        if (c < hn) put_h(c, hv[k]);
    }
    for (int c = threadIdx.x + kHPerThread * static_cast<int>(blockDim.x); c < hn; c += blockDim.x)
        put_h(c, h_at(c));
    __syncthreads();

    const float shared_weight = has_shared ? sigmoid_ref(*shared.logit) : 0.0f;
    float acc[IT];
    int ci = gw, cp = 0;  // current step: output row, pass
    for (int s = 0; s < my_steps; ++s) {
        int ni = ci, np = cp + 1;
        if (np == npass) { np = 0; ni += GW; }
        const bool more = s + 1 < my_steps;
        const int b0 = cp * LPR;
        const int nblk = min(LPR, bpr - b0);
        const int col = li < nblk ? b0 + li : 0;
        if (cp == 0) {
#pragma unroll
            for (int it = 0; it < IT; ++it) acc[it] = 0.0f;
        }
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            if (it >= groups) continue;  // uniform: the trip count stays IT, so the loop unrolls
            // x of this lane's slot, block col.
            const int my_slot = it * G + g;
            const uint8_t* xs = lds_dyn + (my_slot < slots ? my_slot : 0) * xs_bytes;
            float xv[32];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const f32x4 t = *reinterpret_cast<const f32x4*>(xs + x_block_offset(col) + 16 * q);
                xv[4 * q + 0] = t.x; xv[4 * q + 1] = t.y; xv[4 * q + 2] = t.z; xv[4 * q + 3] = t.w;
            }
#pragma unroll
            for (int gg = 0; gg < G; ++gg)
#pragma unroll
                for (int j = 0; j < J; ++j)
                    *reinterpret_cast<u32x4*>(wl + gg * S::SEGP + 1024 * j + 16 * lane) = pre[it][gg][j];
            issue(ni, np, it, more);  // the next step's segments of this slot group
            wave_lds_sync();
            if (li < nblk && my_slot < slots) {
                const uint32_t p = g * S::SEGP + li * BB;
                acc[it] += Q4 ? block_dot_q4_exact(wl, p, xv) : block_dot_q8(wl, p, xv);
            }
            wave_lds_sync();
        }
        if (cp == npass - 1) {
            // Slot results to lane 0, then the ordered combine.
            float out = 0.0f;
#pragma unroll
            for (int it = 0; it < IT; ++it) {
                if (it >= groups) continue;
                const float total = group_sum<LPR>(acc[it]);
#pragma unroll
                for (int gg = 0; gg < G; ++gg) {
                    const int slot = it * G + gg;
                    const float d = read_lane_f32(total, gg * LPR);
                    if (slot < top_k && expert[slot] >= 0) out = fmaf(weights[slot], d, out);
                    if (expert[slot] == kShared) out = fmaf(shared_weight, d, out);
                }
            }
            if (lane == 0) Y[ci] = accumulate ? Y[ci] + out : out;
        }
        ci = ni;
        cp = np;
    }
}

template <uint32_t QT, int LPR>
int launch_moe_down(const uint8_t* down, int experts, int H, int I, const int* ids, const float* weights,
                    int top_k, const float* h, float* Y, int accumulate, const SharedExpert& shared,
                    hipStream_t stream) {
    using S = PipeShape<QT, LPR>;
    constexpr int kWaves = 8;
    const size_t row_bytes = static_cast<size_t>(I / kBlock) * (QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes);
    const int slots = top_k + (shared.down ? 1 : 0);
    const size_t lds = static_cast<size_t>(slots) * pipe_x_bytes(I / kBlock) + kWaves * S::WAVE_LDS;
    if (lds > kLdsPerCU) return Q3X_HIP_ENOTSUP;
    // Slot capacity: the routed experts alone keep the smaller register set.
    auto kernel = shared.down ? moe_down_combine_kernel<QT, LPR, kRouterMaxTopK + 1>
                              : moe_down_combine_kernel<QT, LPR, kRouterMaxTopK>;
    static const bool lds_ready =
        hipFuncSetAttribute(reinterpret_cast<const void*>(moe_down_combine_kernel<QT, LPR, kRouterMaxTopK + 1>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsPerCU)) == hipSuccess &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(moe_down_combine_kernel<QT, LPR, kRouterMaxTopK>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsPerCU)) == hipSuccess;
    if (lds > 64 * 1024 && !lds_ready) return Q3X_HIP_ERUNTIME;
    const int grid = std::min((H + kWaves - 1) / kWaves, kCUs * 2);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(kWaves * kWave), lds, stream, down, row_bytes * H, row_bytes,
                       experts, ids, weights, top_k, h, I, H, Y, accumulate, shared);
    return launch_status();
}

// Decode (one token).  With `logits`, the gate_up launch routes the token
// itself (RoutedGateUpRows) and writes ids / weights, which the down launch
// then reads: two launches for router and experts.
template <uint32_t QT>
int moe_decode(const uint8_t* gate_up, const uint8_t* down, int experts, int H, int I, const float* X,
               const int* ids, const float* weights, int top_k, float* Y, int accumulate,
               uint8_t* ws, const MoeLayout& L, const SharedExpert& shared, hipStream_t stream,
               const uint16_t* norm_w = nullptr, const float* logits = nullptr, int* ids_out = nullptr,
               float* weights_out = nullptr) {
    constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    float* h = reinterpret_cast<float*>(ws + L.gu);  // [top_k (+1), I]
    const size_t gu_row = static_cast<size_t>(H / kBlock) * BB;
    const size_t down_row = static_cast<size_t>(I / kBlock) * BB;
    const size_t shared_down_row = static_cast<size_t>(shared.I / kBlock) * BB;
    const bool shared_ok = !shared.down || (aligned(shared.gate, 16) && aligned(shared.up, 16) &&
                                            aligned(shared.down, 16) && shared_down_row % 16 == 0);
    const bool staged = aligned(gate_up, 16) && aligned(X, 16) && gu_row % 16 == 0 && aligned(down, 16) &&
                        down_row % 16 == 0 && shared_ok;
    if (staged) {
        const int slots = top_k + (shared.down ? 1 : 0);
        ExpertGateUpRows gate{};
        static_cast<ExpertRows&>(gate) = ExpertRows{gate_up, gu_row * 2 * I, gu_row, 2 * I, experts, ids, slots, X, h, {}};
        gate.I = I;
        gate.shared_gate = shared.down ? shared.gate : nullptr;
        gate.shared_up = shared.up;
        gate.shared_I = shared.I;
        // One 64-lane row group, two row iterations (gate, up) per step.
        // With norm_w, X is the raw residual, normalised in the staging.
        int status;
        if (logits) {
            RoutedGateUpRows routed{};
            static_cast<ExpertGateUpRows&>(routed) = gate;
            routed.logits = logits;
            routed.top_k = top_k;
            routed.ids_out = ids_out;
            routed.weights_out = weights_out;
            ids = ids_out;
            weights = weights_out;
            status = norm_w ? launch_pipe<QT, 64, 2, RoutedGateUpRows, 1, 4, NormInput>(
                                  routed, slots * 2 * I, H / kBlock, 16, stream, 2, NormInput{norm_w})
                            : launch_pipe<QT, 64, 2, RoutedGateUpRows>(routed, slots * 2 * I, H / kBlock, 16, stream, 2);
        } else {
            status = norm_w ? launch_pipe<QT, 64, 2, ExpertGateUpRows, 1, 4, NormInput>(
                                  gate, slots * 2 * I, H / kBlock, 16, stream, 2, NormInput{norm_w})
                            : launch_pipe<QT, 64, 2>(gate, slots * 2 * I, H / kBlock, 16, stream, 2);
        }
        if (status == Q3X_HIP_OK) {
            const int bpr = I / kBlock;
            status = bpr <= 16   ? launch_moe_down<QT, 16>(down, experts, H, I, ids, weights, top_k, h, Y,
                                                           accumulate, shared, stream)
                     : bpr <= 32 ? launch_moe_down<QT, 32>(down, experts, H, I, ids, weights, top_k, h, Y,
                                                           accumulate, shared, stream)
                                 : launch_moe_down<QT, 64>(down, experts, H, I, ids, weights, top_k, h, Y,
                                                           accumulate, shared, stream);
        }
        if (status != Q3X_HIP_ENOTSUP) return status;
    }
    // Unaligned or very wide shapes: the caller takes the grouped path, which
    // handles one token too.
    return Q3X_HIP_ENOTSUP;
}

// A shared expert that the grouped GEMMs take as group `group` (its gate,
// up and down matrices of the routed experts' shapes); group -1: none.
struct GroupedShared {
    int group = -1;
    const uint8_t* gate = nullptr;
    const uint8_t* up = nullptr;
    const uint8_t* down = nullptr;
};

template <uint32_t QT, int WM, int WN, int SM, int SN>
int moe_grouped_tiles(const uint8_t* gate_up, const uint8_t* down, int experts, int H, int I, const float* X,
                int tokens, const int* ids, const float* weights, int top_k, float* Y, int accumulate,
                uint8_t* ws, const MoeLayout& L, hipStream_t stream, const GroupedShared& shared) {
    constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    constexpr int BM = WM * SM * 16, BN = WN * SN * 16, NT = WM * WN * kWave;
    static_assert(BM >= kGrpBM, "the workspace bounds the tile count for kGrpBM-pair tiles");
    const int P = tokens * top_k;
    int* ntiles = reinterpret_cast<int*>(ws + L.ntiles);
    int* nvalid = reinterpret_cast<int*>(ws + L.nvalid);
    int* tile_expert = reinterpret_cast<int*>(ws + L.tile_expert);
    int* tile_start = reinterpret_cast<int*>(ws + L.tile_start);
    int* tile_count = reinterpret_cast<int*>(ws + L.tile_count);
    int* pos_of_pair = reinterpret_cast<int*>(ws + L.pos_of_pair);
    int* src_token = reinterpret_cast<int*>(ws + L.src_token);
    float* gu = reinterpret_cast<float*>(ws + L.gu);
    float* h = reinterpret_cast<float*>(ws + L.h);
    float* d = reinterpret_cast<float*>(ws + L.d);

    int* chunk_counts = reinterpret_cast<int*>(ws + L.chunk_counts);
    hipLaunchKernelGGL(moe_rank_kernel, dim3(L.chunks), dim3(kChunk), 0, stream, ids, P, experts, chunk_counts,
                       pos_of_pair);
    int status = launch_status();
    if (status != Q3X_HIP_OK) return status;
    hipLaunchKernelGGL(moe_place_kernel, dim3(L.chunks), dim3(kGroupThreads), 0, stream,
                       static_cast<const int*>(chunk_counts), L.chunks, experts, BM, tile_expert, tile_start,
                       tile_count, ntiles, nvalid, ids, P, top_k, pos_of_pair, src_token);
    if ((status = launch_status()) != Q3X_HIP_OK) return status;

    const size_t gu_row = static_cast<size_t>(H / kBlock) * BB;
    const size_t down_row = static_cast<size_t>(I / kBlock) * BB;
    const int tiles_bound = L.max_tiles;
    if (I % 64 == 0) {
        // SwiGLU in the gate_up epilogue: h directly.
        GroupedGateUp g1{};
        const int nx = (2 * I + BN - 1) / BN;
        static_cast<GroupedGemm&>(g1) = GroupedGemm{nx, X, H, src_token, gate_up, gu_row * 2 * I, gu_row,
                                                    tile_expert, tile_start, tile_count, ntiles, nullptr, 0};
        g1.I = I;
        g1.h = h;
        g1.shared_group = shared.group;
        g1.shared_rows = shared.gate;
        g1.shared_up = shared.up;
        hipLaunchKernelGGL((gemm_x3_kernel<QT, WM, WN, SM, SN, GroupedGateUp, 1, kGrpCF>), dim3(nx * tiles_bound), dim3(NT), 0,
                           stream, g1, 2 * I, H);
        if ((status = launch_status()) != Q3X_HIP_OK) return status;
    } else {
        if (shared.group >= 0) return Q3X_HIP_ENOTSUP;  // a shared group needs the paired gate_up
        const int nx = (2 * I + BN - 1) / BN;
        GroupedGemm g1{nx, X, H, src_token, gate_up, gu_row * 2 * I, gu_row, tile_expert, tile_start, tile_count,
                       ntiles, gu, 2 * I};
        hipLaunchKernelGGL((gemm_x3_kernel<QT, WM, WN, SM, SN, GroupedGemm, 1, kGrpCF>), dim3(nx * tiles_bound), dim3(NT), 0,
                           stream, g1, 2 * I, H);
        if ((status = launch_status()) != Q3X_HIP_OK) return status;
        const size_t sw = static_cast<size_t>(P) * I;
        const int sw_blocks = static_cast<int>(std::min<size_t>((sw + 255) / 256, 65536));
        hipLaunchKernelGGL(swiglu_kernel, dim3(sw_blocks), dim3(256), 0, stream, gu, h, I, 0,
                           static_cast<const int*>(nvalid));
        if ((status = launch_status()) != Q3X_HIP_OK) return status;
    }
    const int nx2 = (H + BN - 1) / BN;
    GroupedGemm g2{nx2, h, I, nullptr, down, down_row * H, down_row, tile_expert, tile_start, tile_count,
                   ntiles, d, H};
    g2.shared_group = shared.group;
    g2.shared_rows = shared.down;
    hipLaunchKernelGGL((gemm_x3_kernel<QT, WM, WN, SM, SN, GroupedGemm, 1, kGrpCF>), dim3(nx2 * tiles_bound), dim3(NT), 0,
                       stream, g2, H, I);
    if ((status = launch_status()) != Q3X_HIP_OK) return status;
    const size_t outs = static_cast<size_t>(tokens) * H;
    if (H % 4 == 0 && aligned(Y, 16)) {
        hipLaunchKernelGGL(combine4_kernel, dim3(static_cast<unsigned>((outs / 4 + 255) / 256)), dim3(256), 0,
                           stream, d, pos_of_pair, weights, tokens, top_k, H, Y, accumulate);
        return launch_status();
    }
    hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>((outs + 255) / 256)), dim3(256), 0,
                       stream, d, pos_of_pair, ids, experts, weights, tokens, top_k, H, Y, accumulate);
    return launch_status();
}

template <uint32_t QT>
int moe_grouped(const uint8_t* gate_up, const uint8_t* down, int experts, int H, int I, const float* X,
                int tokens, const int* ids, const float* weights, int top_k, float* Y, int accumulate,
                uint8_t* ws, const MoeLayout& L, hipStream_t stream, const GroupedShared& shared = {}) {
    // 80 pairs x 256 weight rows on 8 waves of 80x32.  At 2048 tokens x top
    // 8 of 256 experts an expert averages 64 pairs (standard deviation about
    // 8): 64-pair tiles give about half of the experts a second, nearly
    // empty tile that brings the expert's weight rows into the CU again (378
    // tiles for 256 experts at config 4), 80-pair tiles give 261, and the
    // 80x32 wave tile keeps the register count at 128, so two workgroups
    // still share a CU.  Alternating runs of one box at config 4: 197-201
    // TFLOP/s against 188-192 for 64 x 256 on 8 waves of 32x64; 96 x 256 on
    // 12 waves of 32x64 (one workgroup a CU) 191-193, on 8 waves of 48x64
    // (164 registers) 182.  Earlier, with 64-pair tiles: 64 x 128 on 32x32
    // waves, 64 x 512 on 8 waves of 64x64 or 32x128, 64 x 256 on 8 waves of
    // 64x32, on 4 of 64x64 or on 16 of 32x32, and 64 x 128 on 4 waves of
    // 32x64 all ran slower than 64 x 256 on 32x64 waves.
    return moe_grouped_tiles<QT, 1, 8, 5, 2>(gate_up, down, experts, H, I, X, tokens, ids, weights, top_k, Y,
                                             accumulate, ws, L, stream, shared);
}

// ------------------------------------------------------------ MoE layer ----
//
// q3x_hip_moe_layer: the whole MoE layer of engine.cpp:406-430 (CUDA moe(),
// engine.cu:1709-1736): BF16 router matvec, top_k, routed experts, shared
// expert scaled by sigmoid(shared_scale . x) and added after the routed sum.

// logits[r] = router[r] . x for r < experts and *gate_logit = gate_row . x
// (engine.cpp:408, 427, the BF16 branch of mv :200-212): one wave per row,
// eight BF16 values per lane per step, fixed-order DPP sum.  Each wave first
// requests its row's first kRouterHeld steps; then the workgroup stages x in
// LDS once (In: PlainInput, or NormInput forming the RMSNorm exactly as the
// experts' matvec stages it -- same sum order, same products -- so router
// and experts see identical normalised values), and the row's dot reads x
// from there.  Rows and x 16-byte aligned, H % 32 == 0, x within
// router_gemv_lds_bytes.
constexpr int kRouterHeld = 8;
inline size_t router_gemv_lds_bytes(int H) { return pipe_x_bytes(H / kBlock) + 64; }

template <class In>
__global__ __launch_bounds__(256) void router_gemv_bf16_kernel(const uint16_t* __restrict__ router,
                                                               const uint16_t* __restrict__ gate_row, int experts,
                                                               int H, const float* __restrict__ x, In in,
                                                               float* __restrict__ logits,
                                                               float* __restrict__ gate_logit) {
    extern __shared__ __attribute__((aligned(16))) uint8_t router_lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int r = blockIdx.x * 4 + wave;  // rows past the gate row read zeros and store nothing
    const int bpr = H / kBlock;
    const uint16_t* row = r < experts ? router + static_cast<size_t>(r) * H : gate_row;
    // A buffer resource of the row's bytes: zeros past its end (and for rows
    // past the gate row), with no branch around the loads.
    const __amdgpu_buffer_rsrc_t rr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(row), 0, r <= experts ? 2 * H : 0, kBufferFlags);
    u32x4 held[kRouterHeld];
#pragma unroll
    for (int j = 0; j < kRouterHeld; ++j)
        held[j] = __builtin_amdgcn_raw_buffer_load_b128(rr, 2 * (8 * lane + 8 * kWave * j), 0, 0);
    in.stage(x, router_lds, bpr, reinterpret_cast<float*>(router_lds + pipe_x_bytes(bpr)));
    float acc = 0.0f;
    auto step = [&](int c, u32x4 w) {
        const uint8_t* xs = router_lds + x_block_offset(c >> 5) + 4 * (c & 31);
        const f32x4 x0 = *reinterpret_cast<const f32x4*>(xs);
        const f32x4 x1 = *reinterpret_cast<const f32x4*>(xs + 16);
        acc = fmaf(__uint_as_float(w.x << 16), x0.x, acc);
        acc = fmaf(__uint_as_float(w.x & 0xffff0000u), x0.y, acc);
        acc = fmaf(__uint_as_float(w.y << 16), x0.z, acc);
        acc = fmaf(__uint_as_float(w.y & 0xffff0000u), x0.w, acc);
        acc = fmaf(__uint_as_float(w.z << 16), x1.x, acc);
        acc = fmaf(__uint_as_float(w.z & 0xffff0000u), x1.y, acc);
        acc = fmaf(__uint_as_float(w.w << 16), x1.z, acc);
        acc = fmaf(__uint_as_float(w.w & 0xffff0000u), x1.w, acc);
    };
    // Columns in order, the held steps first (a lane's 8 columns lie inside
    // the row or past it together).
#pragma unroll
    for (int j = 0; j < kRouterHeld; ++j) {
        const int c = 8 * lane + 8 * kWave * j;
        if (c < H) step(c, held[j]);
    }
    for (int c = 8 * lane + 8 * kWave * kRouterHeld; c < H; c += 8 * kWave)
        step(c, __builtin_amdgcn_raw_buffer_load_b128(rr, 2 * c, 0, 0));
    const float total = group_sum<kWave>(acc);
    if (lane == 0 && r <= experts) {
        if (r < experts) logits[r] = total;
        else *gate_logit = total;
    }
}

// Dense GEMM policies over the tokens X[count, cols] (1-D grid, tiles of BM
// tokens); each adds its weight rows and its store.  Given a workspace
// (part), a launch may split K over workgroups (gemm_x3_fixup_kernel adds
// the units in K order and stores).
struct TokenTiles {
    static constexpr bool kLinearGrid = true;
    static constexpr bool kPairedColumns = false;
    static constexpr bool kPartialTiles = false;
    int tiles_x;
    const float* X;
    int cols;
    int count;
    int ksplit = 1;         // units per tile over K (set by the launch)
    float* part = nullptr;  // their partial sums
    __device__ bool tile(int ty, int bm, GemmTile& t) const {
        t.m0 = ty * bm;
        t.mcount = min(bm, count - t.m0);
        t.group = 0;
        return t.mcount > 0;
    }
    __device__ const float* a_row(const GemmTile& t, int m) const {
        return X + static_cast<size_t>(t.m0 + m) * cols;
    }
    __device__ void store_pair(const GemmTile&, int, int, float, float) const {}
};

// The router and the shared-expert gate of every token in one BF16 GEMM over
// experts + 1 rows: logits[t, e] for e < experts, gate_logit[t] for the last.
struct RouterGemm : TokenTiles {
    const uint8_t* router;
    const uint8_t* gate_row;
    size_t row_bytes;
    int experts;
    float* logits;
    float* gate_logit;
    __device__ const uint8_t* b_row(const GemmTile&, int n) const {
        return n < experts ? router + static_cast<size_t>(n) * row_bytes : gate_row;
    }
    __device__ void store(const GemmTile& t, int m, int n, float v) const {
        const int token = t.m0 + m;
        if (n < experts) logits[static_cast<size_t>(token) * experts + n] = v;
        else gate_logit[token] = v;
    }
};

// out[t * out_stride + col0 + n] = W[n] . x_t.
struct StridedGemm : TokenTiles {
    const uint8_t* w;
    size_t row_bytes;
    float* out;
    int out_stride;
    int col0;
    __device__ const uint8_t* b_row(const GemmTile&, int n) const { return w + static_cast<size_t>(n) * row_bytes; }
    __device__ void store(const GemmTile& t, int m, int n, float v) const {
        out[static_cast<size_t>(t.m0 + m) * out_stride + col0 + n] = v;
    }
};

// The shared expert's gate and up GEMMs with SwiGLU in the epilogue, paired
// as in GroupedGateUp: h[t, j] = silu(gate_j . x_t) * (up_j . x_t)
// (engine.cpp:422-425).  Launched over 2I rows; I % 64 == 0.
struct PairedGateUpGemm : TokenTiles {
    static constexpr bool kPairedColumns = true;
    const uint8_t* gate;
    const uint8_t* up;
    size_t row_bytes;
    int I;
    float* h;
    __device__ const uint8_t* b_row(const GemmTile&, int n) const {
        const int j = GroupedGateUp::out_col(n);
        return ((n & 16) ? up : gate) + static_cast<size_t>(j) * row_bytes;
    }
    __device__ void store(const GemmTile&, int, int, float) const {}
    __device__ void store_pair(const GemmTile& t, int m, int n, float g, float u) const {
        h[static_cast<size_t>(t.m0 + m) * I + GroupedGateUp::out_col(n)] = silu_ref(g) * u;
    }
};

// The shared expert's down GEMM added to the routed output (engine.cpp:
// 426-429): Y[t, n] = fma(sigmoid(gate_logit[t]), shared_down[n] . h_t, Y[t, n]).
struct SharedDownAdd : TokenTiles {
    const uint8_t* w;
    size_t row_bytes;
    float* Y;
    int H;
    const float* gate_logit;
    __device__ const uint8_t* b_row(const GemmTile&, int n) const { return w + static_cast<size_t>(n) * row_bytes; }
    __device__ void store(const GemmTile& t, int m, int n, float v) const {
        const int token = t.m0 + m;
        float* p = Y + static_cast<size_t>(token) * H + n;
        *p = fmaf(sigmoid_ref(gate_logit[token]), v, *p);
    }
};

// part / part_bytes: the K split's workspace (none: no split).  Calls that
// share it must be ordered, as calls on one stream are.
template <uint32_t QT, class P>
int launch_token_gemm(P pol, int rows, hipStream_t stream, float* part = nullptr, size_t part_bytes = 0) {
    pol.part = part;
    return launch_x3<QT>(pol, rows, pol.count, pol.cols, stream, part ? part_bytes : 0);
}

// Workspace bytes of the K split launch_x3 plans for a token GEMM.
inline size_t token_gemm_part_bytes(int rows, int count, int cols, bool paired) {
    return x3_plan(rows, count, cols, paired, static_cast<size_t>(-1)).workspace_bytes();
}

inline int launch_router_topk(const float* logits, int tokens, int experts, int top_k, int* ids, float* weights,
                              hipStream_t stream, int* ext_ids = nullptr, float* ext_weights = nullptr,
                              const float* shared_logit = nullptr) {
    const dim3 grid((tokens + 3) / 4), block(256);
    auto kernel = experts <= 4 * kWave ? router_topk_kernel<4> : experts <= 8 * kWave ? router_topk_kernel<8>
                                                                                      : router_topk_kernel<16>;
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, logits, tokens, experts, top_k, ids, weights, ext_ids,
                       ext_weights, shared_logit);
    return launch_status();
}

struct MoeLayerLayout {
    size_t logits, gate, ids, weights, gu_s, h_s, part, part_bytes, pair_ids, pair_weights, routed, total;
    bool fold;  // the prefill groups the shared expert with the routed ones
    MoeLayout R;
};

inline MoeLayerLayout moe_layer_layout(int tokens, int experts, int top_k, int H, int I, int shared_I) {
    MoeLayerLayout L{};
    const size_t T = static_cast<size_t>(tokens);
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t at = off; off = align_up(off + bytes, 256); return at; };
    L.logits = take(sizeof(float) * T * experts);
    L.gate = take(sizeof(float) * T);
    L.ids = take(sizeof(int) * T * top_k);
    L.weights = take(sizeof(float) * T * top_k);
    L.gu_s = take(sizeof(float) * T * 2 * shared_I);
    L.h_s = take(sizeof(float) * T * shared_I);
    // The K split of the prefill's token GEMMs (router, shared expert), one
    // at a time on the layer's stream.
    L.part_bytes = 0;
    if (tokens > 1) {
        L.part_bytes = std::max({token_gemm_part_bytes(experts + 1, tokens, H, false),
                                 token_gemm_part_bytes(2 * shared_I, tokens, H, shared_I % 64 == 0),
                                 token_gemm_part_bytes(shared_I, tokens, H, false),
                                 token_gemm_part_bytes(H, tokens, shared_I, false)});
    }
    L.part = take(L.part_bytes);
    // Where the shared expert has the routed experts' shape, the prefill
    // runs it as group `experts` of the grouped GEMMs: every token's pair
    // top_k, weighted by the sigmoid of its gate logit (pair_ids /
    // pair_weights [tokens, top_k + 1]).
    const long long pairs1 = static_cast<long long>(tokens) * (top_k + 1);
    L.fold = tokens > 1 && shared_I == I && I % 64 == 0 && experts + 1 <= kRouterMaxExperts &&
             pairs1 / kGrpBM + std::min<long long>(experts + 1, pairs1) + 1 <= 65535;
    L.pair_ids = take(L.fold ? sizeof(int) * pairs1 : 0);
    L.pair_weights = take(L.fold ? sizeof(float) * pairs1 : 0);
    L.R = L.fold ? moe_layout(tokens, experts + 1, top_k + 1, H, I) : moe_layout(tokens, experts, top_k, H, I);
    L.routed = take(L.R.total);
    L.total = off;
    return L;
}

// accumulate (one token only): Y += the layer output, or Q3X_HIP_ENOTSUP
// before Y is touched where the decode path does not take the shape.
template <uint32_t QT>
int moe_layer_run(const q3x_hip_moe_layer_weights& w, const float* X, int tokens, float* Y, int* ids,
                  float* weights, uint8_t* ws, const MoeLayerLayout& L, hipStream_t stream,
                  bool accumulate = false, const uint16_t* norm_w = nullptr) {
    constexpr int BB = QT == Q3X_HIP_MATRIX_Q8_0 ? kQ8Bytes : kQ4Bytes;
    const int E = w.experts, H = w.H, I = w.I, SI = w.shared_I, K = w.top_k;
    float* logits = reinterpret_cast<float*>(ws + L.logits);
    float* gate = reinterpret_cast<float*>(ws + L.gate);
    int* sel = ids ? ids : reinterpret_cast<int*>(ws + L.ids);
    float* wts = weights ? weights : reinterpret_cast<float*>(ws + L.weights);
    uint8_t* rws = ws + L.routed;
    float* part = L.part_bytes ? reinterpret_cast<float*>(ws + L.part) : nullptr;
    const auto* router = static_cast<const uint8_t*>(w.router);
    const auto* gate_row = static_cast<const uint8_t*>(w.shared_scale);
    const auto* gate_up = static_cast<const uint8_t*>(w.gate_up);
    const auto* down = static_cast<const uint8_t*>(w.down);
    const auto* sg = static_cast<const uint8_t*>(w.shared_gate);
    const auto* su = static_cast<const uint8_t*>(w.shared_up);
    const auto* sd = static_cast<const uint8_t*>(w.shared_down);
    int status;

    // Router logits and the shared expert's gate logit.
    if (tokens == 1 && router_gemv_lds_bytes(H) <= 64 * 1024) {
        const auto* rows = reinterpret_cast<const uint16_t*>(router);
        const auto* grow = reinterpret_cast<const uint16_t*>(gate_row);
        const dim3 grid((E + 1 + 3) / 4);
        if (norm_w)
            hipLaunchKernelGGL(router_gemv_bf16_kernel<NormInput>, grid, dim3(256), router_gemv_lds_bytes(H), stream,
                               rows, grow, E, H, X, NormInput{norm_w}, logits, gate);
        else
            hipLaunchKernelGGL(router_gemv_bf16_kernel<PlainInput>, grid, dim3(256), router_gemv_lds_bytes(H),
                               stream, rows, grow, E, H, X, PlainInput{}, logits, gate);
        status = launch_status();
    } else if (norm_w) {
        return Q3X_HIP_ENOTSUP;  // the caller normalises x and calls again without norm_w
    } else {
        RouterGemm g{};
        g.X = X; g.cols = H; g.count = tokens;
        g.router = router; g.gate_row = gate_row; g.row_bytes = static_cast<size_t>(H) * 2; g.experts = E;
        g.logits = logits; g.gate_logit = gate;
        status = launch_token_gemm<Q3X_HIP_MATRIX_BF16>(g, E + 1, stream, part, L.part_bytes);
    }
    if (status != Q3X_HIP_OK) return status;

    // Decode: routing, routed and shared experts in two launches (the gate_up
    // launch routes the token from the logits).
    if (tokens == 1) {
        const SharedExpert shared{sg, su, sd, SI, gate};
        status = moe_decode<QT>(gate_up, down, E, H, I, X, sel, wts, K, Y, accumulate ? 1 : 0, rws, L.R, shared,
                                stream, norm_w, logits, sel, wts);
        if (status != Q3X_HIP_ENOTSUP || accumulate) return status;
    }
    if (L.fold) {
        // Prefill: the shared expert as group E of the grouped GEMMs, its
        // pair last in every token's combine: Y = fma(sigmoid(gate logit),
        // shared, routed sum) (engine.cpp:426-429), as the separate shared
        // GEMMs below add it.
        int* pair_ids = reinterpret_cast<int*>(ws + L.pair_ids);
        float* pair_wts = reinterpret_cast<float*>(ws + L.pair_weights);
        if ((status = launch_router_topk(logits, tokens, E, K, sel, wts, stream, pair_ids, pair_wts, gate)) !=
            Q3X_HIP_OK)
            return status;
        GroupedShared shared;
        shared.group = E;
        shared.gate = sg;
        shared.up = su;
        shared.down = sd;
        return moe_grouped<QT>(gate_up, down, E + 1, H, I, X, tokens, pair_ids, pair_wts, K + 1, Y, 0, rws, L.R,
                               stream, shared);
    }
    if ((status = launch_router_topk(logits, tokens, E, K, sel, wts, stream)) != Q3X_HIP_OK) return status;
    // Prefill (or an unaligned decode): the grouped routed experts write Y,
    // then the shared expert's GEMMs add to it.
    status = moe_grouped<QT>(gate_up, down, E, H, I, X, tokens, sel, wts, K, Y, 0, rws, L.R, stream);
    if (status != Q3X_HIP_OK) return status;
    const size_t gu_row = static_cast<size_t>(H / kBlock) * BB;
    const size_t sd_row = static_cast<size_t>(SI / kBlock) * BB;
    float* h_s = reinterpret_cast<float*>(ws + L.h_s);
    if (SI % 64 == 0) {
        PairedGateUpGemm g{};
        g.X = X; g.cols = H; g.count = tokens;
        g.gate = sg; g.up = su; g.row_bytes = gu_row; g.I = SI; g.h = h_s;
        status = launch_token_gemm<QT>(g, 2 * SI, stream, part, L.part_bytes);
        if (status != Q3X_HIP_OK) return status;
    } else {
        float* gu_s = reinterpret_cast<float*>(ws + L.gu_s);
        StridedGemm g{};
        g.X = X; g.cols = H; g.count = tokens;
        g.row_bytes = gu_row; g.out = gu_s; g.out_stride = 2 * SI;
        g.w = sg; g.col0 = 0;
        if ((status = launch_token_gemm<QT>(g, SI, stream, part, L.part_bytes)) != Q3X_HIP_OK) return status;
        g.w = su; g.col0 = SI;
        if ((status = launch_token_gemm<QT>(g, SI, stream, part, L.part_bytes)) != Q3X_HIP_OK) return status;
        const size_t n = static_cast<size_t>(tokens) * SI;
        hipLaunchKernelGGL(swiglu_kernel, dim3(static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 65536))),
                           dim3(256), 0, stream, gu_s, h_s, SI, tokens, nullptr);
        if ((status = launch_status()) != Q3X_HIP_OK) return status;
    }
    SharedDownAdd g{};
    g.X = h_s; g.cols = SI; g.count = tokens;
    g.w = sd; g.row_bytes = sd_row; g.Y = Y; g.H = H; g.gate_logit = gate;
    return launch_token_gemm<QT>(g, H, stream, part, L.part_bytes);
}

}  // namespace q3x

using namespace q3x;

extern "C" int q3x_hip_router_topk(const float* logits, int tokens, int experts, int top_k, int* ids,
                                   float* weights, hipStream_t stream) {
    if (!logits || !ids || !weights || tokens <= 0 || experts <= 0 || experts > kRouterMaxExperts ||
        top_k <= 0 || top_k > experts || top_k > kRouterMaxTopK)
        return Q3X_HIP_EINVAL;
    return launch_router_topk(logits, tokens, experts, top_k, ids, weights, stream);
}

static bool moe_shape_ok(uint32_t type, int experts, int H, int I, int tokens, int top_k) {
    size_t bytes;
    if (experts <= 0 || experts > kRouterMaxExperts || tokens <= 0 || top_k <= 0 || top_k > experts)
        return false;
    if (!quantized_size(type, 2 * I, H, &bytes) || !quantized_size(type, H, I, &bytes)) return false;
    // Pool sizes and pair counts must fit the kernels' index types.
    const long long pairs = static_cast<long long>(tokens) * top_k;
    if (pairs > 0x7fffffffLL) return false;
    // Grouped tiles index grid.y (<= 65535).
    if (tokens > 1 && pairs / kGrpBM + std::min<long long>(experts, pairs) + 1 > 65535) return false;
    return true;
}

extern "C" size_t q3x_hip_moe_workspace_bytes(int tokens, int experts, int top_k, int H, int I) {
    if (tokens <= 0 || experts <= 0 || top_k <= 0 || H <= 0 || I <= 0) return 0;
    return moe_layout(tokens, experts, top_k, H, I).total;
}

extern "C" int q3x_hip_moe_routed(const void* gate_up, const void* down, uint32_t type, int experts, int H,
                                  int I, const float* X, int tokens, const int* ids, const float* weights,
                                  int top_k, float* Y, int accumulate, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
    if (type == Q3X_HIP_MATRIX_BF16) return Q3X_HIP_ENOTSUP;
    if (!gate_up || !down || !X || !ids || !weights || !Y || !workspace || !is_quant_type(type) ||
        !moe_shape_ok(type, experts, H, I, tokens, top_k))
        return Q3X_HIP_EINVAL;
    const MoeLayout L = moe_layout(tokens, experts, top_k, H, I);
    if (workspace_bytes < L.total || !aligned(workspace, 256)) return Q3X_HIP_EINVAL;
    if (!aligned(gate_up, 2) || !aligned(down, 2) || !aligned(X, 16)) return Q3X_HIP_EINVAL;
    const uint8_t* gu = static_cast<const uint8_t*>(gate_up);
    const uint8_t* dn = static_cast<const uint8_t*>(down);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    if (tokens == 1) {
        const int status = type == Q3X_HIP_MATRIX_Q8_0
                               ? moe_decode<Q3X_HIP_MATRIX_Q8_0>(gu, dn, experts, H, I, X, ids, weights, top_k, Y,
                                                                 accumulate, ws, L, SharedExpert{}, stream)
                               : moe_decode<Q3X_HIP_MATRIX_Q4_0>(gu, dn, experts, H, I, X, ids, weights, top_k, Y,
                                                                 accumulate, ws, L, SharedExpert{}, stream);
        if (status != Q3X_HIP_ENOTSUP) return status;
    }
    return type == Q3X_HIP_MATRIX_Q8_0
               ? moe_grouped<Q3X_HIP_MATRIX_Q8_0>(gu, dn, experts, H, I, X, tokens, ids, weights, top_k, Y,
                                                  accumulate, ws, L, stream)
               : moe_grouped<Q3X_HIP_MATRIX_Q4_0>(gu, dn, experts, H, I, X, tokens, ids, weights, top_k, Y,
                                                  accumulate, ws, L, stream);
}

extern "C" int q3x_hip_moe_routed_logits(const void* gate_up, const void* down, uint32_t type, int experts, int H,
                                         int I, const float* X, int tokens, const float* logits, int top_k,
                                         int* ids, float* weights, float* Y, int accumulate, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream) {
    if (type == Q3X_HIP_MATRIX_BF16) return Q3X_HIP_ENOTSUP;
    if (!gate_up || !down || !X || !logits || !ids || !weights || !Y || !workspace || !is_quant_type(type) ||
        !moe_shape_ok(type, experts, H, I, tokens, top_k) || top_k > kRouterMaxTopK)
        return Q3X_HIP_EINVAL;
    const MoeLayout L = moe_layout(tokens, experts, top_k, H, I);
    if (workspace_bytes < L.total || !aligned(workspace, 256)) return Q3X_HIP_EINVAL;
    if (!aligned(gate_up, 2) || !aligned(down, 2) || !aligned(X, 16)) return Q3X_HIP_EINVAL;
    const uint8_t* gu = static_cast<const uint8_t*>(gate_up);
    const uint8_t* dn = static_cast<const uint8_t*>(down);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    if (tokens == 1) {
        const int status = type == Q3X_HIP_MATRIX_Q8_0
                               ? moe_decode<Q3X_HIP_MATRIX_Q8_0>(gu, dn, experts, H, I, X, ids, weights, top_k, Y,
                                                                 accumulate, ws, L, SharedExpert{}, stream, nullptr,
                                                                 logits, ids, weights)
                               : moe_decode<Q3X_HIP_MATRIX_Q4_0>(gu, dn, experts, H, I, X, ids, weights, top_k, Y,
                                                                 accumulate, ws, L, SharedExpert{}, stream, nullptr,
                                                                 logits, ids, weights);
        if (status != Q3X_HIP_ENOTSUP) return status;
    }
    const int status = launch_router_topk(logits, tokens, experts, top_k, ids, weights, stream);
    if (status != Q3X_HIP_OK) return status;
    return type == Q3X_HIP_MATRIX_Q8_0
               ? moe_grouped<Q3X_HIP_MATRIX_Q8_0>(gu, dn, experts, H, I, X, tokens, ids, weights, top_k, Y,
                                                  accumulate, ws, L, stream)
               : moe_grouped<Q3X_HIP_MATRIX_Q4_0>(gu, dn, experts, H, I, X, tokens, ids, weights, top_k, Y,
                                                  accumulate, ws, L, stream);
}

static bool moe_layer_ok(const q3x_hip_moe_layer_weights* w, int tokens) {
    if (!w || !w->router || !w->gate_up || !w->down || !w->shared_gate || !w->shared_up || !w->shared_down ||
        !w->shared_scale || !is_quant_type(w->type))
        return false;
    if (w->shared_I <= 0 || w->shared_I > w->I || w->shared_I % kBlock != 0 || w->top_k > kRouterMaxTopK)
        return false;
    size_t bytes;
    if (!quantized_size(w->type, w->shared_I, w->H, &bytes) || !quantized_size(w->type, w->H, w->shared_I, &bytes))
        return false;
    return moe_shape_ok(w->type, w->experts, w->H, w->I, tokens, w->top_k);
}

extern "C" size_t q3x_hip_moe_layer_workspace_bytes(const q3x_hip_moe_layer_weights* layer, int tokens) {
    if (!layer || tokens <= 0 || layer->experts <= 0 || layer->top_k <= 0 || layer->H <= 0 || layer->I <= 0 ||
        layer->shared_I <= 0)
        return 0;
    return moe_layer_layout(tokens, layer->experts, layer->top_k, layer->H, layer->I, layer->shared_I).total;
}

static int moe_layer_checked(const q3x_hip_moe_layer_weights* layer, const float* X, int tokens, float* Y,
                             int* ids, float* weights, void* workspace, size_t workspace_bytes,
                             hipStream_t stream, bool accumulate, const uint16_t* norm_w = nullptr) {
    if (layer && layer->type == Q3X_HIP_MATRIX_BF16) return Q3X_HIP_ENOTSUP;
    if (!X || !Y || !workspace || !moe_layer_ok(layer, tokens)) return Q3X_HIP_EINVAL;
    const q3x_hip_moe_layer_weights& w = *layer;
    const MoeLayerLayout L = moe_layer_layout(tokens, w.experts, w.top_k, w.H, w.I, w.shared_I);
    if (workspace_bytes < L.total || !aligned(workspace, 256)) return Q3X_HIP_EINVAL;
    if (!aligned(w.router, 16) || !aligned(w.shared_scale, 16) || !aligned(X, 16)) return Q3X_HIP_EINVAL;
    if (!aligned(w.gate_up, 2) || !aligned(w.down, 2) || !aligned(w.shared_gate, 2) || !aligned(w.shared_up, 2) ||
        !aligned(w.shared_down, 2))
        return Q3X_HIP_EINVAL;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    return w.type == Q3X_HIP_MATRIX_Q8_0
               ? moe_layer_run<Q3X_HIP_MATRIX_Q8_0>(w, X, tokens, Y, ids, weights, ws, L, stream, accumulate, norm_w)
               : moe_layer_run<Q3X_HIP_MATRIX_Q4_0>(w, X, tokens, Y, ids, weights, ws, L, stream, accumulate, norm_w);
}

extern "C" int q3x_hip_moe_layer(const q3x_hip_moe_layer_weights* layer, const float* X, int tokens, float* Y,
                                 int* ids, float* weights, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
    return moe_layer_checked(layer, X, tokens, Y, ids, weights, workspace, workspace_bytes, stream, false);
}

int q3x::gate_up_swiglu(const void* gate, const void* up, uint32_t type, int I, int H, const float* X, int count,
                        float* h, hipStream_t stream) {
    size_t bytes;
    if (!is_quant_type(type) || count <= 0 || I % 64 != 0 || !quantized_size(type, I, H, &bytes))
        return Q3X_HIP_ENOTSUP;
    if (!aligned(gate, 2) || !aligned(up, 2) || !aligned(X, 16) || !aligned(h, 4)) return Q3X_HIP_ENOTSUP;
    PairedGateUpGemm g{};
    g.X = X; g.cols = H; g.count = count;
    g.gate = static_cast<const uint8_t*>(gate); g.up = static_cast<const uint8_t*>(up);
    g.row_bytes = static_cast<size_t>(H / kBlock) * block_bytes(type); g.I = I; g.h = h;
    return type == Q3X_HIP_MATRIX_Q8_0 ? launch_token_gemm<Q3X_HIP_MATRIX_Q8_0>(g, 2 * I, stream)
                                       : launch_token_gemm<Q3X_HIP_MATRIX_Q4_0>(g, 2 * I, stream);
}

int q3x::moe_layer_decode_add(const q3x_hip_moe_layer_weights& layer, const float* X, const uint16_t* norm_w,
                              float* Y, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    // NormInput loads the norm weights four at a time (8 bytes).
    if (norm_w && !aligned(norm_w, 8)) return Q3X_HIP_ENOTSUP;
    return moe_layer_checked(&layer, X, 1, Y, nullptr, nullptr, workspace, workspace_bytes, stream, true, norm_w);
}

