// The whole decode step of a Qwen2 model as one persistent, cooperative
// launch on gfx950: embedding, every layer (RMSNorm, fused QKV GEMV with bias
// + RoPE + paged KV append, GQA attention, O GEMV + residual, RMSNorm,
// gate/up GEMV + SiLU, down GEMV + residual), the final norm, the LM head and
// the greedy argmax.
//
// Reference: one QwenCudaModel::Decode / DecodeBatch / GreedyRun step
// (backends/cuda/qwen_cuda_model.cu:2641-2776, 2778-3102), whose CPU
// counterpart is QwenModel::Forward (model/architectures/qwen/
// qwen_model.cpp:216-331). The CUDA backend launches ~10 kernels per layer;
// on MI355X each kernel boundary costs a launch, a ramp-up/drain of 256 CUs
// and an L2 write-back across 8 XCDs, which at batch 1 costs more than the
// weights take to stream. Here one workgroup per CU stays resident for the
// whole step and phases hand over through device-scope counters.
//
// Phases and hand-over
//   * GEMV phases use a stream-K split: the (row tile, K chunk) space of the
//     matrix is cut into one contiguous range per workgroup, and each
//     workgroup's range into one contiguous range per wave, so every CU
//     streams the same number of bytes whatever the matrix shape. A tile
//     finished inside one workgroup goes straight to its epilogue; a tile
//     shared by several workgroups is finished by the last of them to arrive
//     (per-tile counter), which adds the partials in workgroup order.
//   * The activation vector of a GEMV phase sits in LDS (only the K chunks
//     the workgroup's range touches), written by the phase prologue: an
//     RMSNorm every workgroup computes for itself from the fp32 residual
//     stream, or a copy of the fp16 attention / MLP activations.
//   * Attention units are (row, kv head, context split); the last split to
//     finish merges the partials in split order.
//   * Between phases a grid barrier: each workgroup adds one to one of 64
//     counters (one per 64-byte line) and polls all of them. Counters only
//     grow; the host passes the barrier count of earlier launches, so targets
//     need no reset.
//   * Data that crosses workgroups (residual stream, q, K/V appends,
//     activations, partials) is written and read with device-scope (sc1)
//     accesses, coherent across the XCDs' L2s; a wave waits for its stores
//     (s_waitcnt 0) before any arrival is counted.
//   * Every wait is bounded: after ~2 s a workgroup records an error in the
//     workspace and the whole grid exits; later launches exit at once until
//     the host resets the workspace.
// All reductions run in a fixed order, so results do not depend on timing,
// and a row's arithmetic does not depend on the other rows of the batch.
#include <algorithm>
#include <type_traits>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "common.h"

namespace lyk {
namespace {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kPieces = 4;       // row tiles one wave's range may touch
constexpr int kBarLines = 64;    // barrier counters
constexpr int kLineWords = 16;   // 64 bytes
constexpr int kNormPer = 16;     // hidden_size <= kNormPer * kThreads
constexpr int kMaxRows = 4;
constexpr int kAttnMaxSplits = 32;   // context splits per (row, kv head)
constexpr int kAttnSplitTokens = 512;
constexpr int kHandoverChunks = 13;  // ~4 us of per-CU streaming
constexpr uint64_t kSpinTicks = 200000000ull;  // s_memrealtime is 100 MHz: 2 s

enum Phase { kQkv = 0, kOut = 1, kGateUp = 2, kDown = 3, kHead = 4 };

struct StepArgs {
    lyk_step_model md;
    lyk_step_io io;
    int* err;
    uint32_t* epoch;      // barriers completed by earlier launches
    unsigned* bar;
    unsigned* tile_cnt;   // per row tile of the current GEMV phase
    float* part;          // [grid][2][M][64] GEMV partials
    float* attn_ml;       // [rows*nkv][splits][G][2] per-split max and sum
    float* attn_acc;      // [rows*nkv][splits][G][hd] per-split unnormalised output
    float* h;             // [2][kMaxRows][hidden] residual entering a layer (by parity)
    float* d_attn;        // [M][hidden] attention block output (O GEMV)
    float* d_mlp;         // [M][hidden] MLP block output (down GEMV)
    float* q;             // [M][nq*hd] rotated queries
    uint16_t* act;        // [M][ld_act] fp16 SiLU(gate) * up
    float* best_v;        // [M][head tiles] greedy candidates
    int* best_i;
    int* best_bad;
    int ld_act;
    int attn_split_tokens;  // context tokens per attention split, about
    int attn_max_splits;    // splits per (row, kv head), at most
    uint32_t barriers;      // grid barriers of one launch
};

// ------------------------------------------------------------ primitives

__device__ __forceinline__ void store_sc1_u16(uint16_t* p, uint16_t v) { store_sc1<uint16_t>(p, v); }
__device__ __forceinline__ uint32_t load_sc1_u32(const uint32_t* p) { return load_sc1<uint32_t>(p); }
__device__ __forceinline__ int load_sc1_i32(const int* p) { return load_sc1<int>(p); }

// The layer table entry (device memory) as 13 pointer-sized loads.
__device__ __forceinline__ lyk_step_layer load_layer(const lyk_step_layer* p) {
    static_assert(sizeof(lyk_step_layer) == 13 * sizeof(uint64_t), "layer table entry layout");
    const LYK_GLOBAL uint64_t* q = (const LYK_GLOBAL uint64_t*)p;
    uint64_t w[13];
#pragma unroll
    for (int i = 0; i < 13; ++i) w[i] = q[i];
    return __builtin_bit_cast(lyk_step_layer, w);
}

// Profiling timestamp of workgroup 0 (lyk_step_io::trace): kind 0 = the
// phase's inputs are ready (x window / queries and K/V loaded), kind 1 = its
// main loop is done.
__device__ __forceinline__ void mark(const StepArgs& a, int phase, int kind) {
    if (a.io.trace && blockIdx.x == 0 && threadIdx.x == 0)
        st(a.io.trace + (2 + kind) * a.barriers + 2 + phase, (uint64_t)__builtin_amdgcn_s_memrealtime());
}

__device__ __forceinline__ bool aborted(const StepArgs& a) { return load_sc1_i32(a.err) != 0; }

// threadIdx.x through an opaque move: values derived from it are recomputed
// in every phase instead of being hoisted out of the layer loop and kept
// live (in registers) across all phases.
__device__ __forceinline__ int phase_tid() {
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
    return t;
}

// Grid barrier number `idx` of this launch, in two halves so that loads
// that do not depend on it can be issued in between. Arrival: every wave
// waits for its own stores (s_waitcnt 0), then one count from the
// workgroup. Wait: wave 0 polls all counters; false (for the whole
// workgroup) when the grid is aborting.
__device__ __forceinline__ void grid_arrive(const StepArgs& a, uint32_t idx) {
    publish_sc1_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int G = gridDim.x;
        const int lines = G < kBarLines ? G : kBarLines;
        if (a.io.trace && blockIdx.x == 0)
            st(a.io.trace + a.barriers + 2 + idx, (uint64_t)__builtin_amdgcn_s_memrealtime());
        __hip_atomic_fetch_add(gp(a.bar + (blockIdx.x % lines) * kLineWords), 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

__device__ __forceinline__ bool grid_wait(const StepArgs& a, uint32_t epoch, uint32_t idx) {
    __shared__ int ok;
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int G = gridDim.x;
        const int lines = G < kBarLines ? G : kBarLines;
        const uint32_t gen = epoch + idx + 1;
        const uint32_t per = lane < lines ? (uint32_t)((G - 1 - lane) / lines + 1) : 0u;
        const uint32_t target = gen * per;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        int good = 1;
        while (true) {
            bool done = true;
            if (lane < lines) {
                const uint32_t v = load_sc1_u32(a.bar + lane * kLineWords);
                done = (int32_t)(v - target) >= 0;
            }
            if (__all(done)) break;
            if (aborted(a)) { good = 0; break; }
            if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
                if (lane == 0) store_sc1(a.err, 1);
                good = 0;
                break;
            }
        }
        if (lane == 0) {
            ok = good;
            if (a.io.trace && blockIdx.x == 0) st(a.io.trace + idx + 1, (uint64_t)__builtin_amdgcn_s_memrealtime());
        }
    }
    __syncthreads();
    return ok != 0;
}

__device__ __forceinline__ bool grid_sync(const StepArgs& a, uint32_t epoch, uint32_t idx) {
    grid_arrive(a, idx);
    return grid_wait(a, epoch, idx);
}

// Sum of v over the workgroup for M rows; every thread gets the sums. Waves
// are added in wave order.
template <int M>
__device__ __forceinline__ void block_sum_rows(float (&v)[M], int tid) {
    __shared__ float part[kWaves][kMaxRows];
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float s = wave_sum(v[m]);
        if (lane == 0) part[wave][m] = s;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += part[w][m];
        v[m] = s;
    }
    __syncthreads();
}

// ------------------------------------------------------------ GEMV phase

struct Mat {
    const u32x4* w;
    const void* s;
    int n;        // output rows (paired: rows of each matrix)
    int k;
    int tiles;
    int chunks;   // K chunks of 8 groups (int4: 256 k) or 8 blocks (int8: 128 k)
};

template <bool Q8>
__device__ __forceinline__ Mat make_mat(const void* w, const void* s, int n, int k, bool paired) {
    Mat m;
    m.w = static_cast<const u32x4*>(w);
    m.s = s;
    m.n = n;
    m.k = k;
    m.tiles = paired ? (n + 31) / 32 : (n + 63) / 64;
    const int unit = Q8 ? 16 : 32;
    m.chunks = ((k + unit - 1) / unit + 7) / 8;
    return m;
}

// The workgroup's share of a phase: chunk range [f0, f1) of the flattened
// (tile, chunk) space and the window of K chunks it reads, as LDS slots
// slot(c) = (c - ca) mod chunks < win.
struct Part {
    int64_t U, f0, f1;
    int gp;   // workgroups with work
    int ca, win;
    bool busy;
};

// Whole row tiles per workgroup (no cross-workgroup sums) unless splitting
// tiles along K saves more chunk-streaming time than the partial-sum hand
// over costs (about kHandoverChunks chunks of streaming at the per-CU share
// of HBM bandwidth).
__host__ __device__ __forceinline__ bool tile_aligned(int64_t tiles, int64_t chunks, int G) {
    const int64_t U = tiles * chunks;
    return (tiles + G - 1) / G * chunks <= (U + G - 1) / G + kHandoverChunks;
}

__device__ __forceinline__ Part partition(const Mat& A) {
    Part p;
    p.U = (int64_t)A.tiles * A.chunks;
    const int G = gridDim.x;
    const int b = blockIdx.x;
    if (tile_aligned(A.tiles, A.chunks, G)) {
        p.gp = A.tiles < G ? A.tiles : G;
        p.busy = b < p.gp;
        p.f0 = p.busy ? (int64_t)A.tiles * b / p.gp * A.chunks : 0;
        p.f1 = p.busy ? (int64_t)A.tiles * (b + 1) / p.gp * A.chunks : 0;
    } else {
        p.gp = (int)(p.U < G ? p.U : G);
        p.busy = b < p.gp;
        p.f0 = p.busy ? p.U * b / p.gp : 0;
        p.f1 = p.busy ? p.U * (b + 1) / p.gp : 0;
    }
    const int64_t len = p.f1 - p.f0;
    if (len >= A.chunks) {
        p.ca = 0;
        p.win = A.chunks;
    } else {
        p.ca = (int)(p.f0 % A.chunks);
        p.win = (int)len;
    }
    return p;
}

// Workgroup holding flattened chunk f (every workgroup < gp has work).
__device__ __forceinline__ int wg_of(int64_t f, const Part& p) {
    return (int)(((f + 1) * p.gp + p.U - 1) / p.U - 1);
}

template <bool Q8>
constexpr int chunk_k() { return Q8 ? 128 : 256; }

// Residual stream of row m entering a norm: base (+ d1) (+ d2), added in
// that order (the reference's h += attn; h += mlp). Every workgroup computes
// the whole row for its RMSNorm; it also stores its own slice [H*b/G,
// H*(b+1)/G) to `out` when given (the next layer's base).
struct ResidualSrc {
    const float* base;   // fp32 rows [M][H] (or embedding rows when embed)
    const float* d1;
    const float* d2;
    float* out;
    bool embed;          // base rows are embed[tokens[m]] (read-only, plain loads)
};

// x window <- RMSNorm(residual) (fp16), for the chunks of the window; zero
// beyond k. Runs on every workgroup (idle ones only write their slice).
template <int M, bool Q8>
__device__ __forceinline__ void fill_norm(const StepArgs& a, const float* gamma, const ResidualSrc& r,
                                          const Mat& A, const Part& p, uint16_t* xs, int tid) {
    constexpr int CK = chunk_k<Q8>();
    const int H = a.md.hidden_size;
    const float* base[M];
#pragma unroll
    for (int m = 0; m < M; ++m)
        base[m] = r.embed ? a.md.embed + (size_t)load_sc1(a.io.tokens + m) * H : r.base + (size_t)m * H;
    float v[M][kNormPer];
#pragma unroll
    for (int j = 0; j < kNormPer; ++j) {
        const int i = tid + j * kThreads;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            float x = 0.0f;
            if (i < H) {
                x = r.embed ? ld(base[m] + i) : load_sc1(base[m] + i);
                if (r.d1) x += load_sc1(r.d1 + (size_t)m * H + i);
                if (r.d2) x += load_sc1(r.d2 + (size_t)m * H + i);
            }
            v[m][j] = x;
        }
    }
    if (r.out) {
        const int b = blockIdx.x, G = gridDim.x;
        const int i0 = (int)((int64_t)H * b / G), i1 = (int)((int64_t)H * (b + 1) / G);
#pragma unroll
        for (int j = 0; j < kNormPer; ++j) {
            const int i = tid + j * kThreads;
            if (i >= i0 && i < i1)
#pragma unroll
                for (int m = 0; m < M; ++m) store_sc1(r.out + (size_t)m * H + i, v[m][j]);
        }
    }
    if (!p.busy) return;
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < kNormPer; ++j) s = fmaf(v[m][j], v[m][j], s);
        ss[m] = s;
    }
    block_sum_rows<M>(ss, tid);
    float scale[M];
#pragma unroll
    for (int m = 0; m < M; ++m) scale[m] = 1.0f / sqrtf(ss[m] / (float)H + a.md.rms_norm_eps);
#pragma unroll
    for (int j = 0; j < kNormPer; ++j) {
        const int i = tid + j * kThreads;
        if (i < H) {
            const int c = i / CK;
            const int slot = (c - p.ca + A.chunks) % A.chunks;
            if (slot < p.win) {
                const float g = ld(gamma + i);
#pragma unroll
                for (int m = 0; m < M; ++m)
                    xs[((size_t)m * p.win + slot) * CK + (i % CK)] = f2h(v[m][j] * scale[m] * g);
            }
        }
    }
    // zero the window past k
    const int kp = A.chunks * CK;
    for (int i = H + tid; i < kp; i += kThreads) {
        const int c = i / CK;
        const int slot = (c - p.ca + A.chunks) % A.chunks;
        if (slot < p.win)
#pragma unroll
            for (int m = 0; m < M; ++m) xs[((size_t)m * p.win + slot) * CK + (i % CK)] = 0;
    }
}

// x window <- fp16 rows src[m*ld ...] (zero-padded to chunks*CK by the
// caller's buffer layout).
template <int M, bool Q8>
__device__ __forceinline__ void fill_copy(const uint16_t* src, int ld, const Mat& A, const Part& p,
                                          uint16_t* xs, int tid) {
    constexpr int CK = chunk_k<Q8>();
    constexpr int W = CK / 2;  // dwords per chunk row
    if (!p.busy) return;
    const int total = M * p.win * W;
    uint32_t* dst = reinterpret_cast<uint32_t*>(xs);
    for (int e0 = tid; e0 < total; e0 += kThreads * 8) {
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = e0 + u * kThreads;
            v[u] = 0;
            if (e < total) {
                const int m = e / (p.win * W), r = e % (p.win * W);
                const int slot = r / W, w = r % W;
                const int c = (p.ca + slot) % A.chunks;
                v[u] = load_sc1_u32(reinterpret_cast<const uint32_t*>(src + (size_t)m * ld + (size_t)c * CK) + w);
            }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = e0 + u * kThreads;
            if (e < total) dst[e] = v[u];
        }
    }
}

// Context split of a row: splits of about split_tokens tokens, at most
// max_splits; a row's arithmetic depends only on its own context length.
__device__ __forceinline__ int attn_splits(int ctx, int split_tokens, int max_splits) {
    const int s = (ctx + split_tokens - 1) / split_tokens;
    return s < 1 ? 1 : (s > max_splits ? max_splits : s);
}

// x window <- the attention output: the fixed-order merge of the context
// splits' partials (max, sum, unnormalised output per head) written by the
// attention phase, out = sum_s e_s acc_s / sum_s e_s l_s with
// e_s = exp(m_s - max_s m_s).
template <int M, bool Q8>
__device__ __forceinline__ void fill_attn(const StepArgs& a, const Mat& A, const Part& p, uint16_t* xs,
                                          int tid) {
    constexpr int CK = chunk_k<Q8>();
    if (!p.busy) return;
    const int nq = a.md.num_heads, nkv = a.md.num_kv_heads, hd = a.md.head_dim, G = nq / nkv;
    const int MS = a.attn_max_splits;
    // heads of the window: consecutive (mod nq) from the head of chunk ca
    const int h0 = p.ca * CK / hd;
    const int nh = min(nq, (p.win * CK + hd - 1) / hd + 1);
    // per (row, window head): e_s = exp(m_s - max) for each split, then L
    float* wts = reinterpret_cast<float*>(xs + (size_t)M * p.win * CK);  // [M][nh][MS + 1]
    for (int e = tid; e < M * nh; e += kThreads) {
        const int m = e / nh, hw = e % nh;
        const int hq = (h0 + hw) % nq;
        const int S = attn_splits(load_sc1(a.io.positions + m) + 1, a.attn_split_tokens, MS);
        const size_t grp = (size_t)m * nkv + hq / G;
        const int h = hq % G;
        float* w = wts + (size_t)e * (MS + 1);
        float mx = -INFINITY;
        for (int s = 0; s < S; ++s) mx = fmaxf(mx, load_sc1(&a.attn_ml[((grp * MS + s) * G + h) * 2]));
        float L = 0.0f;
        for (int s = 0; s < S; ++s) {
            const float* ml = &a.attn_ml[((grp * MS + s) * G + h) * 2];
            const float es = expf(load_sc1(ml) - mx);
            w[s] = es;
            L += load_sc1(ml + 1) * es;
        }
        w[MS] = L;
    }
    __syncthreads();
    const int kq = nq * hd;
    for (int e = tid; e < M * p.win * CK; e += kThreads) {
        const int m = e / (p.win * CK), r = e % (p.win * CK);
        const int slot = r / CK, i = r % CK;
        const int k = ((p.ca + slot) % A.chunks) * CK + i;
        float out = 0.0f;
        if (k < kq) {
            const int hq = k / hd, d = k % hd;
            const int hw = (hq - h0 + nq) % nq;
            const int S = attn_splits(load_sc1(a.io.positions + m) + 1, a.attn_split_tokens, MS);
            const size_t grp = (size_t)m * nkv + hq / G;
            const int h = hq % G;
            const float* w = wts + ((size_t)m * nh + hw) * (MS + 1);
            float o = 0.0f;
            for (int s = 0; s < S; ++s) o += load_sc1(&a.attn_acc[((grp * MS + s) * G + h) * (size_t)hd + d]) * w[s];
            out = o / w[MS];
        }
        xs[((size_t)m * p.win + slot) * CK + i] = f2h(out);
    }
}

// Accumulates chunk f of the matrix into acc (x from the LDS window).
template <int M, bool Q8>
struct ChunkMath;

template <int M>
struct ChunkMath<M, false> {
    static constexpr int CK = 256;
    __device__ __forceinline__ static void load(const Mat& A, int64_t f, int lane, u32x4 (&w)[8], u32x4& s4) {
        const LYK_GLOBAL u32x4* wt = gp(A.w + (size_t)f * 512 + lane);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            w[j] = __builtin_nontemporal_load(wt + j * 64);
            __builtin_amdgcn_sched_barrier(0);
        }
        s4 = __builtin_nontemporal_load(gp(static_cast<const u32x4*>(A.s) + (size_t)f * 64 + lane));
        __builtin_amdgcn_sched_barrier(0);
    }
    __device__ __forceinline__ static void compute(const u32x4 (&w)[8], const u32x4& s4, const uint16_t* xs,
                                                   int xstride, float (&acc)[M], uint32_t vmagic) {
        const half2_t off_a = {(half_t)-1032.0f, (half_t)-1032.0f};
        const half2_t off_b = {(half_t)-1152.0f, (half_t)-1152.0f};
        float gs[M][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t u4[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
            half2_t qa[8], qb[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t u = u4[d], t = u >> 8;
                qa[2 * d] = as_half2((u & 0x000F000Fu) | vmagic) + off_a;
                qb[2 * d] = as_half2((u & 0x00F000F0u) | vmagic) + off_b;
                qa[2 * d + 1] = as_half2((t & 0x000F000Fu) | vmagic) + off_a;
                qb[2 * d + 1] = as_half2((t & 0x00F000F0u) | vmagic) + off_b;
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const u32x4* xv = reinterpret_cast<const u32x4*>(xs + (size_t)m * xstride + j * 32);
                float a = 0.0f, b = 0.0f;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const u32x4 xx = xv[d];
                    a = dot2(qa[2 * d], as_half2(xx.x), a);
                    b = dot2(qb[2 * d], as_half2(xx.y), b);
                    a = dot2(qa[2 * d + 1], as_half2(xx.z), a);
                    b = dot2(qb[2 * d + 1], as_half2(xx.w), b);
                }
                gs[m][j] = b * 0.0625f + a;
            }
            __builtin_amdgcn_sched_barrier(0);  // x reads of one group at a time
        }
        const uint32_t sw[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float s = h2f(uint16_t(sw[j >> 1] >> (16 * (j & 1))));
#pragma unroll
            for (int m = 0; m < M; ++m) acc[m] = fmaf(gs[m][j], s, acc[m]);
        }
    }
};

template <int M>
struct ChunkMath<M, true> {
    static constexpr int CK = 128;
    __device__ __forceinline__ static void load(const Mat& A, int64_t f, int lane, u32x4 (&w)[8], u32x4& s4) {
        const LYK_GLOBAL u32x4* wt = gp(A.w + (size_t)f * 512 + lane);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            w[j] = __builtin_nontemporal_load(wt + j * 64);
            __builtin_amdgcn_sched_barrier(0);
        }
        (void)s4;
    }
    __device__ __forceinline__ static void compute(const u32x4 (&w)[8], const u32x4&, const uint16_t* xs,
                                                   int xstride, float (&acc)[M], uint32_t) {
        const half2_t off = {(half_t)-1152.0f, (half_t)-1152.0f};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t u4[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
            half2_t q[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                q[2 * d] = as_half2(__builtin_amdgcn_perm(0x64646464u, u4[d], 0x04010400u)) + off;
                q[2 * d + 1] = as_half2(__builtin_amdgcn_perm(0x64646464u, u4[d], 0x04030402u)) + off;
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const u32x4* xv = reinterpret_cast<const u32x4*>(xs + (size_t)m * xstride + j * 16);
                const u32x4 x0 = xv[0], x1 = xv[1];
                float a = acc[m];
                a = dot2(q[0], as_half2(x0.x), a);
                a = dot2(q[1], as_half2(x0.y), a);
                a = dot2(q[2], as_half2(x0.z), a);
                a = dot2(q[3], as_half2(x0.w), a);
                a = dot2(q[4], as_half2(x1.x), a);
                a = dot2(q[5], as_half2(x1.y), a);
                a = dot2(q[6], as_half2(x1.z), a);
                a = dot2(q[7], as_half2(x1.w), a);
                acc[m] = a;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// Runs the workgroup's share of one GEMV phase. The wave's first two chunks
// of weights are requested before the grid barrier that publishes the
// phase's inputs (weights never depend on them), so the barrier and the
// input fill overlap the first HBM round trip. `fill` writes the x window;
// `epi(tile, v, lane)` finishes a tile (v = the tile's 64 row sums of each
// batch row, one row per lane; called by one whole wave). bar < 0: no
// barrier before the phase. Returns false when the grid is aborting.
template <int M, bool Q8, class Fill, class Epi>
__device__ __forceinline__ bool gemv_phase(const StepArgs& a, uint32_t epoch, int bar, const Mat& A, Fill fill,
                                           Epi epi) {
    const int tid = phase_tid();
    using CM = ChunkMath<M, Q8>;
    constexpr int CK = CM::CK;
    extern __shared__ __align__(16) unsigned char smem[];
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* red = reinterpret_cast<float*>(smem);  // aliases xs after the stream
    const Part p = partition(A);
    const int b = blockIdx.x;
    const int lane = tid & 63, wave = uniform(tid >> 6);
    const int64_t len = p.f1 - p.f0;
    const int64_t w0 = p.f0 + len * wave / kWaves, w1 = p.f0 + len * (wave + 1) / kWaves;

    if (bar >= 0) grid_arrive(a, (uint32_t)bar);
    u32x4 wa[8], wb[8], sa, sb;
    if (w0 < w1) CM::load(A, w0, lane, wa, sa);
    if (w0 + 1 < w1) CM::load(A, w0 + 1, lane, wb, sb);
    if (bar >= 0 && !grid_wait(a, epoch, (uint32_t)bar)) return false;

    fill(A, p, xs, tid);
    if (!p.busy) return true;
    __syncthreads();
    mark(a, bar < 0 ? 0 : bar, 0);

    const int xstride = p.win * CK;
    float accq[kPieces][M];
#pragma unroll
    for (int q = 0; q < kPieces; ++q)
#pragma unroll
        for (int m = 0; m < M; ++m) accq[q][m] = 0.0f;

    uint32_t vmagic;
    asm("v_mov_b32 %0, %1" : "=v"(vmagic) : "s"(0x64006400u));

    if (w0 < w1) {
        int64_t f = w0;
        int c = (int)(f % A.chunks);
        int t = (int)(f / A.chunks);
        int q = 0;
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.0f;
        // int8 per-row scale of the current tile
        float srow = 1.0f;
        if constexpr (Q8) srow = h2f(ld(static_cast<const uint16_t*>(A.s) + (size_t)t * 64 + lane));
        // One chunk: math on the buffer, then request the chunk two ahead
        // into it; a tile's sums go to its piece slot when the tile ends.
        auto step = [&](u32x4 (&wc)[8], u32x4& sc) -> bool {
            const int slot = (c - p.ca + A.chunks) % A.chunks;
            CM::compute(wc, sc, xs + (size_t)slot * CK, xstride, acc, vmagic);
            const bool end = f + 1 == w1;
            if (c + 1 == A.chunks || end) {
#pragma unroll
                for (int qq = 0; qq < kPieces; ++qq)
                    if (qq == q)
#pragma unroll
                        for (int m = 0; m < M; ++m) accq[qq][m] = acc[m] * srow;
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m] = 0.0f;
                ++q;
                ++t;
                if constexpr (Q8)
                    if (!end) srow = h2f(ld(static_cast<const uint16_t*>(A.s) + (size_t)t * 64 + lane));
            }
            if (end) return true;
            if (f + 2 < w1) CM::load(A, f + 2, lane, wc, sc);
            __builtin_amdgcn_sched_barrier(0);
            ++f;
            c = c + 1 == A.chunks ? 0 : c + 1;
            return false;
        };
        while (true) {
            if (step(wa, sa)) break;
            if (step(wb, sb)) break;
        }
    }
    __syncthreads();  // every wave is done with the x window
    mark(a, bar < 0 ? 0 : bar, 1);
    {
        const int64_t tf = w0 < w1 ? w0 / A.chunks : 0;
        const int np = w0 < w1 ? (int)((w1 - 1) / A.chunks - tf + 1) : 0;
#pragma unroll
        for (int q = 0; q < kPieces; ++q)
            if (q < np)
#pragma unroll
                for (int m = 0; m < M; ++m) red[((wave * kPieces + q) * M + m) * 64 + lane] = accq[q][m];
    }
    __syncthreads();

    const int tA = (int)(p.f0 / A.chunks), tB = (int)((p.f1 - 1) / A.chunks);
    for (int t = tA + wave; t <= tB; t += kWaves) {
        float v[M];
#pragma unroll
        for (int m = 0; m < M; ++m) v[m] = 0.0f;
        for (int w = 0; w < kWaves; ++w) {
            const int64_t a0 = p.f0 + len * w / kWaves, a1 = p.f0 + len * (w + 1) / kWaves;
            if (a0 >= a1) continue;
            const int tf = (int)(a0 / A.chunks), tl = (int)((a1 - 1) / A.chunks);
            if (t < tf || t > tl) continue;
#pragma unroll
            for (int m = 0; m < M; ++m) v[m] += red[((w * kPieces + (t - tf)) * M + m) * 64 + lane];
        }
        const bool full = p.f0 <= (int64_t)t * A.chunks && (int64_t)(t + 1) * A.chunks <= p.f1;
        if (!full) {
            const int slot = t == tA ? 0 : 1;
#pragma unroll
            for (int m = 0; m < M; ++m)
                store_sc1(&a.part[(((size_t)b * 2 + slot) * M + m) * 64 + lane], v[m]);
            const int bf = wg_of((int64_t)t * A.chunks, p);
            const int bl = wg_of((int64_t)(t + 1) * A.chunks - 1, p);
            if (!arrive_last(&a.tile_cnt[t], (unsigned)(bl - bf + 1))) continue;
#pragma unroll
            for (int m = 0; m < M; ++m) v[m] = 0.0f;
            for (int bb = bf; bb <= bl; ++bb) {
                const int64_t fb = p.U * bb / p.gp;
                const int sb = fb / A.chunks == t ? 0 : 1;
#pragma unroll
                for (int m = 0; m < M; ++m) v[m] += load_sc1(&a.part[(((size_t)bb * 2 + sb) * M + m) * 64 + lane]);
            }
            if (lane == 0) store_sc1(&a.tile_cnt[t], 0u);
        }
        epi(t, v, lane);
    }
    return true;
}

// ------------------------------------------------------------ attention

// One attention unit per (row, kv head, context split): the G query heads of
// the group share every K/V element it loads. Tokens go in passes of P:
// lane (token tl, dim slice dl) holds VEC dims of K and V of its token; the
// next pass's K/V are requested before the current one is computed. Scores
// reduce over the LPT lanes of a token, softmax runs online per head (wave
// per head), and the unit writes (max, sum, unnormalised output) per head;
// the O phase merges the splits.
template <int M, int HD>
__device__ __forceinline__ bool attention_phase(const StepArgs& a, uint32_t epoch, int bar,
                                                const lyk_step_layer& Lw) {
    const int tid = phase_tid();
    constexpr int VEC = HD % 8 == 0 ? 8 : 2;       // halves of K/V per lane
    constexpr int LPT = HD / VEC;                  // lanes per token
    constexpr int TPW = 64 / LPT;                  // tokens per wave per round
    constexpr int R = kWaves * TPW;                // tokens per round
    constexpr int kRounds = R >= 64 ? 1 : 64 / R;
    constexpr int P = R * kRounds;                 // tokens per pass
    constexpr int kMaxG = 64 / VEC < 16 ? 64 / VEC : 16;
    static_assert(64 % LPT == 0, "head dim must split evenly over lanes");
    using KV = typename std::conditional<VEC == 8, u32x4, uint32_t>::type;
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float m_s[16], l_s[16], a_s[16];
    const int nq = a.md.num_heads, nkv = a.md.num_kv_heads;
    constexpr int hd = HD;
    const int G = nq / nkv, bt = a.md.block_tokens;
    const int lane = tid & 63, wave = tid >> 6;
    const int dl = lane % LPT, tl = lane / LPT;
    const float scale = 1.0f / sqrtf((float)hd);
    float* q_s = reinterpret_cast<float*>(smem);   // [G][hd]
    float* p_s = q_s + G * hd;                     // [G][P]
    float* o_s = reinterpret_cast<float*>(smem);   // [kWaves][G*hd] (after the passes)
    const int MS = a.attn_max_splits;

    if (!grid_sync(a, epoch, (uint32_t)bar)) return false;

    int splits[M], ctxs[M], units = 0;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        ctxs[m] = load_sc1(a.io.positions + m) + 1;
        splits[m] = attn_splits(ctxs[m], a.attn_split_tokens, MS);
        units += nkv * splits[m];
    }
    for (int u = blockIdx.x; u < units; u += gridDim.x) {
        int m = 0, r = u, S = splits[0], ctx = ctxs[0];
#pragma unroll
        for (int mm = 1; mm < M; ++mm)
            if (m == mm - 1 && r >= nkv * S) {
                r -= nkv * S;
                m = mm;
                S = splits[mm];
                ctx = ctxs[mm];
            }
        const int g = r / S, s = r % S;
        const int per = (ctx + S - 1) / S;
        const int t0 = s * per, t1 = min(ctx, t0 + per);
        const int* tab = a.io.block_tables + (size_t)m * a.io.table_stride;
        const size_t head_stride = (size_t)bt * hd;   // one kv head of a block
        const size_t blk_stride = (size_t)nkv * head_stride;
        const uint16_t* kc = Lw.k_cache + (size_t)g * head_stride + dl * VEC;
        const uint16_t* vc = Lw.v_cache + (size_t)g * head_stride + dl * VEC;

        // K/V of this lane's tokens of the pass starting at c0. Rows before
        // this step's position were written by earlier launches; the row at
        // the position was written with device-scope stores earlier in this
        // launch, before any read of its cache lines.
        auto load_kv = [&](int c0, KV (&kk)[kRounds], KV (&vv)[kRounds]) {
#pragma unroll
            for (int rr = 0; rr < kRounds; ++rr) {
                {
                    const int t = c0 + rr * R + wave * TPW + tl;
                    if (t < t1) {
                        const size_t off = (size_t)ld(tab + t / bt) * blk_stride + (size_t)(t % bt) * hd;
                        kk[rr] = ld(reinterpret_cast<const KV*>(kc + off));
                        vv[rr] = ld(reinterpret_cast<const KV*>(vc + off));
                    }
                }
            }
        };
        KV ka[kRounds], va[kRounds], kb[kRounds], vb[kRounds];
        load_kv(t0, ka, va);

        float acc[kMaxG][VEC];
#pragma unroll
        for (int h = 0; h < kMaxG; ++h)
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[h][e] = 0.0f;
        {
            const float* qg = a.q + (size_t)m * nq * hd + (size_t)g * G * hd;
            for (int i = tid; i < G * hd; i += kThreads) q_s[i] = load_sc1(qg + i);
        }
        if (tid < 16) { m_s[tid] = -INFINITY; l_s[tid] = 0.0f; }
        __syncthreads();
        if (u == (int)blockIdx.x) mark(a, bar, 0);

        auto pass = [&](int c0, const KV (&kk)[kRounds], const KV (&vv)[kRounds]) {
            const int n = min(P, t1 - c0);
            // scores
#pragma unroll
            for (int rr = 0; rr < kRounds; ++rr) {
                {
                    const int j = rr * R + wave * TPW + tl;
                    uint32_t kw[VEC / 2];
                    __builtin_memcpy(kw, &kk[rr], sizeof kw);
#pragma unroll
                    for (int h = 0; h < kMaxG; ++h) {
                        if (h < G) {
                            const float* qh = q_s + h * hd + dl * VEC;
                            float d = 0.0f;
#pragma unroll
                            for (int e = 0; e < VEC / 2; ++e) {
                                const half2_t k2 = as_half2(kw[e]);
                                d = fmaf(qh[2 * e], (float)k2.x, d);
                                d = fmaf(qh[2 * e + 1], (float)k2.y, d);
                            }
#pragma unroll
                            for (int o = 1; o < LPT; o <<= 1) d += __shfl_xor(d, o, 64);
                            if (dl == 0 && j < n) p_s[h * P + j] = d * scale;
                        }
                    }
                }
            }
            __syncthreads();
            // online softmax, one wave per head
            for (int h = wave; h < G; h += kWaves) {
                float mx = -INFINITY;
                for (int j = lane; j < n; j += 64) mx = fmaxf(mx, p_s[h * P + j]);
                mx = wave_max(mx);
                const float mold = m_s[h];
                const float mnew = fmaxf(mold, mx);
                float sum = 0.0f;
                for (int j = lane; j < n; j += 64) {
                    const float e = expf(p_s[h * P + j] - mnew);
                    p_s[h * P + j] = e;
                    sum += e;
                }
                sum = wave_sum(sum);
                if (lane == 0) {
                    const float alpha = expf(mold - mnew);  // 0 on the first pass
                    a_s[h] = alpha;
                    l_s[h] = l_s[h] * alpha + sum;
                    m_s[h] = mnew;
                }
            }
            __syncthreads();
            // acc = alpha * acc + sum_j p[j] v[j] over this lane's tokens
#pragma unroll
            for (int h = 0; h < kMaxG; ++h)
                if (h < G) {
                    const float al = a_s[h];
#pragma unroll
                    for (int e = 0; e < VEC; ++e) acc[h][e] *= al;
                }
#pragma unroll
            for (int rr = 0; rr < kRounds; ++rr) {
                {
                    const int j = rr * R + wave * TPW + tl;
                    if (j < n) {
                        uint32_t vw[VEC / 2];
                        __builtin_memcpy(vw, &vv[rr], sizeof vw);
#pragma unroll
                        for (int h = 0; h < kMaxG; ++h) {
                            if (h < G) {
                                const float pj = p_s[h * P + j];
#pragma unroll
                                for (int e = 0; e < VEC / 2; ++e) {
                                    const half2_t v2 = as_half2(vw[e]);
                                    acc[h][2 * e] = fmaf(pj, (float)v2.x, acc[h][2 * e]);
                                    acc[h][2 * e + 1] = fmaf(pj, (float)v2.y, acc[h][2 * e + 1]);
                                }
                            }
                        }
                    }
                }
            }
            __syncthreads();  // p_s is rewritten by the next pass
        };
        for (int c0 = t0; c0 < t1; c0 += 2 * P) {
            if (c0 + P < t1) load_kv(c0 + P, kb, vb);
            pass(c0, ka, va);
            if (c0 + P >= t1) break;
            if (c0 + 2 * P < t1) load_kv(c0 + 2 * P, ka, va);
            pass(c0 + P, kb, vb);
        }
        if (u == (int)blockIdx.x) mark(a, bar, 1);
        // reduce over the tokens of a wave, then over waves (in wave order)
#pragma unroll
        for (int h = 0; h < kMaxG; ++h)
            if (h < G)
#pragma unroll
                for (int e = 0; e < VEC; ++e) {
                    float x = acc[h][e];
#pragma unroll
                    for (int o = LPT; o < 64; o <<= 1) x += __shfl_xor(x, o, 64);
                    acc[h][e] = x;
                }
        if (tl == 0)
#pragma unroll
            for (int h = 0; h < kMaxG; ++h)
                if (h < G)
#pragma unroll
                    for (int e = 0; e < VEC; ++e) o_s[(size_t)wave * G * hd + h * hd + dl * VEC + e] = acc[h][e];
        __syncthreads();
        const size_t grp = (size_t)m * nkv + g;
        float* ml = a.attn_ml + (grp * MS + s) * G * 2;
        float* pa = a.attn_acc + (grp * MS + s) * (size_t)G * hd;
        if (tid < G) { store_sc1(&ml[2 * tid], m_s[tid]); store_sc1(&ml[2 * tid + 1], l_s[tid]); }
        for (int idx = tid; idx < G * hd; idx += kThreads) {
            float o = 0.0f;
            for (int w = 0; w < kWaves; ++w) o += o_s[(size_t)w * G * hd + idx];
            store_sc1(&pa[idx], o);
        }
        __syncthreads();  // o_s / q_s are rewritten by the next unit
    }
    return true;
}

// ------------------------------------------------------------ epilogues

// CPU's rotation with separately rounded products (no FMA).
__device__ __forceinline__ float rot_lo(float a, float b, float c, float s) {
#pragma clang fp contract(off)
    return a * c - b * s;
}
__device__ __forceinline__ float rot_hi(float a, float b, float c, float s) {
#pragma clang fp contract(off)
    return b * c + a * s;
}

struct Best {
    float v;
    int i;
};
__device__ __forceinline__ Best better(Best x, Best y) {
    if (y.v > x.v || (y.v == x.v && y.i < x.i)) return y;
    return x;
}

// ------------------------------------------------------------ the kernel

template <int M, bool Q8, int HD>
__global__ __launch_bounds__(kThreads) void decode_step_kernel(const StepArgs* __restrict__ args) {
    const StepArgs& a = *args;
    if (aborted(a)) return;
    // Every workgroup reads the barrier epoch before its first arrival;
    // workgroup 0 advances it once the first barrier shows all have read it.
    const uint32_t epoch = load_sc1(a.epoch);
    if (a.io.trace && blockIdx.x == 0 && threadIdx.x == 0) st(a.io.trace, (uint64_t)__builtin_amdgcn_s_memrealtime());
    const int b = blockIdx.x;
    const int H = a.md.hidden_size, nq = a.md.num_heads, nkv = a.md.num_kv_heads, hd = a.md.head_dim;
    const int In = a.md.intermediate_size;
    int bar = 0;
    const int L = a.md.num_layers;

    for (int l = 0; l < L; ++l) {
        const lyk_step_layer Lw = load_layer(a.md.layers + l);
        float* base = a.h + (size_t)(l & 1) * kMaxRows * H;            // residual entering layer l
        const float* prev = a.h + (size_t)((l + 1) & 1) * kMaxRows * H;  // base of layer l - 1
        // ---- RMSNorm + fused QKV GEMV + bias + RoPE + KV append
        {
            const Mat A = make_mat<Q8>(Lw.qkv_w, Lw.qkv_s, (nq + 2 * nkv) * hd, H, false);
            const int half = hd / 2, xr = half < 32 ? half : 32;
            const int qrows = nq * hd, krows = nkv * hd;
            const ResidualSrc rs = l == 0 ? ResidualSrc{nullptr, nullptr, nullptr, base, true}
                                          : ResidualSrc{prev, a.d_attn, a.d_mlp, base, false};
            const bool ok = gemv_phase<M, Q8>(
                a, epoch, l == 0 ? -1 : bar++, A,
                [&](const Mat& AA, const Part& pp, uint16_t* xs, int ftid) {
                    fill_norm<M, Q8>(a, Lw.input_norm, rs, AA, pp, xs, ftid);
                },
                [&](int t, float (&v)[M], int lane) {
                    const int pr = t * 64 + lane;
                    const bool valid = pr < A.n;
                    // packed row -> (head, natural dim): heads of hd > 64 are
                    // stored in blocks of 64 rows holding 32 rotation pairs
                    // (lanes j, j+32); smaller heads keep the natural order.
                    const int head = pr / hd, e = pr % hd;
                    int dim = e;
                    if (hd > 64) {
                        const int blk = e / 64, Lr = e % 64;
                        dim = Lr < 32 ? blk * 32 + Lr : half + blk * 32 + (Lr - 32);
                    }
                    const float bias = valid ? ld(Lw.qkv_bias + pr) : 0.0f;
                    const int sec = pr < qrows ? 0 : (pr < qrows + krows ? 1 : 2);
                    const int i = dim % half;
                    const bool lo = dim < half;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float val = v[m] + bias;
                        const float other = __shfl_xor(val, xr, 64);
                        const int pos = load_sc1(a.io.positions + m);
                        const float c = ld(a.md.rope_cos + (size_t)pos * half + i);
                        const float s = ld(a.md.rope_sin + (size_t)pos * half + i);
                        const float rot = lo ? rot_lo(val, other, c, s) : rot_hi(other, val, c, s);
                        if (!valid) continue;
                        if (sec == 0) {
                            store_sc1(&a.q[(size_t)m * qrows + (size_t)head * hd + dim], rot);
                        } else {
                            const int kvh = sec == 1 ? head - nq : head - nq - nkv;
                            const int blk = ld(a.io.block_tables + (size_t)m * a.io.table_stride +
                                               pos / a.md.block_tokens);
                            const size_t off = (((size_t)blk * nkv + kvh) * a.md.block_tokens +
                                                pos % a.md.block_tokens) * hd + dim;
                            if (sec == 1) store_sc1_u16(Lw.k_cache + off, f2h(rot));
                            else store_sc1_u16(Lw.v_cache + off, f2h(val));
                        }
                    }
                });
            if (!ok) return;
        }
        // ---- attention
        if (!attention_phase<M, HD>(a, epoch, bar++, Lw)) return;
        if (l == 0 && b == 0 && threadIdx.x == 0) store_sc1(a.epoch, epoch + a.barriers);
        // ---- O GEMV (input: merged attention splits) -> attention delta
        {
            const Mat A = make_mat<Q8>(Lw.o_w, Lw.o_s, H, nq * hd, false);
            const bool ok = gemv_phase<M, Q8>(
                a, epoch, bar++, A,
                [&](const Mat& AA, const Part& pp, uint16_t* xs, int ftid) { fill_attn<M, Q8>(a, AA, pp, xs, ftid); },
                [&](int t, float (&v)[M], int lane) {
                    const int r = t * 64 + lane;
                    if (r >= H) return;
#pragma unroll
                    for (int m = 0; m < M; ++m) store_sc1(&a.d_attn[(size_t)m * H + r], v[m]);
                });
            if (!ok) return;
        }
        // ---- RMSNorm + gate/up GEMV + SiLU
        {
            const Mat A = make_mat<Q8>(Lw.gateup_w, Lw.gateup_s, In, H, true);
            const ResidualSrc rs{base, a.d_attn, nullptr, nullptr, false};
            const bool ok = gemv_phase<M, Q8>(
                a, epoch, bar++, A,
                [&](const Mat& AA, const Part& pp, uint16_t* xs, int ftid) {
                    fill_norm<M, Q8>(a, Lw.post_norm, rs, AA, pp, xs, ftid);
                },
                [&](int t, float (&v)[M], int lane) {
                    const int j = t * 32 + lane;
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float u = __shfl_down(v[m], 32, 64);
                        if (lane < 32 && j < In) {
                            const float g = v[m];
                            store_sc1_u16(&a.act[(size_t)m * a.ld_act + j], f2h(g / (1.0f + expf(-g)) * u));
                        }
                    }
                });
            if (!ok) return;
        }
        // ---- down GEMV -> MLP delta
        {
            const Mat A = make_mat<Q8>(Lw.down_w, Lw.down_s, H, In, false);
            const bool ok = gemv_phase<M, Q8>(
                a, epoch, bar++, A,
                [&](const Mat& AA, const Part& pp, uint16_t* xs, int ftid) { fill_copy<M, Q8>(a.act, a.ld_act, AA, pp, xs, ftid); },
                [&](int t, float (&v)[M], int lane) {
                    const int r = t * 64 + lane;
                    if (r >= H) return;
#pragma unroll
                    for (int m = 0; m < M; ++m) store_sc1(&a.d_mlp[(size_t)m * H + r], v[m]);
                });
            if (!ok) return;
        }
    }
    if (a.io.mode == LYK_STEP_HIDDEN) {
        if (a.io.trace && b == 0 && threadIdx.x == 0) st(a.io.trace + bar + 1, (uint64_t)__builtin_amdgcn_s_memrealtime());
        return;
    }

    // ---- final norm + LM head (+ per-tile greedy candidates)
    const int V = a.md.vocab_size;
    const bool greedy = a.io.mode == LYK_STEP_GREEDY;
    const Mat A = make_mat<Q8>(a.md.lm_head_w, a.md.lm_head_s, V, H, false);
    const ResidualSrc rs{a.h + (size_t)((L - 1) & 1) * kMaxRows * H, a.d_attn, a.d_mlp, nullptr, false};
    const bool ok = gemv_phase<M, Q8>(
        a, epoch, bar++, A,
        [&](const Mat& AA, const Part& pp, uint16_t* xs, int ftid) {
            fill_norm<M, Q8>(a, a.md.final_norm, rs, AA, pp, xs, ftid);
        },
        [&](int t, float (&v)[M], int lane) {
            const int r = t * 64 + lane;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                if (r < V) st(a.io.logits + (size_t)m * a.io.ld_logits + r, v[m]);
                if (!greedy) continue;
                float x = v[m];
                int bad = 0;
                if (r < V && !isfinite(x)) {
                    bad = 1;
                    if (isnan(x)) x = -INFINITY;
                }
                Best bst = r < V ? Best{x, r} : Best{-INFINITY, 0x7fffffff};
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) bst = better(bst, Best{__shfl_xor(bst.v, o, 64), __shfl_xor(bst.i, o, 64)});
                bad = (int)wave_sum((float)bad);
                if (lane == 0) {
                    const size_t sl = (size_t)m * A.tiles + t;
                    store_sc1(&a.best_v[sl], bst.v);
                    store_sc1(&a.best_i[sl], bst.i);
                    store_sc1(&a.best_bad[sl], bad);
                }
            }
        });
    if (!ok) return;
    if (!greedy) {
        if (a.io.trace && b == 0 && threadIdx.x == 0) st(a.io.trace + bar + 1, (uint64_t)__builtin_amdgcn_s_memrealtime());
        return;
    }
    if (!grid_sync(a, epoch, (uint32_t)bar++)) return;
    if (b != 0) return;
    // ---- greedy token of row 0 (M == 1): first index of the maximum
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ float bv[kWaves];
    __shared__ int bi[kWaves], bb[kWaves];
    Best bst{-INFINITY, 0x7fffffff};
    int bad = 0;
    for (int t = tid; t < A.tiles; t += kThreads) {
        bst = better(bst, Best{load_sc1(&a.best_v[t]), load_sc1_i32(&a.best_i[t])});
        bad += load_sc1_i32(&a.best_bad[t]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) bst = better(bst, Best{__shfl_xor(bst.v, o, 64), __shfl_xor(bst.i, o, 64)});
    bad = (int)wave_sum((float)bad);
    if (lane == 0) { bv[wave] = bst.v; bi[wave] = bst.i; bb[wave] = bad; }
    __syncthreads();
    if (tid == 0) {
        Best r{bv[0], bi[0]};
        int nb = bb[0];
        for (int w = 1; w < kWaves; ++w) { r = better(r, Best{bv[w], bi[w]}); nb += bb[w]; }
        const int token = r.i < V ? r.i : 0;
        // device-scope stores: the next step may run on other XCDs
        store_sc1(a.io.tokens, token);
        store_sc1(a.io.positions, load_sc1(a.io.positions) + 1);
        if (a.io.nonfinite) st(a.io.nonfinite, ld(a.io.nonfinite) + nb);
        if (a.io.history && a.io.step) {
            const int s = ld(a.io.step);
            st(a.io.history + s, token);
            st(a.io.step, s + 1);
        }
        if (a.io.trace) st(a.io.trace + bar + 1, (uint64_t)__builtin_amdgcn_s_memrealtime());
    }
}

// ------------------------------------------------------------ host side


int chunks_of(int64_t k, bool q8) {
    const int unit = q8 ? 16 : 32;
    return (int)(((k + unit - 1) / unit + 7) / 8);
}

int vec_of(int hd) { return hd % 8 == 0 ? 8 : 2; }

// Tokens per attention pass (the kernel's P for this head dim).
int pass_tokens(int hd) {
    const int lpt = hd / vec_of(hd), tpw = 64 / lpt, R = kWaves * tpw;
    return R >= 64 ? R : R * (64 / R);
}

// Head dims with a compiled attention path.
bool head_dim_supported(int hd) { return hd == 4 || hd == 64 || hd == 128; }

int step_grid() {
    static int grid = 0;
    if (grid == 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
        grid = prop.multiProcessorCount;
    }
    return grid;
}

// Checks the model geometry against what the kernel supports.
int check_model(const lyk_step_model& md) {
    if (md.vocab_size < 1 || md.hidden_size < 2 || md.num_layers < 1 || md.num_heads < 1 ||
        md.num_kv_heads < 1 || md.head_dim < 2 || md.intermediate_size < 2 || md.block_tokens < 1 ||
        md.num_blocks < 1 || md.rope_positions < 1)
        return LYK_ERR_INVALID_ARG;
    if (!md.embed || !md.final_norm || !md.lm_head_w || !md.lm_head_s || !md.layers || !md.rope_cos ||
        !md.rope_sin)
        return LYK_ERR_INVALID_ARG;
    const int hd = md.head_dim;
    if (md.num_heads % md.num_kv_heads) return LYK_ERR_INVALID_ARG;
    const int G = md.num_heads / md.num_kv_heads;
    const int vec = vec_of(hd);
    if (!head_dim_supported(hd)) return LYK_ERR_SHAPE;
    if (G > (64 / vec < 16 ? 64 / vec : 16)) return LYK_ERR_SHAPE;
    if (md.hidden_size > kNormPer * kThreads || (md.intermediate_size & 1) ||
        ((int64_t)md.num_heads * hd) & 1)
        return LYK_ERR_SHAPE;
    return LYK_OK;
}

struct Layout {
    uint64_t err, epoch, args, bar, tile_cnt, part, attn_ml, attn_acc, h, d_attn, d_mlp, q, act, best_v,
        best_i, best_bad, total;
    int ld_act, head_tiles;
};

Layout layout(const lyk_step_model& md, int rows, int grid) {
    Layout L{};
    const bool q8 = md.q8 != 0;
    const int ck = q8 ? 128 : 256;
    const int nq = md.num_heads, nkv = md.num_kv_heads, hd = md.head_dim, G = nq / nkv;
    L.ld_act = chunks_of(md.intermediate_size, q8) * ck;
    L.head_tiles = (md.vocab_size + 63) / 64;
    const int tiles_max = std::max({L.head_tiles, (md.intermediate_size + 31) / 32,
                                    (md.hidden_size + 63) / 64, ((nq + 2 * nkv) * hd + 63) / 64});
    uint64_t at = 0;
    auto take = [&](uint64_t bytes) {
        const uint64_t o = at;
        at += (bytes + 255) / 256 * 256;
        return o;
    };
    L.err = take(4);
    L.epoch = take(4);
    L.args = take(sizeof(StepArgs));
    L.bar = take((uint64_t)kBarLines * kLineWords * 4);
    L.tile_cnt = take((uint64_t)tiles_max * 4);
    L.part = take((uint64_t)grid * 2 * rows * 64 * 4);
    L.attn_ml = take((uint64_t)rows * nkv * kAttnMaxSplits * G * 2 * 4);
    L.attn_acc = take((uint64_t)rows * nkv * kAttnMaxSplits * G * hd * 4);
    L.h = take((uint64_t)2 * kMaxRows * md.hidden_size * 4);
    L.d_attn = take((uint64_t)rows * md.hidden_size * 4);
    L.d_mlp = take((uint64_t)rows * md.hidden_size * 4);
    L.q = take((uint64_t)rows * nq * hd * 4);
    L.act = take((uint64_t)rows * L.ld_act * 2);
    L.best_v = take((uint64_t)rows * L.head_tiles * 4);
    L.best_i = take((uint64_t)rows * L.head_tiles * 4);
    L.best_bad = take((uint64_t)rows * L.head_tiles * 4);
    L.total = at;
    return L;
}

// The five GEMVs of a step: {rows, k, paired}.
struct MatShape {
    int64_t n, k;
    bool paired;
};
void step_mats(const lyk_step_model& md, MatShape (&out)[5]) {
    const int64_t H = md.hidden_size, In = md.intermediate_size, nq = md.num_heads, nkv = md.num_kv_heads,
                  hd = md.head_dim;
    out[0] = {(nq + 2 * nkv) * hd, H, false};
    out[1] = {H, nq * hd, false};
    out[2] = {In, H, true};
    out[3] = {H, In, false};
    out[4] = {md.vocab_size, H, false};
}

// Largest chunk range of one workgroup in a phase (as partition() cuts it).
int64_t max_range(const MatShape& mt, bool q8, int grid, int64_t* chunks_out) {
    const int64_t tiles = mt.paired ? (mt.n + 31) / 32 : (mt.n + 63) / 64;
    const int64_t chunks = chunks_of(mt.k, q8);
    const int64_t U = tiles * chunks;
    *chunks_out = chunks;
    if (tile_aligned(tiles, chunks, grid)) return (tiles + grid - 1) / grid * chunks;
    const int64_t gp = U < grid ? U : grid;
    return (U + gp - 1) / gp;
}

// Dynamic LDS of a launch: the largest x window (plus, for the O phase, the
// split-merge weights) or reduction buffer of any GEMV phase, or the
// attention buffers.
size_t lds_bytes(const lyk_step_model& md, int rows, int grid) {
    const bool q8 = md.q8 != 0;
    const int ck = q8 ? 128 : 256;
    MatShape mats[5];
    step_mats(md, mats);
    size_t need = (size_t)kWaves * kPieces * rows * 64 * 4;
    for (int i = 0; i < 5; ++i) {
        int64_t chunks = 0;
        const int64_t per = max_range(mats[i], q8, grid, &chunks);
        const int64_t win = per >= chunks ? chunks : per;
        size_t bytes = (size_t)rows * win * ck * 2;
        if (i == 1) {  // O phase: merge weights of the heads in the window
            const int64_t nh = std::min<int64_t>(md.num_heads, (win * ck + md.head_dim - 1) / md.head_dim + 1);
            bytes += (size_t)rows * nh * (kAttnMaxSplits + 1) * 4;
        }
        need = std::max(need, bytes);
    }
    const int G = md.num_heads / md.num_kv_heads, hd = md.head_dim;
    need = std::max(need, (size_t)G * (pass_tokens(hd) + hd) * 4);
    need = std::max(need, (size_t)kWaves * G * hd * 4);
    return need;
}

// Largest number of row tiles one wave's range can touch, over the phases.
bool pieces_ok(const lyk_step_model& md, int grid) {
    const bool q8 = md.q8 != 0;
    MatShape mats[5];
    step_mats(md, mats);
    for (const MatShape& mt : mats) {
        int64_t chunks = 0;
        const int64_t per = max_range(mt, q8, grid, &chunks);
        const int64_t lw = (per + kWaves - 1) / kWaves;   // chunks per wave, at most
        if (1 + (lw - 1 + chunks - 1) / chunks > kPieces) return false;
    }
    return true;
}

template <int M, bool Q8, int HD>
int launch(const StepArgs* d_args, int grid, size_t lds, hipStream_t st) {
    auto kern = decode_step_kernel<M, Q8, HD>;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, kThreads, lds) != hipSuccess || occ < 1)
        return LYK_ERR_SHAPE;
    void* params[] = {&d_args};
    if (hipLaunchCooperativeKernel(reinterpret_cast<const void*>(kern), dim3(grid), dim3(kThreads), params,
                                   (unsigned)lds, st) != hipSuccess)
        return LYK_ERR_LAUNCH;
    return LYK_OK;
}

template <bool Q8, int HD>
int launch_rows(int m, const StepArgs* d_args, int grid, size_t lds, hipStream_t st) {
    switch (m) {
        case 1: return launch<1, Q8, HD>(d_args, grid, lds, st);
        case 2: return launch<2, Q8, HD>(d_args, grid, lds, st);
        case 3: return launch<3, Q8, HD>(d_args, grid, lds, st);
        default: return launch<4, Q8, HD>(d_args, grid, lds, st);
    }
}

template <bool Q8>
int launch_hd(int hd, int m, const StepArgs* d_args, int grid, size_t lds, hipStream_t st) {
    switch (hd) {
        case 128: return launch_rows<Q8, 128>(m, d_args, grid, lds, st);
        case 64: return launch_rows<Q8, 64>(m, d_args, grid, lds, st);
        default: return launch_rows<Q8, 4>(m, d_args, grid, lds, st);
    }
}

// Launch arguments live in the workspace; they are uploaded (in stream
// order) only when they differ from the last ones written to that
// workspace, so a run of identical steps (GreedyRun) uploads once.
struct ArgsCache {
    std::mutex mu;
    std::unordered_map<const void*, StepArgs> last;
};
ArgsCache& args_cache() {
    static ArgsCache c;
    return c;
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

uint64_t lyk_hip_step_workspace_bytes(const lyk_step_model* model, int max_rows) {
    if (!model || max_rows < 1 || max_rows > kMaxRows || check_model(*model) != LYK_OK) return 0;
    const int grid = step_grid();
    if (grid < 1) return 0;
    return layout(*model, max_rows, grid).total;
}

uint32_t lyk_hip_step_barriers(const lyk_step_model* model, int mode) {
    if (!model) return 0;
    // per layer: before attention, O, gate/up, down, and before the next
    // layer's QKV; the last of these is the LM head's (LOGITS, GREEDY); the
    // greedy argmax waits for one more
    const uint32_t layers = (uint32_t)model->num_layers * 5u;
    return mode == LYK_STEP_HIDDEN ? layers - 1u : (mode == LYK_STEP_GREEDY ? layers + 1u : layers);
}

int lyk_hip_decode_step(const lyk_step_model* model, const lyk_step_io* io, void* d_workspace,
                        uint64_t workspace_bytes, int max_rows, void* stream) {
    if (!model || !io || !d_workspace) return LYK_ERR_INVALID_ARG;
    int rc = check_model(*model);
    if (rc != LYK_OK) return rc;
    const int m = io->m;
    if (m < 1 || m > max_rows || max_rows > kMaxRows || !io->tokens || !io->positions || !io->block_tables ||
        io->table_stride < 1)
        return LYK_ERR_INVALID_ARG;
    if (io->mode < LYK_STEP_HIDDEN || io->mode > LYK_STEP_GREEDY) return LYK_ERR_INVALID_ARG;
    if (io->mode != LYK_STEP_HIDDEN && (!io->logits || io->ld_logits < model->vocab_size)) return LYK_ERR_INVALID_ARG;
    if (io->mode == LYK_STEP_GREEDY && m != 1) return LYK_ERR_INVALID_ARG;
    const int grid = step_grid();
    if (grid < 1) return LYK_ERR_HIP;
    if (!pieces_ok(*model, grid)) return LYK_ERR_SHAPE;
    const Layout L = layout(*model, max_rows, grid);
    if (L.total > workspace_bytes) return LYK_ERR_WORKSPACE;
    const size_t lds = lds_bytes(*model, m, grid);
    if (lds > 48 * 1024) return LYK_ERR_SHAPE;

    char* ws = static_cast<char*>(d_workspace);
    StepArgs a;
    std::memset(&a, 0, sizeof a);
    a.md = *model;
    a.io = *io;
    a.err = reinterpret_cast<int*>(ws + L.err);
    a.epoch = reinterpret_cast<uint32_t*>(ws + L.epoch);
    a.bar = reinterpret_cast<unsigned*>(ws + L.bar);
    a.tile_cnt = reinterpret_cast<unsigned*>(ws + L.tile_cnt);
    a.part = reinterpret_cast<float*>(ws + L.part);
    a.attn_ml = reinterpret_cast<float*>(ws + L.attn_ml);
    a.attn_acc = reinterpret_cast<float*>(ws + L.attn_acc);
    a.h = reinterpret_cast<float*>(ws + L.h);
    a.d_attn = reinterpret_cast<float*>(ws + L.d_attn);
    a.d_mlp = reinterpret_cast<float*>(ws + L.d_mlp);
    a.q = reinterpret_cast<float*>(ws + L.q);
    a.act = reinterpret_cast<uint16_t*>(ws + L.act);
    a.best_v = reinterpret_cast<float*>(ws + L.best_v);
    a.best_i = reinterpret_cast<int*>(ws + L.best_i);
    a.best_bad = reinterpret_cast<int*>(ws + L.best_bad);
    a.ld_act = L.ld_act;
    a.attn_split_tokens = kAttnSplitTokens;
    a.attn_max_splits = kAttnMaxSplits;
    a.barriers = lyk_hip_step_barriers(model, io->mode);
    hipStream_t st = static_cast<hipStream_t>(stream);
    StepArgs* d_args = reinterpret_cast<StepArgs*>(ws + L.args);
    {
        ArgsCache& cache = args_cache();
        std::lock_guard<std::mutex> lock(cache.mu);
        auto it = cache.last.find(d_workspace);
        if (it == cache.last.end() || std::memcmp(&it->second, &a, sizeof a) != 0) {
            if (hipMemcpyAsync(d_args, &a, sizeof a, hipMemcpyHostToDevice, st) != hipSuccess) return LYK_ERR_HIP;
            cache.last[d_workspace] = a;
        }
    }
    rc = model->q8 ? launch_hd<true>(model->head_dim, m, d_args, grid, lds, st)
                   : launch_hd<false>(model->head_dim, m, d_args, grid, lds, st);
    return rc;
}

int lyk_hip_step_reset(void* d_workspace, uint64_t workspace_bytes, void* stream) {
    if (!d_workspace) return LYK_ERR_INVALID_ARG;
    {
        ArgsCache& cache = args_cache();
        std::lock_guard<std::mutex> lock(cache.mu);
        cache.last.erase(d_workspace);
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (hipMemsetAsync(d_workspace, 0, workspace_bytes, st) != hipSuccess) return LYK_ERR_HIP;
    return LYK_OK;
}

int lyk_hip_step_error(const void* d_workspace, int32_t* error_out, void* stream) {
    if (!d_workspace || !error_out) return LYK_ERR_INVALID_ARG;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(error_out, d_workspace, 4, hipMemcpyDeviceToHost, st) != hipSuccess) return LYK_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return LYK_ERR_HIP;
    return LYK_OK;
}

void lyk_qkv_rope_order(int nq, int nkv, int hd, int32_t* perm) {
    const int rows = (nq + 2 * nkv) * hd, half = hd / 2;
    for (int pr = 0; pr < rows; ++pr) {
        const int head = pr / hd, e = pr % hd;
        int dim = e;
        if (hd > 64) {
            const int blk = e / 64, L = e % 64;
            dim = L < 32 ? blk * 32 + L : half + blk * 32 + (L - 32);
        }
        perm[pr] = head * hd + dim;
    }
}

}  // extern "C"
