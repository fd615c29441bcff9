// The whole decode step of a Qwen2 model as one persistent, cooperative
// launch on gfx950: embedding, every layer (RMSNorm, fused QKV GEMV, bias +
// RoPE + paged KV append, GQA attention, O GEMV + residual, RMSNorm, gate/up
// GEMV + SiLU, down GEMV + residual), the final norm, the LM head and the
// greedy argmax.
//
// Reference: one QwenCudaModel::Decode / DecodeBatch / GreedyRun step
// (backends/cuda/qwen_cuda_model.cu:2641-2776, 2778-3102), whose CPU
// counterpart is QwenModel::Forward (model/architectures/qwen/
// qwen_model.cpp:216-331). The CUDA backend launches ~10 kernels per layer;
// on MI355X each kernel boundary costs a launch, a ramp-up/drain of 256 CUs
// and an L2 write-back across 8 XCDs, which at batch 1 costs more than the
// weights take to stream. Here one workgroup per CU stays resident for the
// whole step.
//
// Dataflow instead of barriers
//   * Every value one workgroup hands to another is a 64-bit word: a 32-bit
//     payload and a 32-bit tag (launch number << 8 | layer), written with one
//     device-scope (sc1) store, coherent across the XCDs' L2s. A consumer
//     polls exactly the words it needs until their tags match; the producer
//     never waits. Phases overlap: a workgroup starts the next phase as soon
//     as its own inputs are there.
//   * Before polling, each wave requests its first weight chunks of the
//     phase (weights never depend on the inputs), and attention requests the
//     K/V rows of earlier positions, so the wait overlaps HBM traffic.
//   * The residual stream lives in registers: every workgroup keeps the whole
//     fp32 vector (7 values per thread at hidden 3584) and adds the attention
//     and MLP outputs itself, in the reference's order, before each RMSNorm.
//   * GEMV phases: each workgroup takes whole row tiles (64 rows, one per
//     lane), its 8 waves split the tile's K chunks and combine in LDS. When a
//     matrix has too few tiles for the grid (down projection) every tile's K
//     range is cut into pieces; piece 0's workgroup adds the others' tagged
//     partials in piece order (for QKV, attention adds the pieces as it
//     reads them). The activation vector sits in LDS.
//   * Attention units are (row, kv head, context split), q.k and p.v on the
//     matrix cores; the splits of a kv head merge in split order, each split
//     finishing a slice of the outputs.
//   * Buffers are reused across layers; tags carry the layer, and every
//     reader of a reused buffer produces data that the next writer of that
//     buffer (a later layer) waits for, so no write overtakes a read. The
//     attention / MLP outputs that every workgroup reads for its residual
//     have one buffer per layer.
//   * Every wait is bounded: after ~2 s the workgroup records an error in the
//     workspace and the grid exits; later launches exit at once until the
//     host resets the workspace.
// All reductions run in a fixed order, so results do not depend on timing,
// and a row's arithmetic does not depend on the other rows of the batch.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace lyk {
namespace {

typedef unsigned long long u64;

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kPieces = 4;           // row tiles one wave's range may touch
constexpr int kNormPer = 10;         // hidden_size <= kNormPer * kThreads
constexpr int kMaxRows = 4;
constexpr int kAttnMaxSplits = 64;   // context splits per (row, kv head), at most (a lane each in the merge)
constexpr int kAttnDefaultSplits = 32;   // the default cap, at most (attn_splits_cap)
constexpr int kAttnMinDefaultSplits = 8;  // and at least
constexpr int kAttnSplitTokens = 32; // default: tokens per split, at least
constexpr int kChunkBlocks = 4;      // 16-byte blocks per lane in a GEMV chunk
constexpr int kMinPieceChunks = 4;   // K chunks per piece of a split tile, at least
constexpr int kMaxPieces = 8;        // pieces per split tile, at most
constexpr uint64_t kSpinTicks = 200000000ull;  // default wait limit; s_memrealtime is 100 MHz: 2 s
constexpr size_t kMaxDynamicLds = 158 * 1024;   // of gfx950's 160 KiB per workgroup; the rest is static
// Batches of up to kFoldRows rows fold the int4/int8 code offsets out of the
// GEMV inner loop (a per-unit correction table beside the x window); wider
// batches, whose windows leave no LDS for the table, subtract them in the loop.
constexpr int kFoldRows = 2;

struct StepArgs {
    lyk_step_model md;
    lyk_step_io io;
    int* err;
    uint32_t* seq;        // [grid] launches completed, per workgroup
    u64* qkv;             // [M][(nq+2nkv)*hd] raw QKV sums (fp32 bits)
    u64* attn_ml;         // [M][nkv][splits][G][2] per-split max and sum
    u64* attn_acc;        // [M][nkv][splits][G][hd] per-split unnormalised output
    u64* attn_out;        // [M][nq*hd] attention output
    u64* d_attn;          // [layers][M][hidden] attention block output
    u64* d_mlp;           // [layers][M][hidden] MLP block output
    u64* act;             // [M][intermediate/2] fp16 pairs of SiLU(gate) * up
    u64* dpart;           // [5][dpart_stride] split-tile partials [tiles][pieces][M][64] per GEMV kind
    size_t dpart_stride;
    u64* best;            // [M][head tiles][3] greedy candidates (value, index, non-finite)
    int attn_split_tokens;  // context tokens per attention split, at least (multiple of 16)
    int attn_max_splits;    // attention splits per (row, kv head), at most
    int phases;             // phases of one launch (trace layout)
    int pf_off;             // LDS byte offset of the gate/up staging region
    int pf_chunks;          // gate/up chunks per wave staged there (0: none)
    int o_grid;             // workgroups of the o phase: the lowest o_grid of the grid
    uint64_t spin_ticks;    // a wait gives up after this many s_memrealtime ticks
};

// ------------------------------------------------------------ primitives

__device__ __forceinline__ void store_sc1_u16(uint16_t* p, uint16_t v) { store_sc1<uint16_t>(p, v); }

__device__ __forceinline__ void put(u64* p, uint32_t payload, uint32_t tag) {
    store_sc1<u64>(p, ((u64)tag << 32) | payload);
}
__device__ __forceinline__ bool take(const u64* p, uint32_t tag, uint32_t& payload) {
    const u64 w = load_sc1<u64>(p);
    payload = (uint32_t)w;
    return (uint32_t)(w >> 32) == tag;
}
__device__ __forceinline__ uint32_t fbits(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float bitsf(uint32_t u) { return __builtin_bit_cast(float, u); }

// One attempt at N tagged words. The loads of every word still missing are
// issued before any is tested, so an attempt costs one memory round trip for
// the whole batch (testing a word before the next load is issued costs a
// round trip per word); words already in are not read again (Skip; the
// multi-row kernels re-read them, which keeps their register budget). (Polling one
// word until something arrives, then the rest, was measured slower: the
// extra round trip lands on the late workgroups.) at(u) must give a readable
// address for every u; word u is
// wanted when bit u of `want` is set and it has not arrived yet (bit u of
// `have`), and got(u, payload) takes it on arrival. Returns the wanted
// words still missing.
template <int N, bool Skip = true, class At, class Got>
__device__ __forceinline__ int poll_batch(uint32_t want, uint32_t& have, uint32_t tag, At at, Got got) {
    static_assert(N <= 32, "batch");
    const uint32_t pend = want & ~have;
    u64 w[N];
#pragma unroll
    for (int u = 0; u < N; ++u) w[u] = !Skip || (pend >> u & 1) ? load_sc1(at(u)) : 0ull;
    int missing = 0;
#pragma unroll
    for (int u = 0; u < N; ++u) {
        const bool wanted = pend >> u & 1;
        const bool hit = (uint32_t)(w[u] >> 32) == tag;
        if (wanted && hit) {
            have |= 1u << u;
            got(u, (uint32_t)w[u]);
        }
        missing += wanted && !hit ? 1 : 0;
    }
    return missing;
}

__device__ __forceinline__ bool aborted(const StepArgs& a) { return load_sc1<int>(a.err) != 0; }

// Polls until `pending()` (which re-reads the words still missing and
// returns how many remain) reaches 0. Bounded: records an error after ~2 s
// and gives up when any workgroup has. Per thread; the caller combines the
// result over the workgroup.
template <class F>
__device__ __forceinline__ bool spin(const StepArgs& a, F pending) {
    if (pending() == 0) return true;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 1;; ++it) {
        __builtin_amdgcn_s_sleep(2);
        if (pending() == 0) return true;
        if (__builtin_amdgcn_s_memrealtime() - t0 > a.spin_ticks) {
            store_sc1(a.err, 1);
            return false;
        }
        if ((it & 15) == 0 && aborted(a)) return false;
    }
}

// threadIdx.x through an opaque move: values derived from it are recomputed
// in every phase instead of being hoisted out of the layer loop and kept
// live (in registers) across all phases.
__device__ __forceinline__ int phase_tid() {
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
    return t;
}

// The layer table entry (device memory) as 13 pointer-sized loads.
__device__ __forceinline__ lyk_step_layer load_layer(const lyk_step_layer* p) {
    static_assert(sizeof(lyk_step_layer) == 13 * sizeof(uint64_t), "layer table entry layout");
    const LYK_GLOBAL uint64_t* q = (const LYK_GLOBAL uint64_t*)p;
    uint64_t w[13];
#pragma unroll
    for (int i = 0; i < 13; ++i) w[i] = q[i];
    return __builtin_bit_cast(lyk_step_layer, w);
}

// Profiling timestamp (lyk_step_io::trace) of this workgroup: phase ph
// entered (0), inputs ready (1), main loop done (2), outputs written (3).
__device__ __forceinline__ void mark(const StepArgs& a, int ph, int kind) {
    if (a.io.trace && threadIdx.x == 0)
        st(a.io.trace + (size_t)blockIdx.x * (2 + 4 * a.phases) + 2 + 4 * ph + kind,
           (uint64_t)__builtin_amdgcn_s_memrealtime());
}

// Whether x holds in any thread of the workgroup. (HIP's __syncthreads_or
// reads the workgroup size from the dispatch packet with a vector load; the
// wait for it also waits for every load issued before, prefetched weight
// chunks included.)
// Each call site (Site) has its own votes, so one barrier suffices: a wave
// rewrites a site's votes only at that site's next call, and a barrier lies
// between any two calls of one site, which every wave reaches only once it
// has read the votes.
template <int Site>
__device__ __forceinline__ bool block_any(bool x) {
    __shared__ uint32_t votes[kWaves];
    const int t = threadIdx.x;
    const bool w = __ballot(x) != 0;
    if ((t & 63) == 0) votes[t >> 6] = w ? 1u : 0u;
    __syncthreads();
    uint32_t r = 0;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) r |= votes[i];
    return r != 0;
}

// Sum of v over the workgroup for M rows; every thread gets the sums. Waves
// are added in wave order. One barrier: the caller (the RMSNorm window) is
// followed by a barrier before any next call rewrites the partials.
template <int M>
__device__ __forceinline__ void block_sum_rows(float (&v)[M], int tid) {
    __shared__ float part[kWaves][kMaxRows];
    const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float s = wave_total(v[m]);
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
}

// ------------------------------------------------------------ GEMV phase

// A matrix in the tiled layout (lyk_q*_pack_tiled): tiles of tr rows; lane l
// of a block covers row l % tr and unit l / tr of the block's lpr = 64 / tr
// units (a unit = 32 k for int4, 16 k for int8); 4 blocks per chunk.
struct Mat {
    const u32x4* w;
    const void* s;
    int n;        // output rows (paired: rows of each matrix)
    int k;
    int tr, lpr;  // rows per tile, lanes per row
    int tiles;
    int nb;       // valid blocks per tile
    int chunks;   // chunks per tile
    int ck;       // k values of one chunk
};

template <bool Q8>
__device__ __forceinline__ Mat make_mat(const void* w, const void* s, int n, int k, bool paired, int tr) {
    Mat m;
    m.w = static_cast<const u32x4*>(w);
    m.s = s;
    m.n = n;
    m.k = k;
    m.tr = tr;
    m.lpr = 64 / tr;
    m.tiles = paired ? (n + tr / 2 - 1) / (tr / 2) : (n + tr - 1) / tr;
    const int unit = Q8 ? 16 : 32;
    m.nb = ((k + unit - 1) / unit + m.lpr - 1) / m.lpr;
    m.chunks = (m.nb + kChunkBlocks - 1) / kChunkBlocks;
    m.ck = kChunkBlocks * m.lpr * unit;
    return m;
}

// Pieces each row tile's K range is cut into: 1 unless the matrix has too
// few tiles to give every workgroup work and each piece keeps at least
// kMinPieceChunks chunks.
__host__ __device__ __forceinline__ int tile_pieces(int tiles, int chunks, int G) {
    if (tiles * 2 > G) return 1;
    int p = G / tiles;
    const int pmax = chunks / kMinPieceChunks;
    if (p > pmax) p = pmax;
    if (p > kMaxPieces) p = kMaxPieces;
    return p < 1 ? 1 : (int)p;
}

// The workgroup's share of a phase: chunk range [f0, f1) of the flattened
// (tile, chunk) space (whole tiles, or one piece of one tile) and the window
// of K chunks it reads: LDS slot s holds chunk ca + s. 32-bit throughout: the
// space has at most a few 10^5 chunks, and 64-bit division is a long
// software sequence on the GPU.
struct Part {
    int f0, f1;
    int pieces, gp;   // pieces per tile; workgroups with work
    int ca, win;
    bool busy;
};

// G: the workgroups the phase spreads over, from blockIdx 0 (the whole grid
// but for o, which keeps off the top of the grid where attention units run).
__device__ __forceinline__ Part partition(const Mat& A, int G) {
    Part p;
    const int b = blockIdx.x;
    p.pieces = tile_pieces(A.tiles, A.chunks, G);
    if (p.pieces == 1) {
        p.gp = A.tiles < G ? A.tiles : G;
        p.busy = b < p.gp;
        p.f0 = p.busy ? A.tiles * b / p.gp * A.chunks : 0;
        p.f1 = p.busy ? A.tiles * (b + 1) / p.gp * A.chunks : 0;
        p.ca = 0;
        p.win = A.chunks;
    } else {
        p.gp = A.tiles * p.pieces;
        p.busy = b < p.gp;
        const int t = b / p.pieces, s = b % p.pieces;
        const int c0 = A.chunks * s / p.pieces, c1 = A.chunks * (s + 1) / p.pieces;
        p.f0 = p.busy ? t * A.chunks + c0 : 0;
        p.f1 = p.busy ? t * A.chunks + c1 : 0;
        p.ca = c0;
        p.win = c1 - c0;
    }
    return p;
}

// The shapes of the five GEMV phases' matrices (qkv, o, gate/up, down, LM
// head: the phase slots) and this workgroup's share of each, computed once
// per launch into LDS by geo_init: make_mat and partition divide by run-time
// values (a VALU division is ~25 ops), and done at every phase entry they
// sat on the critical path of the workgroups that finish a phase last.
struct Geo {
    int n, k, tr, lpr, tiles, nb, chunks, ck;
    int f0, f1, pieces, gp, ca, win, busy;
    uint32_t cmag;   // x / chunks == (x * cmag) >> csh for 0 <= x < 2^24
    int csh;
};
// Granlund-Montgomery reciprocal of d (1 <= d < 2^24) for 24-bit dividends:
// l = ceil(log2 d), m = floor(2^(24+l) / d) + 1 < 2^26; then m*d lies in
// (2^(24+l), 2^(24+l) + 2^l], which makes floor(x*m / 2^(24+l)) == x / d.
__host__ __device__ __forceinline__ void recip24(int d, uint32_t& m, int& sh) {
    int l = 0;
    while ((1 << l) < d) ++l;
    sh = 24 + l;
    m = (uint32_t)((1ull << sh) / (uint64_t)d + 1);
}
__device__ __forceinline__ int div24(int x, uint32_t m, int sh) {
    return (int)(((uint64_t)(uint32_t)x * m) >> sh);
}
// x / d for 0 <= x < 2^20, 1 <= d < 2^12, through the hardware fp32
// reciprocal: x * rcp(d) is within 1/8 of x / d (relative error below
// 2^-22), so its truncation is off by at most one, which one comparison each
// way corrects. A few VALU ops instead of an integer division's ~25.
__device__ __forceinline__ int sdiv(int x, int d) {
    int q = (int)((float)x * __builtin_amdgcn_rcpf((float)d));
    if (q * d > x) --q;
    else if ((q + 1) * d <= x) ++q;
    return q;
}
__device__ __forceinline__ Geo* geo_table() {
    __shared__ Geo geo[5];
    return geo;
}
template <bool Q8>
__device__ __forceinline__ void geo_init(const StepArgs& a) {
    const int i = threadIdx.x;
    if (i < 5) {
        const int H = a.md.hidden_size, nq = a.md.num_heads, nkv = a.md.num_kv_heads, hd = a.md.head_dim;
        const int In = a.md.intermediate_size, V = a.md.vocab_size;
        const int n = i == 0 ? (nq + 2 * nkv) * hd : i == 1 || i == 3 ? H : i == 2 ? In : V;
        const int k = i == 1 ? nq * hd : i == 3 ? In : H;
        const Mat A = make_mat<Q8>(nullptr, nullptr, n, k, i == 2, a.md.tile_rows[i]);
        const Part p = partition(A, i == 1 ? a.o_grid : (int)gridDim.x);
        uint32_t cm;
        int cs;
        recip24(A.chunks, cm, cs);
        geo_table()[i] = Geo{A.n, A.k, A.tr, A.lpr, A.tiles, A.nb, A.chunks, A.ck,
                             p.f0, p.f1, p.pieces, p.gp, p.ca, p.win, p.busy ? 1 : 0, cm, cs};
    }
}
// Slot i's matrix over the given weights and scales, and this workgroup's
// share (wave-uniform values, kept in SGPRs).
__device__ __forceinline__ Mat geo_mat(int i, const void* w, const void* s) {
    const Geo& g = geo_table()[i];
    Mat m;
    m.w = static_cast<const u32x4*>(w);
    m.s = s;
    m.n = uniform(g.n);
    m.k = uniform(g.k);
    m.tr = uniform(g.tr);
    m.lpr = uniform(g.lpr);
    m.tiles = uniform(g.tiles);
    m.nb = uniform(g.nb);
    m.chunks = uniform(g.chunks);
    m.ck = uniform(g.ck);
    return m;
}
__device__ __forceinline__ Part geo_part(int i) {
    const Geo& g = geo_table()[i];
    Part p;
    p.f0 = uniform(g.f0);
    p.f1 = uniform(g.f1);
    p.pieces = uniform(g.pieces);
    p.gp = uniform(g.gp);
    p.ca = uniform(g.ca);
    p.win = uniform(g.win);
    p.busy = uniform(g.busy) != 0;
    return p;
}

// Accumulates one chunk of the matrix into acc (x from the LDS window).
template <int M, bool Q8>
struct ChunkMath;

template <int M>
struct ChunkMath<M, false> {
    static constexpr int kUnit = 32;
    // Chunk f (nv valid blocks): the lane's 4 blocks and its 4 group scales.
    // Blocks past nv hold code 0 (nibble 8) without a load.
    __device__ __forceinline__ static void load(const Mat& A, int f, int nv, int lane, u32x4 (&w)[kChunkBlocks],
                                                u64& s) {
        const LYK_GLOBAL u32x4* wt = gp(A.w + (size_t)f * (kChunkBlocks * 64) + lane);
#pragma unroll
        for (int j = 0; j < kChunkBlocks; ++j) {
            if (j < nv) w[j] = __builtin_nontemporal_load(wt + j * 64);
            else w[j] = u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
            __builtin_amdgcn_sched_barrier(0);
        }
        s = __builtin_nontemporal_load(gp(static_cast<const u64*>(A.s) + (size_t)f * 64 + lane));
        __builtin_amdgcn_sched_barrier(0);
    }
    // The same from a chunk staged in LDS (stage_chunk's layout).
    __device__ __forceinline__ static void load_lds(const unsigned char* slot, int nv, int lane,
                                                    u32x4 (&w)[kChunkBlocks], u64& s) {
#pragma unroll
        for (int j = 0; j < kChunkBlocks; ++j)
            w[j] = j < nv ? reinterpret_cast<const u32x4*>(slot + j * 1024)[lane]
                          : u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
        s = reinterpret_cast<const u64*>(slot + kChunkBlocks * 1024)[lane];
    }
    // One group (32 codes) against x[32]. A code's nibble c = q + 8 becomes
    // the fp16 subnormal c * 2^-24 by masking alone (low nibbles; high ones
    // give 16c * 2^-24), exact, and so are its products with fp16 x in the
    // fp32 dot2 chains. The offsets (8 per code) are removed afterwards from
    // the group sum, rescaled by 2^24: the correction is 8 * (sum of the
    // group's x), computed once per x window. The offset is small next to
    // the codes, so the chains lose no precision to cancellation. Four
    // independent dot2 chains.
    // (Unfolded, for wide batches: the offsets come off each code first,
    // exactly, in the subnormal range.)
    __device__ __forceinline__ static float group(const u32x4& w, const u32x4* xv, float corr) {
        constexpr bool fold = M <= kFoldRows;
        const half2_t off_a = as_half2(0x80088008u);   // -8 * 2^-24, twice
        const half2_t off_b = as_half2(0x80808080u);   // -128 * 2^-24, twice
        const uint32_t u4[4] = {w.x, w.y, w.z, w.w};
        float a0 = 0.0f, a1 = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t u = u4[d], t = u >> 8;
            const u32x4 xx = xv[d];
            half2_t ha = as_half2(u & 0x000F000Fu), hb = as_half2(u & 0x00F000F0u);
            half2_t hc = as_half2(t & 0x000F000Fu), hd = as_half2(t & 0x00F000F0u);
            if constexpr (!fold) {
                ha += off_a;
                hb += off_b;
                hc += off_a;
                hd += off_b;
            }
            a0 = dot2(ha, as_half2(xx.x), a0);
            b0 = dot2(hb, as_half2(xx.y), b0);
            a1 = dot2(hc, as_half2(xx.z), a1);
            b1 = dot2(hd, as_half2(xx.w), b1);
        }
        const float g = (b0 + b1) * 0.0625f + (a0 + a1);   // sum of c * x, times 2^-24
        if constexpr (fold) return fmaf(g, 16777216.0f, -corr);
        return g * 16777216.0f;
    }
    // xc: the lane's x of block 0 of the chunk; block j is xstep halves on.
    // cc: the lane's correction of block 0; block j is lpr entries on.
    __device__ __forceinline__ static void compute(const u32x4 (&w)[kChunkBlocks], u64 s, const uint16_t* xc,
                                                   const float* cc, int xstride, int cstride, int xstep, int lpr,
                                                   float (&acc)[M]) {
        const uint32_t sw[2] = {(uint32_t)s, (uint32_t)(s >> 32)};
        // blocks in pairs: two groups' math interleaves
#pragma unroll
        for (int j = 0; j < kChunkBlocks; j += 2) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint16_t* xm = xc + (size_t)m * xstride + j * xstep;
                const float* cm = cc + (size_t)m * cstride + j * lpr;
                const float g0 = group(w[j], reinterpret_cast<const u32x4*>(xm), cm[0]);
                const float g1 = group(w[j + 1], reinterpret_cast<const u32x4*>(xm + xstep), cm[lpr]);
                acc[m] = fmaf(g0, h2f(uint16_t(sw[j >> 1])), acc[m]);
                acc[m] = fmaf(g1, h2f(uint16_t(sw[j >> 1] >> 16)), acc[m]);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

template <int M>
struct ChunkMath<M, true> {
    static constexpr int kUnit = 16;
    // Chunk f (nv valid blocks): the lane's 4 blocks; past nv, code 0 (128).
    __device__ __forceinline__ static void load(const Mat& A, int f, int nv, int lane, u32x4 (&w)[kChunkBlocks],
                                                u64& s) {
        const LYK_GLOBAL u32x4* wt = gp(A.w + (size_t)f * (kChunkBlocks * 64) + lane);
#pragma unroll
        for (int j = 0; j < kChunkBlocks; ++j) {
            if (j < nv) w[j] = __builtin_nontemporal_load(wt + j * 64);
            else w[j] = u32x4{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
            __builtin_amdgcn_sched_barrier(0);
        }
        (void)s;
    }
    __device__ __forceinline__ static void load_lds(const unsigned char* slot, int nv, int lane,
                                                    u32x4 (&w)[kChunkBlocks], u64& s) {
#pragma unroll
        for (int j = 0; j < kChunkBlocks; ++j)
            w[j] = j < nv ? reinterpret_cast<const u32x4*>(slot + j * 1024)[lane]
                          : u32x4{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
        (void)s;
    }
    // One block (16 codes) against x[16]: a byte c = q + 128 becomes the
    // fp16 subnormal c * 2^-24 (one v_perm per pair, zero high bytes), exact;
    // the block's correction (128 * sum of its x) removes the offset from the
    // sum rescaled by 2^24.
    // (Unfolded, for wide batches: the offset comes off each code first.)
    __device__ __forceinline__ static float block(const u32x4& w, const u32x4* xv, float corr) {
        constexpr bool fold = M <= kFoldRows;
        const half2_t off = as_half2(0x80808080u);   // -128 * 2^-24, twice
        const uint32_t u4[4] = {w.x, w.y, w.z, w.w};
        const u32x4 x0 = xv[0], x1 = xv[1];
        const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            half2_t lo = as_half2(__builtin_amdgcn_perm(0u, u4[d], 0x0c010c00u));
            half2_t hi = as_half2(__builtin_amdgcn_perm(0u, u4[d], 0x0c030c02u));
            if constexpr (!fold) {
                lo += off;
                hi += off;
            }
            a0 = dot2(lo, as_half2(xw[2 * d]), a0);
            a1 = dot2(hi, as_half2(xw[2 * d + 1]), a1);
        }
        if constexpr (fold) return fmaf(a0 + a1, 16777216.0f, -corr);
        return (a0 + a1) * 16777216.0f;
    }
    __device__ __forceinline__ static void compute(const u32x4 (&w)[kChunkBlocks], u64, const uint16_t* xc,
                                                   const float* cc, int xstride, int cstride, int xstep, int lpr,
                                                   float (&acc)[M]) {
#pragma unroll
        for (int j = 0; j < kChunkBlocks; j += 2) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint16_t* xm = xc + (size_t)m * xstride + j * xstep;
                const float* cm = cc + (size_t)m * cstride + j * lpr;
                const float g0 = block(w[j], reinterpret_cast<const u32x4*>(xm), cm[0]);
                const float g1 = block(w[j + 1], reinterpret_cast<const u32x4*>(xm + xstep), cm[lpr]);
                acc[m] += g0;
                acc[m] += g1;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

// ------------------------------------------------------------ gate/up staging

// LDS bytes of one staged chunk: its blocks lane-major (64 lanes x 16 B
// each), then for int4 the lanes' group scales (64 x 8 B).
template <bool Q8>
constexpr int kSlotBytes = kChunkBlocks * 1024 + (Q8 ? 0 : 512);

// Requests into LDS the first pf_chunks chunks of every wave's share of the
// layer's gate/up matrix (gemv_step's split: the workgroup's range cut evenly
// over its waves), by LDS DMA: no registers are held, and completion counts
// in the issuing wave's vmcnt, so each wave stages the chunks it will itself
// consume. Called once the workgroup's attention work is done: the loads
// stream while the attention and O phases wait on their inputs, which have
// little HBM traffic of their own.
template <bool Q8>
__device__ __forceinline__ void stage_gateup(const StepArgs& a, const lyk_step_layer& Lw) {
    if (a.pf_chunks == 0) return;
    extern __shared__ __align__(16) unsigned char smem[];
    const Mat A = geo_mat(2, Lw.gateup_w, Lw.gateup_s);
    const Part p = geo_part(2);
    if (!p.busy) return;
    const int tid = phase_tid();
    const int lane = tid & 63, wave = uniform(tid >> 6);
    const int len = p.f1 - p.f0;
    const int w0 = p.f0 + len * wave / kWaves, w1 = p.f0 + len * (wave + 1) / kWaves;
    const int n = min(a.pf_chunks, w1 - w0);
    const int tail = A.nb - (A.chunks - 1) * kChunkBlocks;
    unsigned char* base = smem + a.pf_off + wave * a.pf_chunks * kSlotBytes<Q8>;
    for (int i = 0; i < n; ++i) {
        const int f = w0 + i;
        const int nv = tail == kChunkBlocks || (f + 1) % A.chunks ? kChunkBlocks : tail;
        unsigned char* slot = base + i * kSlotBytes<Q8>;
        for (int j = 0; j < nv; ++j)
            __builtin_amdgcn_global_load_lds(gp(A.w + ((size_t)f * kChunkBlocks + j) * 64 + lane),
                                             (LYK_LOCAL void*)(slot + j * 1024), 16, 0, 0);
        if constexpr (!Q8) {
            if (lane < 32) {
                const u32x4* sv = reinterpret_cast<const u32x4*>(static_cast<const u64*>(A.s) + (size_t)f * 64);
                __builtin_amdgcn_global_load_lds(gp(sv + lane), (LYK_LOCAL void*)(slot + kChunkBlocks * 1024), 16,
                                                 0, 0);
            }
        }
    }
}

// ------------------------------------------------------------ phase inputs

// Inputs are fetched by resumable pollers: attempt() makes one pass over
// the words still missing (one memory round trip) and returns how many
// remain, so a phase can make its first attempt before queueing any weight
// load of its own (a load waits behind every load its CU issued before it).

// The tagged block output d[m*H + i] of this layer for the thread's
// residual elements (i = tid + j*kThreads of each row), added to the
// residual rows by apply().
template <int M>
struct ResidualIn {
    // rows in batches of up to two: word u = (j, row m0 + u % RB) of a batch
    static constexpr int RB = M < 2 ? M : 2, NB = (M + RB - 1) / RB;
    static_assert(kNormPer * 2 <= 32, "residual batch");
    uint32_t want, have[NB];
    float add[M][kNormPer];
    __device__ __forceinline__ void init(int H, int tid) {
        want = 0;
#pragma unroll
        for (int j = 0; j < kNormPer; ++j)
            if (tid + j * kThreads < H) want |= ((1u << RB) - 1) << (j * RB);
#pragma unroll
        for (int q = 0; q < NB; ++q) have[q] = 0;
    }
    __device__ __forceinline__ int attempt(const u64* d, uint32_t tag, int H, int tid) {
        int missing = 0;
#pragma unroll
        for (int q = 0; q < NB; ++q) {
            const int m0 = q * RB;
            const uint32_t wq = m0 + RB <= M ? want : want & 0x55555555u;   // last batch of odd M: one row
            missing += poll_batch<kNormPer * RB, M == 1>(
                wq, have[q], tag,
                [&](int u) {
                    return d + (size_t)min(m0 + u % RB, M - 1) * H + min(tid + (u / RB) * kThreads, H - 1);
                },
                [&](int u, uint32_t v) {
                    if (m0 + u % RB < M) add[m0 + u % RB][u / RB] = bitsf(v);
                });
        }
        return missing;
    }
    __device__ __forceinline__ void apply(float (&h)[M][kNormPer], int H, int tid) const {
#pragma unroll
        for (int j = 0; j < kNormPer; ++j)
            if (tid + j * kThreads < H)
#pragma unroll
                for (int m = 0; m < M; ++m) h[m][j] += add[m][j];
    }
};

// A window of n tagged words per row, src[m] + e for e < n (entries at or
// past `valid` read as 0): the thread's words e = tid + u*kThreads, u <
// kWinWords (the host keeps windows within kThreads * kWinWords words).
constexpr int kWinWords = 8;
template <int M>
struct WindowIn {
    uint32_t want[M], have[M], v[M][kWinWords];
    __device__ __forceinline__ void init(int n, int valid, int tid) {
#pragma unroll
        for (int m = 0; m < M; ++m) {
            want[m] = have[m] = 0;
#pragma unroll
            for (int u = 0; u < kWinWords; ++u) {
                const int e = tid + u * kThreads;
                v[m][u] = 0;
                if (e < n && e < valid) want[m] |= 1u << u;
            }
        }
    }
    template <class Src>
    __device__ __forceinline__ int attempt(Src src, int valid, uint32_t tag, int tid) {
        int missing = 0;
#pragma unroll
        for (int m = 0; m < M; ++m)
            missing += poll_batch<kWinWords, M == 1>(want[m], have[m], tag,
                                             [&](int u) { return src(m) + min(tid + u * kThreads, valid - 1); },
                                             [&](int u, uint32_t x) { v[m][u] = x; });
        return missing;
    }
    template <class Out>
    __device__ __forceinline__ void finish(int n, int tid, Out out) const {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int u = 0; u < kWinWords; ++u)
                if (tid + u * kThreads < n) out(m, tid + u * kThreads, v[m][u]);
    }
};

// The gamma values of this thread's residual elements that fall in the
// workgroup's window, requested before the residual poll so that their
// latency overlaps the wait.
__device__ __forceinline__ void load_gamma(const StepArgs& a, const float* gamma, const Mat& A, const Part& p,
                                           int tid, float (&g)[kNormPer]) {
    const int H = a.md.hidden_size;
    const int lo = p.ca * A.ck, hi = (p.ca + p.win) * A.ck;   // the window's k range
#pragma unroll
    for (int j = 0; j < kNormPer; ++j) {
        const int i = tid + j * kThreads;
        g[j] = p.busy && i < H && i >= lo && i < hi ? ld(gamma + i) : 0.0f;
    }
}

// x window <- fp16 RMSNorm(h) * gamma over the chunks of the window, zero
// beyond k (the reference order: h * (1/sqrt(mean(h^2) + eps)) * gamma).
template <int M, bool Q8>
__device__ __forceinline__ void norm_window(const StepArgs& a, const float (&h)[M][kNormPer],
                                            const float (&gv)[kNormPer], const Mat& A, const Part& p,
                                            uint16_t* xs, int tid) {
    const int CK = A.ck;
    const int H = a.md.hidden_size;
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < kNormPer; ++j) s = fmaf(h[m][j], h[m][j], s);   // zero past H
        ss[m] = s;
    }
    block_sum_rows<M>(ss, tid);
    float scale[M];
#pragma unroll
    for (int m = 0; m < M; ++m) scale[m] = 1.0f / sqrtf(ss[m] / (float)H + a.md.rms_norm_eps);
    // window slot s holds chunk ca + s, so k index i sits at i - lo
    const int lo = p.ca * CK, hi = (p.ca + p.win) * CK, xstride = p.win * CK;
#pragma unroll
    for (int j = 0; j < kNormPer; ++j) {
        const int i = tid + j * kThreads;
        if (i < H && i >= lo && i < hi) {
            const float g = gv[j];
#pragma unroll
            for (int m = 0; m < M; ++m) xs[(size_t)m * xstride + (i - lo)] = f2h(h[m][j] * scale[m] * g);
        }
    }
    for (int i = (H > lo ? H : lo) + tid; i < hi; i += kThreads)
#pragma unroll
        for (int m = 0; m < M; ++m) xs[(size_t)m * xstride + (i - lo)] = 0;
}

struct Best {
    float v;
    int i;
};
__device__ __forceinline__ Best better(Best x, Best y) {
    if (y.v > x.v || (y.v == x.v && y.i < x.i)) return y;
    return x;
}
// The wave's best (largest value, then smallest index) in every lane, without
// LDS: DPP rotations within each 16-lane row, then the permlane swaps. better
// selects from a total order, so the combination order does not matter.
template <int CTRL>
__device__ __forceinline__ Best dpp_better(Best b) {
    return better(b, Best{__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, b.v), CTRL,
                                                                                 0xf, 0xf, false)),
                          __builtin_amdgcn_update_dpp(0, b.i, CTRL, 0xf, 0xf, false)});
}
template <bool Row32>
__device__ __forceinline__ Best pair_better(Best b) {
    float xv, yv, xi, yi;
    pair_of<Row32>(b.v, xv, yv);
    pair_of<Row32>(__builtin_bit_cast(float, b.i), xi, yi);
    return better(Best{xv, __builtin_bit_cast(int, xi)}, Best{yv, __builtin_bit_cast(int, yi)});
}
__device__ __forceinline__ Best wave_best(Best b) {
    b = dpp_better<0x128>(b);   // row_ror:8
    b = dpp_better<0x124>(b);   // row_ror:4
    b = dpp_better<0x122>(b);   // row_ror:2
    b = dpp_better<0x121>(b);   // row_ror:1
    return pair_better<true>(pair_better<false>(b));
}

enum Kind { kQkv = 0, kAttn = 1, kOut = 2, kGateUp = 3, kDown = 4, kHead = 5 };

// Runs the workgroup's share of one GEMV phase of the given kind. The wave's
// first two chunks are requested first; then the phase's inputs are polled
// into the x window (every workgroup takes part in the residual updates, so
// idle ones keep theirs current); then the stream. A tile cut into K pieces
// is finished by piece 0's workgroup, which adds the others' tagged partials
// in piece order. Returns false when the grid is aborting.
template <int M, bool Q8>
__device__ __forceinline__ bool gemv_step(const StepArgs& a, int ph, int kind, int l, const lyk_step_layer& Lw,
                                          float (&h)[M][kNormPer], uint32_t tag0) {
    const int tid = phase_tid();
    using CM = ChunkMath<M, Q8>;
    extern __shared__ __align__(16) unsigned char smem[];
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
    float* red = reinterpret_cast<float*>(smem);  // aliases xs after the stream
    const int H = a.md.hidden_size, nq = a.md.num_heads, nkv = a.md.num_kv_heads, hd = a.md.head_dim;
    const int In = a.md.intermediate_size, L = a.md.num_layers, V = a.md.vocab_size;
    const int rows = (nq + 2 * nkv) * hd;
    const uint32_t tag = tag0 | (uint32_t)l;   // l == L for the LM head
    const void* wp;
    const void* sp;
    switch (kind) {
        case kQkv: wp = Lw.qkv_w; sp = Lw.qkv_s; break;
        case kOut: wp = Lw.o_w; sp = Lw.o_s; break;
        case kGateUp: wp = Lw.gateup_w; sp = Lw.gateup_s; break;
        case kDown: wp = Lw.down_w; sp = Lw.down_s; break;
        default: wp = a.md.lm_head_w; sp = a.md.lm_head_s; break;
    }
    // matrices of a phase kind share a slot: qkv 0, o 1, gate/up 2, down 3, head 4
    const int slot = kind == kQkv ? 0 : kind - 1;
    const Mat A = geo_mat(slot, wp, sp);
    const int CK = A.ck;
    mark(a, ph, 0);
    const Part p = geo_part(slot);
    // tile of a chunk index: x / A.chunks by the phase's reciprocal (chunk
    // indices stay far below 2^24)
    const uint32_t cmag = uniform((int)geo_table()[slot].cmag);
    const int csh = uniform(geo_table()[slot].csh);
    auto tile_of = [&](int f) { return div24(f, cmag, csh); };
    const int b = blockIdx.x;
    const int lane = tid & 63, wave = uniform(tid >> 6);
    const int len = p.f1 - p.f0;
    const int w0 = p.f0 + len * wave / kWaves, w1 = p.f0 + len * (wave + 1) / kWaves;
    // valid blocks of chunk f: all but in a tile's last chunk when the tile's
    // blocks do not fill it
    const int tail = A.nb - (A.chunks - 1) * kChunkBlocks;
    auto nv_of = [&](int f) { return tail == kChunkBlocks || f + 1 != (tile_of(f) + 1) * A.chunks ? kChunkBlocks : tail; };
    // gate/up: the wave's chunks [w0, w0 + npf) wait in LDS (stage_gateup);
    // the register pipeline starts after them
    const int npf = kind == kGateUp ? min(a.pf_chunks, w1 - w0) : 0;
    const int g0 = w0 + npf;
    const unsigned char* pfb = smem + a.pf_off + wave * a.pf_chunks * kSlotBytes<Q8>;
    if (npf > 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // ---- inputs: the residual's block output (normed phases) or the
    // polled window (o, down), fetched by resumable pollers
    const bool normed = kind == kQkv || kind == kGateUp || kind == kHead;
    const u64* d = nullptr;   // the block output the residual adds (normed phases)
    uint32_t dtag = 0;
    const float* gamma = a.md.final_norm;
    if (kind == kQkv) {
        if (l > 0) {
            d = a.d_mlp + (size_t)(l - 1) * kMaxRows * H;
            dtag = tag - 1;
        }
        gamma = Lw.input_norm;
    } else if (kind == kGateUp) {
        d = a.d_attn + (size_t)l * kMaxRows * H;
        dtag = tag;
        gamma = Lw.post_norm;
    } else if (kind == kHead) {
        d = a.d_mlp + (size_t)(L - 1) * kMaxRows * H;
        dtag = tag - 1;
    }
    float gv[kNormPer];
    if (normed) load_gamma(a, gamma, A, p, tid, gv);
    // o: fp32 attention outputs [M][nq*hd]; down: SiLU(gate) * up fp16 pairs
    // [M][In/2]; the window of chunks [ca, ca + win)
    const int wlen = kind == kDown ? CK / 2 : CK;
    const int wn = p.win * wlen, w0e = p.ca * wlen;
    const int wtot = kind == kDown ? In / 2 : nq * hd;
    const u64* wsrc = kind == kDown ? a.act : a.attn_out;
    auto wrow = [&](int m) { return wsrc + (size_t)m * wtot + w0e; };
    ResidualIn<M> rin;
    WindowIn<M> win;
    auto attempt = [&]() -> int {
        if (normed) return d ? rin.attempt(d, dtag, H, tid) : 0;
        return p.busy ? win.attempt(wrow, wtot - w0e, tag, tid) : 0;
    };
    if (normed) {
        if (d) rin.init(H, tid);
    } else if (p.busy) {
        win.init(wn, wtot - w0e, tid);
    }
    // The wave's first two weight chunks are requested before the inputs
    // are polled (they stream while it waits); the stream then keeps two
    // chunks in flight per wave. (Polling first and requesting only when an
    // input is missing was measured slower: the late workgroups then wait
    // out the chunks' latency after their inputs. Four chunks in flight was
    // slower too: 32 MB of requests queued across the grid delay every poll
    // and partial-sum read behind them, and the workgroups that finish a
    // phase last wait longest.)
    u32x4 wa[kChunkBlocks], wb[kChunkBlocks];
    u64 sa = 0, sb = 0;
    if (g0 < w1) CM::load(A, g0, nv_of(g0), lane, wa, sa);
    if (g0 + 1 < w1) CM::load(A, g0 + 1, nv_of(g0 + 1), lane, wb, sb);
    const bool ok = spin(a, attempt);
    // one decision for the workgroup before any code with barriers
    if (block_any<0>(!ok)) return false;
    if (normed) {
        if (d) rin.apply(h, H, tid);
        if (p.busy) norm_window<M, Q8>(a, h, gv, A, p, xs, tid);
    } else if (p.busy) {
        if (kind == kDown)
            win.finish(wn, tid, [&](int m, int e, uint32_t v) { reinterpret_cast<uint32_t*>(xs)[(size_t)m * wn + e] = v; });
        else
            win.finish(wn, tid, [&](int m, int e, uint32_t v) { xs[(size_t)m * wn + e] = f2h(bitsf(v)); });
    }
    __syncthreads();   // the x window is complete before any wave reads it
    mark(a, ph, 1);
    if (!p.busy) {
        mark(a, ph, 2);
        mark(a, ph, 3);
        return true;
    }

    // ---- offset corrections of the window's units (after the x window):
    // int4 group 8 * (sum of its 32 x); int8 block 128 * (sum of its 16 x)
    const int xstride = p.win * CK;
    const int cstride = xstride / CM::kUnit;
    float* corr = reinterpret_cast<float*>(smem + ((size_t)M * xstride * 2 + 15) / 16 * 16);
    for (int i = tid; i < (M <= kFoldRows ? M * cstride : 0); i += kThreads) {
        const uint16_t* xu = xs + (size_t)i * CM::kUnit;   // rows are contiguous: unit i of the window
        float sum = 0.0f;
#pragma unroll
        for (int e = 0; e < CM::kUnit; ++e) sum += h2f(xu[e]);
        corr[i] = (Q8 ? 128.0f : 8.0f) * sum;
    }
    if constexpr (M <= kFoldRows) __syncthreads();

    // ---- stream
    // this lane's unit within a block, and the distance between blocks, in x
    const int usub = lane >> (A.tr == 16 ? 4 : A.tr == 32 ? 5 : 6);   // tr: 16, 32 or 64
    const int xsub = usub * CM::kUnit, xstep = A.lpr * CM::kUnit;
    float accq[kPieces][M];
#pragma unroll
    for (int q = 0; q < kPieces; ++q)
#pragma unroll
        for (int m = 0; m < M; ++m) accq[q][m] = 0.0f;

    if (w0 < w1) {
        int f = w0;
        int t = tile_of(f);
        int c = f - t * A.chunks;
        int q = 0;
        float acc[M];
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] = 0.0f;
        // int8 per-row scale of the current tile
        float srow = 1.0f;
        if constexpr (Q8) srow = h2f(ld(static_cast<const uint16_t*>(A.s) + (size_t)t * 64 + lane));
        const int cend = p.pieces == 1 ? A.chunks : p.f1 - t * A.chunks;
        // One chunk: math on the buffer, then (register chunks) request the
        // chunk two ahead into it; a tile's sums go to its piece slot when
        // the tile ends.
        auto step = [&](u32x4 (&wbuf)[kChunkBlocks], u64& sbuf, bool refill) -> bool {
            CM::compute(wbuf, sbuf, xs + (size_t)(c - p.ca) * CK + xsub,
                        corr + (size_t)(c - p.ca) * (CK / CM::kUnit) + usub, xstride, cstride, xstep, A.lpr, acc);
            const bool end = f + 1 == w1;
            if (c + 1 == cend || c + 1 == A.chunks || end) {
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
            if (refill && f + 2 < w1) {
                // chunk f + 2's place in its tile, from c (no division)
                int c2 = c + 2;
                while (c2 >= A.chunks) c2 -= A.chunks;
                CM::load(A, f + 2, tail == kChunkBlocks || c2 + 1 < A.chunks ? kChunkBlocks : tail, lane, wbuf, sbuf);
            }
            __builtin_amdgcn_sched_barrier(0);
            ++f;
            c = c + 1 == A.chunks ? 0 : c + 1;
            return false;
        };
        bool done = false;
        for (int i = 0; i < npf && !done; ++i) {
            u32x4 wl[kChunkBlocks];
            u64 sl = 0;
            CM::load_lds(pfb + i * kSlotBytes<Q8>, tail == kChunkBlocks || c + 1 < A.chunks ? kChunkBlocks : tail,
                         lane, wl, sl);
            done = step(wl, sl, false);
        }
        while (!done) {
            if (step(wa, sa, true)) break;
            if (step(wb, sb, true)) break;
        }
    }
    __syncthreads();  // every wave is done with the x window
    mark(a, ph, 2);
    // the lanes of one row (l, l+tr, ...) add their sums, in a fixed order
#pragma unroll
    for (int q = 0; q < kPieces; ++q)
#pragma unroll
        for (int m = 0; m < M; ++m)
        {
            if (A.tr <= 16) accq[q][m] = pair16_sum(accq[q][m]);
            if (A.tr <= 32) accq[q][m] = pair32_sum(accq[q][m]);
        }
    // each wave's tile sums, and the tiles [first, last] its range touched
    __shared__ int span[kWaves][2];
    {
        const int tf = w0 < w1 ? tile_of(w0) : 0;
        const int tl = w0 < w1 ? tile_of(w1 - 1) : -1;
        if (lane == 0) {
            span[wave][0] = tf;
            span[wave][1] = tl;
        }
#pragma unroll
        for (int q = 0; q < kPieces; ++q)
            if (q <= tl - tf)
#pragma unroll
                for (int m = 0; m < M; ++m) red[((wave * kPieces + q) * M + m) * 64 + lane] = accq[q][m];
    }
    __syncthreads();

    // ---- finish the workgroup's tiles, one wave per tile
    const int tA = tile_of(p.f0), tB = tile_of(p.f1 - 1);   // busy: f1 >= 1
    const bool greedy = a.io.mode == LYK_STEP_GREEDY;
    // a region per GEMV kind: the kinds of one layer share tags
    u64* dpart = a.dpart + (size_t)(kind == kQkv ? 0 : kind - 1) * a.dpart_stride;
    bool good = true;
    for (int t = tA + wave; t <= tB; t += kWaves) {
        float v[M];
#pragma unroll
        for (int m = 0; m < M; ++m) v[m] = 0.0f;
        // every wave's slot read first (independent LDS reads, issued
        // together), then the in-range ones added in wave order
        float x[kWaves][M];
        bool in[kWaves];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const int tf = span[w][0], tl = span[w][1];
            in[w] = t >= tf && t <= tl;
            const int q = min(max(t - tf, 0), kPieces - 1);
#pragma unroll
            for (int m = 0; m < M; ++m) x[w][m] = red[((w * kPieces + q) * M + m) * 64 + lane];
        }
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
            if (in[w])
#pragma unroll
                for (int m = 0; m < M; ++m) v[m] += x[w][m];
        if (p.pieces > 1) {
            const int np = p.pieces, s = b % np;
            if (s > 0) {
#pragma unroll
                for (int m = 0; m < M; ++m)
                    put(dpart + (((size_t)t * np + s) * M + m) * 64 + lane, fbits(v[m]), tag);
                continue;
            }
            // rows in batches of up to two; word u of a batch: piece
            // 1 + u / RB, row m0 + u % RB
            constexpr int RB = M < 2 ? M : 2, NB = (M + RB - 1) / RB;
            float got[kMaxPieces][M];
            uint32_t have[NB];
#pragma unroll
            for (int q = 0; q < NB; ++q) have[q] = 0;
            const u64* part = dpart + ((size_t)t * np + 1) * M * 64 + lane;
            auto pending = [&]() {
                int missing = 0;
#pragma unroll
                for (int q = 0; q < NB; ++q) {
                    const int m0 = q * RB, rb = m0 + RB <= M ? RB : M - m0;
                    uint32_t want = 0;
                    for (int s2 = 1; s2 < np; ++s2) want |= ((1u << rb) - 1) << ((s2 - 1) * RB);
                    missing += poll_batch<(kMaxPieces - 1) * RB, M == 1>(
                        want, have[q], tag,
                        [&](int u) {
                            return part + ((size_t)min(u / RB, np - 2) * M + min(m0 + u % RB, M - 1)) * 64;
                        },
                        [&](int u, uint32_t x) {
                            if (m0 + u % RB < M) got[1 + u / RB][m0 + u % RB] = bitsf(x);
                        });
                }
                return missing;
            };
            if (!spin(a, pending)) {
                good = false;
                continue;
            }
#pragma unroll
            for (int s2 = 1; s2 < kMaxPieces; ++s2)
                if (s2 < np)
#pragma unroll
                    for (int m = 0; m < M; ++m) v[m] += got[s2][m];
        }
        // tile row `lane` (lanes below tr hold the rows' sums)
        const int r = t * A.tr + lane;
        const bool rv = lane < A.tr;
        switch (kind) {
            case kQkv:
                if (rv && r < rows)
#pragma unroll
                    for (int m = 0; m < M; ++m) put(a.qkv + (size_t)m * rows + r, fbits(v[m]), tag);
                break;
            case kOut:
            case kDown: {
                u64* dst = (kind == kOut ? a.d_attn : a.d_mlp) + (size_t)l * kMaxRows * H;
                if (rv && r < H)
#pragma unroll
                    for (int m = 0; m < M; ++m) put(dst + (size_t)m * H + r, fbits(v[m]), tag);
                break;
            }
            case kGateUp: {
                // lanes 0..tr/2-1 hold gate rows t*tr/2.., lanes tr/2..tr-1
                // the up rows; pairs of neighbouring rows go out as one word
                const int half = A.tr / 2;
                const int j = t * half + lane;
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    // lane + half's value (the up row) and lane + 1's act, in
                    // VGPRs: permlane swaps across rows or halves, DPP within
                    // a row (only lanes below half use them)
                    float up, own;
                    if (A.tr == 64) pair_of<true>(v[m], own, up);
                    else if (A.tr == 32) pair_of<false>(v[m], own, up);
                    else up = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v[m]),
                                                                                     0x128, 0xf, 0xf, false));   // row_ror:8
                    const float g = v[m];
                    const uint32_t act = f2h(g / (1.0f + expf(-g)) * up);
                    const uint32_t next = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)act, 0x101, 0xf, 0xf, false);   // row_shl:1
                    if (lane < half && (lane & 1) == 0 && j < In)
                        put(a.act + (size_t)m * (In / 2) + j / 2, act | (next << 16), tag);
                }
                break;
            }
            default: {
                // LM head: logits, and each tile's greedy candidate (first
                // index of the maximum, NaN never wins) and non-finite count
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const bool live = rv && r < V;
                    if (live) st(a.io.logits + (size_t)m * a.io.ld_logits + r, v[m]);
                    if (!greedy) continue;
                    float x = v[m];
                    int bad = 0;
                    if (live && !isfinite(x)) {
                        bad = 1;
                        if (isnan(x)) x = -INFINITY;
                    }
                    Best bst = live ? Best{x, r} : Best{-INFINITY, 0x7fffffff};
                    bst = wave_best(bst);
                    bad = (int)wave_total((float)bad);
                    if (lane == 0) {
                        u64* w = a.best + ((size_t)m * A.tiles + t) * 3;
                        put(w, fbits(bst.v), tag);
                        put(w + 1, (uint32_t)bst.i, tag);
                        put(w + 2, (uint32_t)bad, tag);
                    }
                }
                break;
            }
        }
    }
    if (block_any<1>(!good)) return false;
    mark(a, ph, 3);
    return true;
}

// ------------------------------------------------------------ attention

constexpr int kTileT = 16;                       // tokens per MFMA tile
constexpr int kChunkT = 256;                     // tokens per softmax chunk (4 per lane)
constexpr int kChunkTiles = kChunkT / kTileT;
constexpr int kKTiles = kChunkTiles / kWaves;    // q.k tiles per wave per chunk

// Context split of a row: equal runs of whole tiles, at least split_tokens
// long, at most max_splits of them; a row's split depends only on its own
// context length.
__device__ __forceinline__ int split_size(int ctx, int split_tokens, int max_splits) {
    int t = (ctx + max_splits - 1) / max_splits;
    t = (t + kTileT - 1) / kTileT * kTileT;
    return t > split_tokens ? t : split_tokens;
}

// Attention units are (row, kv head, context split); the G <= 16 query heads
// of a kv head share every K/V element a unit loads, and both products run
// on the matrix cores:
//   * q.k: S^T[t][h] = K[t][:] . q[h][:] with v_mfma_f32_16x16x32_f16, A = a
//     16-token K tile (each lane loads 16 bytes of one K row straight from
//     the paged cache), B = the rotated queries split into fp16 high and low
//     parts (two MFMAs), so the scores carry fp32 query precision. The result
//     leaves lane l with head l%16 and tokens 4*(l/16)..+3 of the tile.
//   * p.v: O[h][d] += P[h][t] V[t][d] with v_mfma_f32_16x16x16_f16; wave w
//     owns head dims 16w..16w+15 over all of the unit's tokens. The V cache
//     is stored transposed per block ([d][slot]), so the B operand, 4
//     consecutive tokens of one dim, is one 8-byte load. P (split hi/lo like
//     q) is read from LDS in exactly the layout q.k left it in.
// Tokens run in chunks of up to 256: q.k of the chunk (tiles spread over the
// waves) -> scores in LDS -> chunk max per head -> weights exp(s - max) and
// their sum (one wave per head) -> p.v, the accumulator rescaled when the
// running max grows. Each unit's K and V registers for the first chunk are
// requested before it polls its inputs (the raw q, k, v sums of the QKV
// phase, to which it adds the bias and applies RoPE); the unit holding the
// current position appends its K row and V column to the cache and uses
// them from LDS. With several splits, every unit writes its (max, sum,
// unnormalised output) as tagged words; once a workgroup has computed all of
// its units, each unit merges a 1/splits slice of its kv head's outputs over
// the splits, in split order (no unit waits for a unit its own workgroup has
// yet to compute).
template <int M, int HD>
__device__ __forceinline__ bool attention_phase(const StepArgs& a, int ph, const lyk_step_layer& Lw, uint32_t tag) {
    constexpr int KS = (HD + 31) / 32;   // 32-dim steps of q.k
    constexpr int DB = (HD + 15) / 16;   // 16-dim blocks of p.v, one per wave
    constexpr int QS = KS * 32 + 8;      // LDS row of q (halves), padded against bank conflicts
    constexpr int SS = kChunkT + 4;      // LDS row of scores (floats)
    constexpr int half = HD / 2;
    static_assert(DB <= kWaves && (HD % 8 == 0 || HD == 4), "head dim");
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float m_s[16], l_s[16], al_s[16], wmax[kWaves][16];
    const int tid = phase_tid();
    mark(a, ph, 0);
    const int nq = a.md.num_heads, nkv = a.md.num_kv_heads;
    const int G = nq / nkv, bt = a.md.block_tokens;
    const int bt_log = (bt & (bt - 1)) == 0 ? __builtin_ctz(bt) : -1;   // block lookups by shift
    const int lane = tid & 63, wave = tid >> 6;
    const int col = lane & 15, quad = lane >> 4;   // MFMA column / row quad of this lane
    const float scale = 1.0f / sqrtf((float)HD);
    const int GH = G * HD;
    uint16_t* qh = reinterpret_cast<uint16_t*>(smem);    // [16][QS] rotated q, fp16 high part
    uint16_t* ql = qh + 16 * QS;                          // [16][QS] low part
    uint16_t* wh = ql + 16 * QS;                          // [G][kChunkT] softmax weights, high
    uint16_t* wl = wh + G * kChunkT;                      // low
    uint16_t* kcur = wl + G * kChunkT;                    // [KS*32] current key (rotated), fp16
    uint16_t* vcur = kcur + KS * 32;                      // [KS*32] current value, fp16
    float* k_f = reinterpret_cast<float*>(vcur + KS * 32);  // [HD] current key, fp32
    float* sc = k_f + (HD + 3) / 4 * 4;                   // [G][SS] chunk scores / raw q / merge
    const int kq = nq * HD, rows = (nq + 2 * nkv) * HD;

    int S[M], T[M], ctxs[M], units = 0;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        ctxs[m] = ld(a.io.positions + m) + 1;
        T[m] = split_size(ctxs[m], a.attn_split_tokens, a.attn_max_splits);
        S[m] = (ctxs[m] + T[m] - 1) / T[m];
        units += nkv * S[m];
    }
    auto unit_of = [&](int u, int& m, int& g, int& s, int& Sm, int& Tm, int& ctx) {
        int r = u;
        m = 0;
        Sm = S[0];
        Tm = T[0];
        ctx = ctxs[0];
#pragma unroll
        for (int mm = 1; mm < M; ++mm)
            if (m == mm - 1 && r >= nkv * Sm) {
                r -= nkv * Sm;
                m = mm;
                Sm = S[mm];
                Tm = T[mm];
                ctx = ctxs[mm];
            }
        g = sdiv(r, Sm);
        s = r - g * Sm;
    };
    // units go to the workgroups from the top of the grid down: the QKV
    // tiles fill the grid from the bottom, so the first units land on
    // workgroups with no QKV work, which reach this phase early and have
    // their K/V loads in flight when q arrives
    const int rb = (int)gridDim.x - 1 - (int)blockIdx.x;
    bool ok = true;
    for (int u = rb; u < units; u += gridDim.x) {
        int m, g, s, Sm, Tm, ctx;
        unit_of(u, m, g, s, Sm, Tm, ctx);
        const int pos = ctx - 1;
        const int t0 = s * Tm, t1 = min(ctx, t0 + Tm);
        const bool last = s == Sm - 1;   // holds the current position
        const int* tab = a.io.block_tables + (size_t)m * a.io.table_stride;
        const size_t head_stride = (size_t)bt * HD;   // one kv head of a block
        const size_t blk_stride = (size_t)nkv * head_stride;
        const uint16_t* kc = Lw.k_cache + (size_t)g * head_stride;
        const uint16_t* vc = Lw.v_cache + (size_t)g * head_stride;
        const int dv = wave * kTileT + col;   // this lane's dim in p.v

        // K rows of this wave's q.k tiles and V runs of its dims, for the
        // chunk at c0 (zero past the split and at the current position). A
        // tile never straddles a block (block_tokens is a multiple of 16):
        // one block lookup per tile, with wave-uniform arithmetic.
        u32x4 kr[kKTiles][KS];
        u64 vr[kChunkTiles];
        auto tile_block = [&](int tt, int& slot) -> size_t {   // tt: first token of a tile
            const int tb = bt_log >= 0 ? uniform(tt) >> bt_log : uniform(tt) / bt;
            slot = uniform(tt) - tb * bt;
            return (size_t)ld(tab + tb) * blk_stride;
        };
        auto load_k = [&](int c0) {
#pragma unroll
            for (int i = 0; i < kKTiles; ++i) {
                const int tt = c0 + (wave + i * kWaves) * kTileT, t = tt + col;
                const bool live = t < t1 && t != pos;
                size_t row = 0;
                if (tt < t1) {
                    int slot;
                    row = tile_block(tt, slot) + (size_t)(slot + col) * HD;
                }
#pragma unroll
                for (int ks = 0; ks < KS; ++ks) {
                    const int d = ks * 32 + quad * 8;
                    kr[i][ks] = u32x4{0u, 0u, 0u, 0u};
                    if (live && d < HD) {
                        if constexpr (HD % 8 == 0) {
                            kr[i][ks] = ld(reinterpret_cast<const u32x4*>(kc + row + d));
                        } else {
                            const u64 w = ld(reinterpret_cast<const u64*>(kc + row + d));
                            kr[i][ks].x = (uint32_t)w;
                            kr[i][ks].y = (uint32_t)(w >> 32);
                        }
                    }
                }
            }
        };
        auto load_v = [&](int c0) {
#pragma unroll
            for (int j = 0; j < kChunkTiles; ++j) {
                const int tt = c0 + j * kTileT, r0 = tt + quad * 4;   // r0: first of the lane's 4 tokens
                vr[j] = 0;
                if (wave < DB && tt < t1) {
                    int slot;
                    const size_t bo = tile_block(tt, slot);
                    if (dv < HD && r0 < t1) {
                        u64 w = ld(reinterpret_cast<const u64*>(vc + bo + (size_t)dv * bt + slot + quad * 4));
                        const int valid = t1 - r0;
                        if (valid < 4) w &= (1ull << (16 * valid)) - 1;
                        vr[j] = w;
                    }
                }
            }
        };
        load_k(t0);
        load_v(t0);
        // zero what the MFMA operands read but RoPE does not write: q rows of
        // absent heads, dims past the head dim
        for (int e = tid; e < 16 * QS; e += kThreads) {
            const int h = e / QS, d = e % QS;
            if (h >= G || d >= HD) qh[e] = ql[e] = 0;
        }
        for (int e = tid; e < 2 * KS * 32; e += kThreads)
            if (e % (KS * 32) >= HD) kcur[e] = 0;

        // this thread's RoPE factors (its dim i = tid % (HD/2) in every
        // pass, HD/2 dividing the block), requested before the inputs
        const float rc = ld(a.md.rope_cos + (size_t)pos * half + tid % half);
        const float rs = ld(a.md.rope_sin + (size_t)pos * half + tid % half);
        // raw q (and current k, v) sums + bias, polled
        float* q_f = sc;   // [G][HD]
        const u64* src = a.qkv + (size_t)m * rows;
        {
            const int nw = GH + (last ? 2 * HD : 0);
            for (int e0 = tid; e0 < nw; e0 += kThreads * 4) {
                uint32_t v[4];
                int idx[4];
                float bias[4];
#pragma unroll
                for (int u2 = 0; u2 < 4; ++u2) {
                    const int e = e0 + u2 * kThreads;
                    idx[u2] = e < GH ? g * GH + e
                                     : (e < GH + HD ? kq + g * HD + (e - GH) : kq + nkv * HD + g * HD + (e - GH - HD));
                    bias[u2] = e < nw ? ld(Lw.qkv_bias + idx[u2]) : 0.0f;
                }
                uint32_t want = 0, have = 0;
#pragma unroll
                for (int u2 = 0; u2 < 4; ++u2)
                    if (e0 + u2 * kThreads < nw) want |= 1u << u2;
                auto pending = [&]() {
                    return poll_batch<4>(want, have, tag, [&](int u2) { return src + (want >> u2 & 1 ? idx[u2] : idx[0]); },
                                         [&](int u2, uint32_t x) { v[u2] = x; });
                };
                ok = spin(a, pending) && ok;
#pragma unroll
                for (int u2 = 0; u2 < 4; ++u2) {
                    const int e = e0 + u2 * kThreads;
                    if (e >= nw) continue;
                    const float x = bitsf(v[u2]) + bias[u2];
                    if (e < GH) q_f[e] = x;
                    else if (e < GH + HD) k_f[e - GH] = x;
                    else vcur[e - GH - HD] = f2h(x);
                }
            }
        }
        if (block_any<2>(!ok)) return false;
        // RoPE on q (every head, split into fp16 parts) and on the current
        // key, from the host-built cos/sin tables
        {
            static_assert(kThreads % (HD / 2) == 0, "RoPE dims per thread");
            for (int e = tid; e < (G + (last ? 1 : 0)) * half; e += kThreads) {
                const int h = e / half, i = e % half;
                const float* base = h < G ? q_f + h * HD : k_f;
                const float lo = base[i], hi = base[i + half];
                const float rl = rot_lo(lo, hi, rc, rs), rh = rot_hi(lo, hi, rc, rs);
                if (h < G) {
                    split_f16(rl, qh[h * QS + i], ql[h * QS + i]);
                    split_f16(rh, qh[h * QS + i + half], ql[h * QS + i + half]);
                } else {
                    kcur[i] = f2h(rl);
                    kcur[i + half] = f2h(rh);
                }
            }
        }
        if (tid < 16) {
            m_s[tid] = -INFINITY;
            l_s[tid] = 0.0f;
        }
        __syncthreads();
        if (last) {
            // the current row into the cache: K row-major, V transposed
            const int pb = bt_log >= 0 ? pos >> bt_log : pos / bt, ps = pos - pb * bt;
            const int blk = ld(tab + pb);
            const size_t base = (size_t)blk * blk_stride + (size_t)g * head_stride;
            for (int i = tid; i < HD; i += kThreads) {
                store_sc1_u16(Lw.k_cache + base + (size_t)ps * HD + i, kcur[i]);
                store_sc1_u16(Lw.v_cache + base + (size_t)i * bt + ps, vcur[i]);
            }
        }
        if (u == rb) mark(a, ph, 1);

        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};   // O[4*quad + j][dv]
        const int nch = (t1 - t0 + kChunkT - 1) / kChunkT;
        for (int c = 0; c < nch; ++c) {
            const int c0 = t0 + c * kChunkT;
            const int n = min(kChunkT, t1 - c0);
            // q.k of this wave's tiles -> scores; the wave's max per head
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < kKTiles; ++i) {
                const int tl = wave + i * kWaves;
                if (tl * kTileT < n) {
                    const int t = c0 + tl * kTileT + col;   // the K row this lane supplies
                    f32x4 sv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int ks = 0; ks < KS; ++ks) {
                        u32x4 kv = kr[i][ks];
                        if (t == pos) kv = *reinterpret_cast<const u32x4*>(kcur + ks * 32 + quad * 8);
                        const u32x4 qa = *reinterpret_cast<const u32x4*>(qh + col * QS + ks * 32 + quad * 8);
                        const u32x4 qb = *reinterpret_cast<const u32x4*>(ql + col * QS + ks * 32 + quad * 8);
                        const f16x8 kf = __builtin_bit_cast(f16x8, kv);
                        sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, __builtin_bit_cast(f16x8, qa), sv, 0, 0, 0);
                        sv = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, __builtin_bit_cast(f16x8, qb), sv, 0, 0, 0);
                    }
                    // this lane: head col, chunk tokens tl*16 + 4*quad + j
                    const int tt = tl * kTileT + quad * 4;
                    float o[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        o[j] = tt + j < n ? sv[j] * scale : -INFINITY;
                        mx = fmaxf(mx, o[j]);
                    }
                    if (col < G) {
                        float* d = sc + col * SS + tt;
                        d[0] = o[0];
                        d[1] = o[1];
                        d[2] = o[2];
                        d[3] = o[3];
                    }
                }
            }
            mx = pair32_max(pair16_max(mx));
            if (lane < 16) wmax[wave][lane] = mx;
            if (c + 1 < nch) load_k(c0 + kChunkT);   // next chunk, in flight meanwhile
            __syncthreads();
            if (tid < G) {
                float cm = wmax[0][tid];
#pragma unroll
                for (int w = 1; w < kWaves; ++w) cm = fmaxf(cm, wmax[w][tid]);
                const float mold = m_s[tid], mnew = fmaxf(mold, cm);
                al_s[tid] = expf(mold - mnew);   // 0 on the first chunk
                m_s[tid] = mnew;
            }
            __syncthreads();
            // weights of head h (wave h), 4 tokens per lane, and their sum
            for (int h = wave; h < G; h += kWaves) {
                const int tt = lane * 4;
                float p[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (tt < n) {
                    const float mh = m_s[h];
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (tt + j < n) p[j] = expf(sc[h * SS + tt + j] - mh);
                }
                const float sum = wave_total((p[0] + p[1]) + (p[2] + p[3]));
                uint16_t hi[4], lo[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) split_f16(p[j], hi[j], lo[j]);
                uint16_t* dh = wh + h * kChunkT + tt;
                uint16_t* dl = wl + h * kChunkT + tt;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    dh[j] = hi[j];
                    dl[j] = lo[j];
                }
                if (lane == 0) l_s[h] = l_s[h] * al_s[h] + sum;
            }
            __syncthreads();
            // p.v over the chunk's tiles for this wave's dims
            if (wave < DB) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int h = quad * 4 + j;
                    acc[j] *= h < G ? al_s[h] : 0.0f;
                }
                const int ntl = (n + kTileT - 1) / kTileT;
#pragma unroll
                for (int j = 0; j < kChunkTiles; ++j) {
                    if (j < ntl) {
                        u64 vw = vr[j];
                        const int r0 = c0 + j * kTileT + quad * 4;
                        if (pos >= r0 && pos < r0 + 4) {
                            const int sh = 16 * (pos - r0);
                            vw = (vw & ~(0xffffull << sh)) | ((u64)vcur[dv] << sh);
                        }
                        u64 pa = 0, pb = 0;
                        if (col < G) {
                            pa = *reinterpret_cast<const u64*>(wh + col * kChunkT + j * kTileT + quad * 4);
                            pb = *reinterpret_cast<const u64*>(wl + col * kChunkT + j * kTileT + quad * 4);
                        }
                        const f16x4 vf = __builtin_bit_cast(f16x4, vw);
                        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, pa), vf, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, pb), vf, acc, 0, 0, 0);
                    }
                }
                if (c + 1 < nch) load_v(c0 + kChunkT);
            }
            __syncthreads();   // scores and weights are rewritten by the next chunk
        }
        if (u == rb) mark(a, ph, 2);
        const size_t grp = (size_t)m * nkv + g;
        if (wave < DB && dv < HD) {
            u64* out = a.attn_out + (size_t)m * kq + (size_t)g * GH;
            u64* pa = a.attn_acc + (grp * kAttnMaxSplits + s) * (size_t)GH;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int h = quad * 4 + j;
                if (h < G) {
                    if (Sm == 1) put(&out[h * HD + dv], fbits(acc[j] / l_s[h]), tag);
                    else put(&pa[h * HD + dv], fbits(acc[j]), tag);
                }
            }
        }
        if (Sm > 1 && tid < G) {
            u64* ml = a.attn_ml + (grp * kAttnMaxSplits + s) * G * 2;
            put(&ml[2 * tid], fbits(m_s[tid]), tag);
            put(&ml[2 * tid + 1], fbits(l_s[tid]), tag);
        }
        __syncthreads();   // LDS is rewritten by the next unit
    }

    // merge: unit s of a split kv head finishes outputs [s*E, (s+1)*E) of
    // its G*HD: out = sum_s e_s acc_s / sum_s e_s l_s, e_s = exp(m_s - max)
    for (int u = rb; u < units; u += gridDim.x) {
        int m, g, s, Sm, Tm, ctx;
        unit_of(u, m, g, s, Sm, Tm, ctx);
        if (Sm == 1) continue;
        const size_t grp = (size_t)m * nkv + g;
        const int E = sdiv(GH + Sm - 1, Sm), e0 = s * E, ne = max(0, min(GH, e0 + E) - e0);
        float* mlv = sc;                                // [Sm][G][2] max, sum -> weight, sum
        float* vals = sc + kAttnMaxSplits * 16 * 2;     // [ne][Sm]
        __shared__ float lsum[16];
        const int nml = Sm * G * 2, nw = nml + ne * Sm;
        for (int b0 = tid; b0 < nw; b0 += kThreads * 4) {
            uint32_t v[4];
            auto word = [&](int e) -> const u64* {
                if (e < nml) {
                    const int sp = sdiv(e, 2 * G);
                    return a.attn_ml + (grp * kAttnMaxSplits + sp) * G * 2 + (e - sp * 2 * G);
                }
                const int k = e - nml, kq2 = sdiv(k, Sm);
                return a.attn_acc + (grp * kAttnMaxSplits + (k - kq2 * Sm)) * (size_t)GH + e0 + kq2;
            };
            uint32_t want = 0, have = 0;
            const u64* at[4];   // the words' addresses, once for every attempt
#pragma unroll
            for (int u2 = 0; u2 < 4; ++u2) {
                if (b0 + u2 * kThreads < nw) want |= 1u << u2;
                at[u2] = word(min(b0 + u2 * kThreads, nw - 1));
            }
            auto pending = [&]() {
                return poll_batch<4>(want, have, tag, [&](int u2) { return at[u2]; },
                                     [&](int u2, uint32_t x) { v[u2] = x; });
            };
            ok = spin(a, pending) && ok;
#pragma unroll
            for (int u2 = 0; u2 < 4; ++u2) {
                const int e = b0 + u2 * kThreads;
                if (e < nml) mlv[e] = bitsf(v[u2]);
                else if (e < nw) vals[e - nml] = bitsf(v[u2]);
            }
        }
        if (block_any<3>(!ok)) return false;
        // split weights e_s = exp(m_s - max) and the total sum, one wave per
        // head and a lane per split (splits <= 64)
        for (int h = wave; h < G; h += kWaves) {
            const bool live = lane < Sm;
            const float ms = live ? mlv[(lane * G + h) * 2] : -INFINITY;
            const float mx = wave_top(ms);
            const float es = live ? expf(ms - mx) : 0.0f;
            const float L = wave_total(live ? mlv[(lane * G + h) * 2 + 1] * es : 0.0f);
            if (live) mlv[(lane * G + h) * 2] = es;
            if (lane == 0) lsum[h] = L;
        }
        __syncthreads();
        u64* out = a.attn_out + (size_t)m * kq + (size_t)g * GH;
        for (int k = tid; k < ne; k += kThreads) {
            const int h = (e0 + k) / HD;
            // four interleaved partial sums (split sp into sum sp % 4), added
            // in a fixed order; four splits' LDS loads issued together
            float o4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            int sp = 0;
            for (; sp + 4 <= Sm; sp += 4) {
                float v4[4], w4[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    v4[j] = vals[k * Sm + sp + j];
                    w4[j] = mlv[((sp + j) * G + h) * 2];
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) o4[j] += v4[j] * w4[j];
            }
            for (; sp < Sm; ++sp) o4[sp & 3] += vals[k * Sm + sp] * mlv[(sp * G + h) * 2];
            const float o = (o4[0] + o4[1]) + (o4[2] + o4[3]);
            put(&out[e0 + k], fbits(o / lsum[h]), tag);
        }
        __syncthreads();   // LDS is rewritten by the next unit
    }
    mark(a, ph, 3);
    return true;
}

// ------------------------------------------------------------ the kernel

template <int M, bool Q8, int HD>
__global__ __launch_bounds__(kThreads) void decode_step_kernel(const StepArgs* __restrict__ args) {
    const StepArgs& a = *args;
    if (aborted(a)) return;
    const int b = blockIdx.x;
    // tags of this launch: (launches completed + 1) << 8 | layer; every
    // workgroup counts its own launches, so all agree without talking
    const uint32_t seq = load_sc1(a.seq + b);
    const uint32_t tag0 = (seq + 1u) << 8;
    if (a.io.trace && threadIdx.x == 0)
        st(a.io.trace + (size_t)b * (2 + 4 * a.phases), (uint64_t)__builtin_amdgcn_s_memrealtime());
    const int H = a.md.hidden_size, L = a.md.num_layers;

    // the residual stream of every row, whole, in registers
    float h[M][kNormPer];
    {
        const int tid = threadIdx.x;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float* e = a.md.embed + (size_t)load_sc1(a.io.tokens + m) * H;
#pragma unroll
            for (int j = 0; j < kNormPer; ++j) {
                const int i = tid + j * kThreads;
                h[m][j] = i < H ? ld(e + i) : 0.0f;
            }
        }
    }

    geo_init<Q8>(a);
    __syncthreads();   // the phase geometry is in LDS before any phase reads it

    // per layer: QKV, attention, O, gate/up, down; then the LM head
    const int nph = 5 * L + (a.io.mode == LYK_STEP_HIDDEN ? 0 : 1);
    lyk_step_layer Lw = load_layer(a.md.layers);
#pragma nounroll
    for (int ph = 0; ph < nph; ++ph) {
        const int l = ph / 5, kind = ph < 5 * L ? ph % 5 : (int)kHead;
        if (kind == kQkv && l > 0) Lw = load_layer(a.md.layers + l);
        const bool ok = kind == kAttn ? attention_phase<M, HD>(a, ph, Lw, tag0 | (uint32_t)l)
                                      : gemv_step<M, Q8>(a, ph, kind, l, Lw, h, tag0);
        if (!ok) return;
        if (kind == kAttn) stage_gateup<Q8>(a, Lw);
    }

    if (a.io.mode == LYK_STEP_GREEDY && b == 0) {
        // ---- greedy token of row 0 (M == 1): first index of the maximum
        const int V = a.md.vocab_size, tiles = (V + a.md.tile_rows[4] - 1) / a.md.tile_rows[4];
        const uint32_t htag = tag0 | (uint32_t)L;
        mark(a, nph, 0);
        const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
        __shared__ float bv[kWaves];
        __shared__ int bi[kWaves], bb[kWaves];
        Best bst{-INFINITY, 0x7fffffff};
        int bad = 0;
        bool good = true;
        // four tiles' candidates per thread per round trip
        constexpr int TB = 4;
        for (int t0 = tid; t0 < tiles; t0 += kThreads * TB) {
            uint32_t w[TB * 3];
            uint32_t want = 0, have = 0;
#pragma unroll
            for (int q = 0; q < TB; ++q)
                if (t0 + q * kThreads < tiles) want |= 7u << (3 * q);
            auto pending = [&]() {
                return poll_batch<TB * 3>(
                    want, have, htag,
                    [&](int u) { return a.best + (size_t)min(t0 + (u / 3) * kThreads, tiles - 1) * 3 + u % 3; },
                    [&](int u, uint32_t x) { w[u] = x; });
            };
            good = spin(a, pending) && good;
#pragma unroll
            for (int q = 0; q < TB; ++q)
                if (t0 + q * kThreads < tiles) {
                    bst = better(bst, Best{bitsf(w[3 * q]), (int)w[3 * q + 1]});
                    bad += (int)w[3 * q + 2];
                }
        }
        // The token and position change only after every other workgroup
        // has finished this launch (and so read them).
        for (int w = tid + 1; w < (int)gridDim.x; w += kThreads) {
            auto pending = [&]() { return load_sc1(a.seq + w) == seq + 1u ? 0 : 1; };
            good = spin(a, pending) && good;
        }
        if (block_any<4>(!good)) return;
        bst = wave_best(bst);
        bad = (int)wave_total((float)bad);
        if (lane == 0) { bv[wave] = bst.v; bi[wave] = bst.i; bb[wave] = bad; }
        __syncthreads();
        if (tid == 0) {
            Best r{bv[0], bi[0]};
            int nb = bb[0];
            for (int w = 1; w < kWaves; ++w) { r = better(r, Best{bv[w], bi[w]}); nb += bb[w]; }
            const int token = r.i < V ? r.i : 0;
            store_sc1(a.io.tokens, token);
            store_sc1(a.io.positions, ld(a.io.positions) + 1);
            if (a.io.nonfinite) st(a.io.nonfinite, ld(a.io.nonfinite) + nb);
            if (a.io.history && a.io.step) {
                const int s = ld(a.io.step);
                st(a.io.history + s, token);
                st(a.io.step, s + 1);
            }
        }
        mark(a, nph, 3);
    }
    if (threadIdx.x == 0) store_sc1(a.seq + b, seq + 1u);
    if (a.io.trace && threadIdx.x == 0)
        st(a.io.trace + (size_t)b * (2 + 4 * a.phases) + 1, (uint64_t)__builtin_amdgcn_s_memrealtime());
}

// ------------------------------------------------------------ host side

// Tiles and chunks of an [n, k] matrix in the tiled layout of tile height tr.
void tiled_shape(int64_t n, int64_t k, bool paired, bool q8, int tr, int64_t& tiles, int64_t& chunks,
                 int64_t& ck) {
    const int lpr = 64 / tr, unit = q8 ? 16 : 32;
    tiles = paired ? (n + tr / 2 - 1) / (tr / 2) : (n + tr - 1) / tr;
    const int64_t nb = ((k + unit - 1) / unit + lpr - 1) / lpr;
    chunks = (nb + kChunkBlocks - 1) / kChunkBlocks;
    ck = (int64_t)kChunkBlocks * lpr * unit;
}

// Tile height for an [n, k] matrix on a grid of `grid` workgroups.
// A matrix whose input is the RMSNorm of the residual (QKV, gate/up, LM head)
// gains nothing from cutting tiles into K pieces (every workgroup holds the
// whole residual), and each piece costs a merge hop: the height whose busiest
// workgroup streams the fewest chunks, a merge counted as kMergeChunks more
// (about the chunks a CU streams in the hop's time), ties to the taller.
// Otherwise (polled inputs: O, down), the tallest whose busiest workgroup
// streams at most 15% more chunks than the average busy one (pieces poll
// only their share of the input window); failing that, the one whose
// busiest workgroup streams least. Taller tiles also keep a wave's lanes on
// more rows, so fewer lane sums to combine.
constexpr int64_t kMergeChunks = 16;
int choose_tile_rows(int64_t n, int64_t k, bool paired, bool q8, bool normed_input, int grid) {
    int best = 0;
    int64_t best_max = -1;
    for (int tr : {64, 32, 16}) {
        int64_t tiles, chunks, ck;
        tiled_shape(n, k, paired, q8, tr, tiles, chunks, ck);
        const int pieces = tile_pieces((int)tiles, (int)chunks, grid);
        int64_t per_wg, busy;
        if (pieces == 1) {
            busy = tiles < grid ? tiles : grid;
            per_wg = (tiles + busy - 1) / busy * chunks;
        } else {
            busy = tiles * pieces;
            per_wg = (chunks + pieces - 1) / pieces;
        }
        // a wave's chunk range may touch at most kPieces tiles
        const int64_t lw = (per_wg + kWaves - 1) / kWaves;
        if (1 + (lw - 1 + chunks - 1) / chunks > kPieces) continue;
        if (normed_input) {
            const int64_t cost = per_wg + (pieces > 1 ? kMergeChunks : 0);
            if (best_max < 0 || cost < best_max) {
                best = tr;
                best_max = cost;
            }
            continue;
        }
        const double avg = (double)tiles * chunks / (double)busy;
        if ((double)per_wg <= 1.15 * avg) return tr;
        if (best_max < 0 || per_wg < best_max) {
            best = tr;
            best_max = per_wg;
        }
    }
    return best ? best : 64;
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
    if (!head_dim_supported(hd) || G > 16 || md.block_tokens % 16) return LYK_ERR_SHAPE;
    if (md.attn_split_tokens < 0 || md.attn_split_tokens % 16 || md.attn_max_splits < 0 ||
        md.attn_max_splits > kAttnMaxSplits)
        return LYK_ERR_INVALID_ARG;
    if (md.hidden_size > kNormPer * kThreads || (md.intermediate_size & 1) || md.num_layers > 255)
        return LYK_ERR_SHAPE;
    for (int i = 0; i < 5; ++i)
        if (md.tile_rows[i] != 16 && md.tile_rows[i] != 32 && md.tile_rows[i] != 64) return LYK_ERR_INVALID_ARG;
    if (md.lds_prefetch < -1) return LYK_ERR_INVALID_ARG;
    return LYK_OK;
}

// The five GEMVs of a step: {rows, k, paired, tile height}.
struct MatShape {
    int64_t n, k;
    bool paired;
    int tr;
};
void step_mats(const lyk_step_model& md, MatShape (&out)[5]) {
    const int64_t H = md.hidden_size, In = md.intermediate_size, nq = md.num_heads, nkv = md.num_kv_heads,
                  hd = md.head_dim;
    out[0] = {(nq + 2 * nkv) * hd, H, false, md.tile_rows[0]};
    out[1] = {H, nq * hd, false, md.tile_rows[1]};
    out[2] = {In, H, true, md.tile_rows[2]};
    out[3] = {H, In, false, md.tile_rows[3]};
    out[4] = {md.vocab_size, H, false, md.tile_rows[4]};
}

struct PhaseShape {
    int64_t tiles, chunks, range, win, ck;  // range: chunks of one workgroup, at most
    int pieces;
};
// Attention splits per (row, kv head), at most: the model's setting, else as
// many as the workgroups with no QKV tile can take, within
// [kAttnMinDefaultSplits, kAttnDefaultSplits]. A unit on a workgroup with a
// QKV tile starts its K/V loads and q poll only once that tile is done
// (measured at 7B, one row, 116 units: those units' q arrived 8 us after
// QKV was done everywhere, against 2 us for the others, and the phase took
// 17.5 us instead of 11).
PhaseShape phase_shape(const MatShape& mt, bool q8, int grid);
int attn_splits_cap(const lyk_step_model& md, int rows, int grid) {
    if (md.attn_max_splits) return md.attn_max_splits;
    MatShape mats[5];
    step_mats(md, mats);
    const PhaseShape q = phase_shape(mats[0], md.q8 != 0, grid);
    const int64_t busy = q.pieces == 1 ? std::min<int64_t>(q.tiles, grid) : q.tiles * q.pieces;
    const int64_t cap = (grid - busy) / ((int64_t)rows * md.num_kv_heads);
    return (int)std::clamp<int64_t>(cap, kAttnMinDefaultSplits, kAttnDefaultSplits);
}

// Whether GEMV phase i (0 qkv, 1 o, 2 gate/up, 3 down, 4 head) of matrix mt
// spread over G workgroups keeps within the kernel's limits: the polled
// input window of o (fp32 words) and down (fp16 pairs) within kThreads *
// kWinWords words (the RMSNorm-fed phases hold the whole residual instead),
// and each wave's chunk range within kPieces row tiles.
bool phase_fits(const MatShape& mt, bool q8, int G, int i) {
    const PhaseShape ps = phase_shape(mt, q8, G);
    if ((i == 1 || i == 3) && ps.win * ps.ck / (i == 3 ? 2 : 1) > kThreads * kWinWords) return false;
    const int64_t lw = (ps.range + kWaves - 1) / kWaves;   // chunks per wave, at most
    return 1 + (lw - 1 + ps.chunks - 1) / ps.chunks <= kPieces;
}

// Workgroups of the o phase at `rows` rows: those below the attention units,
// which fill the grid from the top (at most rows * nkv * max_splits of
// them), so that no workgroup runs both; the whole grid when that leaves
// fewer than a quarter of it or o does not fit on fewer workgroups.
int o_phase_grid(const lyk_step_model& md, int rows, int grid) {
    const int splits = attn_splits_cap(md, rows, grid);
    const int64_t units = (int64_t)rows * md.num_kv_heads * splits;
    const int64_t og = grid - units;
    if (og < grid / 4) return grid;
    MatShape mats[5];
    step_mats(md, mats);
    return phase_fits(mats[1], md.q8 != 0, (int)og, 1) ? (int)og : grid;
}
// The grid phase i (0 qkv, 1 o, 2 gate/up, 3 down, 4 head) spreads over.
int phase_grid(const lyk_step_model& md, int i, int rows, int grid) {
    return i == 1 ? o_phase_grid(md, rows, grid) : grid;
}

PhaseShape phase_shape(const MatShape& mt, bool q8, int grid) {
    PhaseShape ps;
    tiled_shape(mt.n, mt.k, mt.paired, q8, mt.tr, ps.tiles, ps.chunks, ps.ck);
    ps.pieces = tile_pieces((int)ps.tiles, (int)ps.chunks, grid);
    if (ps.pieces == 1) {
        const int64_t gp = ps.tiles < grid ? ps.tiles : grid;
        ps.range = (ps.tiles + gp - 1) / gp * ps.chunks;
        ps.win = ps.chunks;
    } else {
        ps.range = (ps.chunks + ps.pieces - 1) / ps.pieces;
        ps.win = ps.range;
    }
    return ps;
}

struct Layout {
    uint64_t err, seq, args, qkv, attn_ml, attn_acc, attn_out, d_attn, d_mlp, act, dpart, best, total;
    uint64_t dpart_stride;   // in words
};

Layout layout(const lyk_step_model& md, int rows, int grid) {
    Layout L{};
    const bool q8 = md.q8 != 0;
    const int64_t nq = md.num_heads, nkv = md.num_kv_heads, hd = md.head_dim, G = nq / nkv;
    const int64_t H = md.hidden_size;
    MatShape mats[5];
    step_mats(md, mats);
    uint64_t dpart_words = 1;
    for (int r = 1; r <= rows; ++r)   // the o phase's grid depends on the launch's rows
        for (int i = 0; i < 5; ++i) {
            const PhaseShape ps = phase_shape(mats[i], q8, phase_grid(md, i, r, grid));
            if (ps.pieces > 1)
                dpart_words = std::max<uint64_t>(dpart_words, (uint64_t)ps.tiles * ps.pieces * rows * 64);
        }
    L.dpart_stride = (dpart_words * 8 + 255) / 256 * 256 / 8;
    const int64_t head_tiles = (md.vocab_size + md.tile_rows[4] - 1) / md.tile_rows[4];
    uint64_t at = 0;
    auto take = [&](uint64_t bytes) {
        const uint64_t o = at;
        at += (bytes + 255) / 256 * 256;
        return o;
    };
    L.err = take(4);
    L.seq = take((uint64_t)grid * 4);
    L.args = take(sizeof(StepArgs));
    L.qkv = take((uint64_t)rows * (nq + 2 * nkv) * hd * 8);
    L.attn_ml = take((uint64_t)rows * nkv * kAttnMaxSplits * G * 2 * 8);
    L.attn_acc = take((uint64_t)rows * nkv * kAttnMaxSplits * G * hd * 8);
    L.attn_out = take((uint64_t)rows * nq * hd * 8);
    L.d_attn = take((uint64_t)md.num_layers * kMaxRows * H * 8);
    L.d_mlp = take((uint64_t)md.num_layers * kMaxRows * H * 8);
    L.act = take((uint64_t)rows * (md.intermediate_size / 2) * 8);
    L.dpart = take((uint64_t)5 * L.dpart_stride * 8);
    L.best = take((uint64_t)rows * head_tiles * 3 * 8);
    L.total = at;
    return L;
}

// Dynamic LDS of a launch: the largest x window or reduction buffer of any
// GEMV phase, or the attention buffers.
// LDS of a GEMV phase: its x window (+ the fold's correction table), or the
// reduction buffer it aliases after the stream.
size_t gemv_lds(const MatShape& mt, bool q8, int rows, int grid) {
    const PhaseShape ps = phase_shape(mt, q8, grid);
    const size_t unit = q8 ? 16 : 32;
    const size_t corr = rows <= kFoldRows ? (size_t)rows * ps.win * ps.ck / unit * 4 : 0;
    return std::max((size_t)kWaves * kPieces * rows * 64 * 4,
                    ((size_t)rows * ps.win * ps.ck * 2 + 15) / 16 * 16 + corr);
}

// The gate/up staging region (stage_gateup): above the LDS of the O and
// gate/up phases, which run while it is held, as many chunks per wave as
// fit (and the option allows), at most a wave's share.
struct Staging {
    int off, chunks;
    size_t end;
};
Staging gateup_staging(const lyk_step_model& md, int rows, int grid) {
    const bool q8 = md.q8 != 0;
    MatShape mats[5];
    step_mats(md, mats);
    Staging sg;
    sg.off = (int)((std::max(gemv_lds(mats[1], q8, rows, o_phase_grid(md, rows, grid)), gemv_lds(mats[2], q8, rows, grid)) +
                    255) / 256 * 256);
    const int64_t slot = q8 ? 4096 : 4608;
    const PhaseShape ps = phase_shape(mats[2], q8, grid);
    int64_t chunks = ((int64_t)kMaxDynamicLds - sg.off) / (kWaves * slot);
    chunks = std::min<int64_t>(chunks, (ps.range + kWaves - 1) / kWaves);
    if (md.lds_prefetch < 0) chunks = 0;
    else if (md.lds_prefetch > 0) chunks = std::min<int64_t>(chunks, md.lds_prefetch);
    sg.chunks = (int)std::max<int64_t>(chunks, 0);
    sg.end = sg.chunks ? (size_t)sg.off + (size_t)sg.chunks * kWaves * slot : 0;
    return sg;
}

size_t lds_bytes(const lyk_step_model& md, int rows, int grid) {
    const bool q8 = md.q8 != 0;
    MatShape mats[5];
    step_mats(md, mats);
    size_t need = gateup_staging(md, rows, grid).end;
    for (int i = 0; i < 5; ++i) need = std::max(need, gemv_lds(mats[i], q8, rows, phase_grid(md, i, rows, grid)));
    // attention: q high/low parts, chunk weights high/low, current k and v
    // (fp16), current k (fp32), then the larger of the chunk scores, the raw
    // q and the merge's (max, sum) table + partial slice
    const size_t G = md.num_heads / md.num_kv_heads, hd = md.head_dim;
    const size_t KS = (hd + 31) / 32, QS = KS * 32 + 8;
    const size_t front = 2 * 16 * QS * 2 + 2 * G * kChunkT * 2 + 2 * KS * 32 * 2 + (hd + 3) / 4 * 4 * 4;
    const size_t tail = std::max({G * (kChunkT + 4), G * hd, (size_t)kAttnMaxSplits * 16 * 2 + G * hd + kAttnMaxSplits});
    need = std::max(need, front + tail * 4);
    return need;
}

// Whether every phase fits the kernel: a wave's range touches at most
// kPieces row tiles, and the polled windows of o and down (words per row)
// fit the window poller.
bool pieces_ok(const lyk_step_model& md, int grid) {
    const bool q8 = md.q8 != 0;
    MatShape mats[5];
    step_mats(md, mats);
    for (int r = 1; r <= kMaxRows; ++r)
        for (int i = 0; i < 5; ++i)
            if (!phase_fits(mats[i], q8, phase_grid(md, i, r, grid), i)) return false;
    return true;
}

template <int M, bool Q8, int HD>
int launch(const StepArgs* d_args, int grid, size_t lds, hipStream_t st) {
    auto kern = decode_step_kernel<M, Q8, HD>;
    // Dynamic LDS beyond the default limit needs the kernel's opt-in; done
    // once per instantiation (the attribute holds for the process).
    static const bool opted_in =
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)kMaxDynamicLds) == hipSuccess;
    if (!opted_in) return LYK_ERR_LAUNCH;
    // one workgroup per CU must fit (registers, LDS); checked once per LDS size
    static thread_local size_t fits_lds = 0;
    if (fits_lds != lds) {
        int occ = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, kThreads, lds) != hipSuccess || occ < 1)
            return LYK_ERR_SHAPE;
        fits_lds = lds;
    }
    // A plain launch: with more than half of a CU's LDS per workgroup the
    // grid (one workgroup per CU) is resident at once on an otherwise idle
    // device, which the occupancy check above guarantees the kernel can
    // reach; were a workgroup ever held back, the waits it blocks are
    // bounded and end the launch with the workspace error word set.
    kern<<<dim3(grid), dim3(kThreads), lds, st>>>(d_args);
    if (hipGetLastError() != hipSuccess) return LYK_ERR_LAUNCH;
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

// Launches one workspace serves before it is zeroed again. Tags are
// (launches completed + 1) << 8 | layer in 32 bits, so they stay nonzero and
// distinct for 2^24 - 1 launches; the host re-zeroes the workspace (every
// tagged word and counter) first when the next launch would reach that.
constexpr uint64_t kTagEpochLaunches = (1ull << 24) - 1;

// Host-side state per workspace: the launch arguments last uploaded (they
// live in the workspace and are re-uploaded, in stream order, only when
// they change, so a run of identical steps uploads once) and the launches
// queued since the workspace was last zeroed.
struct WorkspaceState {
    StepArgs last;
    bool has_last = false;
    uint64_t launches = 0;
};
struct WorkspaceTable {
    std::mutex mu;
    std::unordered_map<const void*, WorkspaceState> by_ws;
};
WorkspaceTable& workspaces() {
    static WorkspaceTable* t = new WorkspaceTable;   // never destroyed: no teardown-order dependence at exit
    return *t;
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

uint64_t lyk_hip_step_workspace_bytes(const lyk_step_model* model, int max_rows) {
    if (!model || max_rows < 1 || max_rows > kMaxRows || check_model(*model) != LYK_OK) return 0;
    const int grid = step_grid();
    if (!pieces_ok(*model, grid)) return 0;
    for (int m = 1; m <= max_rows; ++m)   // narrow batches carry the fold's correction table
        if (lds_bytes(*model, m, grid) > kMaxDynamicLds) return 0;
    return layout(*model, max_rows, grid).total;
}

uint32_t lyk_hip_step_phases(const lyk_step_model* model, int mode) {
    if (!model) return 0;
    // per layer QKV, attention, O, gate/up, down; the LM head; the argmax
    return (uint32_t)model->num_layers * 5u + (mode == LYK_STEP_HIDDEN ? 0u : 1u) +
           (mode == LYK_STEP_GREEDY ? 1u : 0u);
}

int lyk_hip_step_grid(void) { return step_grid(); }

int lyk_hip_step_tile_rows(int64_t n, int64_t k, int paired, int q8, int normed_input) {
    const int grid = step_grid();
    if (n <= 0 || k <= 0 || grid < 1) return 0;
    return choose_tile_rows(n, k, paired != 0, q8 != 0, normed_input != 0, grid);
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
    if (lds > kMaxDynamicLds) return LYK_ERR_SHAPE;

    char* ws = static_cast<char*>(d_workspace);
    StepArgs a;
    std::memset(&a, 0, sizeof a);
    a.md = *model;
    a.io = *io;
    a.err = reinterpret_cast<int*>(ws + L.err);
    a.seq = reinterpret_cast<uint32_t*>(ws + L.seq);
    a.qkv = reinterpret_cast<u64*>(ws + L.qkv);
    a.attn_ml = reinterpret_cast<u64*>(ws + L.attn_ml);
    a.attn_acc = reinterpret_cast<u64*>(ws + L.attn_acc);
    a.attn_out = reinterpret_cast<u64*>(ws + L.attn_out);
    a.d_attn = reinterpret_cast<u64*>(ws + L.d_attn);
    a.d_mlp = reinterpret_cast<u64*>(ws + L.d_mlp);
    a.act = reinterpret_cast<u64*>(ws + L.act);
    a.dpart = reinterpret_cast<u64*>(ws + L.dpart);
    a.dpart_stride = (size_t)L.dpart_stride;
    a.best = reinterpret_cast<u64*>(ws + L.best);
    a.attn_split_tokens = model->attn_split_tokens ? model->attn_split_tokens : kAttnSplitTokens;
    a.attn_max_splits = attn_splits_cap(*model, m, grid);
    a.phases = (int)lyk_hip_step_phases(model, io->mode);
    a.spin_ticks = model->wait_limit_us ? (uint64_t)model->wait_limit_us * 100u : kSpinTicks;
    const Staging sg = gateup_staging(*model, m, grid);
    a.pf_off = sg.off;
    a.pf_chunks = sg.chunks;
    a.o_grid = o_phase_grid(*model, m, grid);
    hipStream_t st = static_cast<hipStream_t>(stream);
    StepArgs* d_args = reinterpret_cast<StepArgs*>(ws + L.args);
    WorkspaceTable& tab = workspaces();
    std::lock_guard<std::mutex> lock(tab.mu);
    WorkspaceState& w = tab.by_ws[d_workspace];
    if (w.launches >= kTagEpochLaunches) {
        // a new tag epoch: no word from before can match a tag again
        if (hipMemsetAsync(d_workspace, 0, workspace_bytes, st) != hipSuccess) return LYK_ERR_HIP;
        w.launches = 0;
        w.has_last = false;
    }
    if (!w.has_last || std::memcmp(&w.last, &a, sizeof a) != 0) {
        if (hipMemcpyAsync(d_args, &a, sizeof a, hipMemcpyHostToDevice, st) != hipSuccess) return LYK_ERR_HIP;
        w.last = a;
        w.has_last = true;
    }
    rc = model->q8 ? launch_hd<true>(model->head_dim, m, d_args, grid, lds, st)
                   : launch_hd<false>(model->head_dim, m, d_args, grid, lds, st);
    if (rc == LYK_OK) ++w.launches;
    return rc;
}

int lyk_hip_step_reset(void* d_workspace, uint64_t workspace_bytes, void* stream) {
    if (!d_workspace) return LYK_ERR_INVALID_ARG;
    WorkspaceTable& tab = workspaces();
    std::lock_guard<std::mutex> lock(tab.mu);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (hipMemsetAsync(d_workspace, 0, workspace_bytes, st) != hipSuccess) return LYK_ERR_HIP;
    tab.by_ws[d_workspace] = WorkspaceState{};
    return LYK_OK;
}

uint64_t lyk_hip_step_launches(const void* d_workspace) {
    WorkspaceTable& tab = workspaces();
    std::lock_guard<std::mutex> lock(tab.mu);
    const auto it = tab.by_ws.find(d_workspace);
    return it == tab.by_ws.end() ? 0 : it->second.launches;
}

int lyk_hip_step_set_launches(const lyk_step_model* model, int max_rows, void* d_workspace,
                              uint64_t workspace_bytes, uint64_t launches, void* stream) {
    if (!model || !d_workspace || max_rows < 1 || max_rows > kMaxRows || launches > kTagEpochLaunches)
        return LYK_ERR_INVALID_ARG;
    if (check_model(*model) != LYK_OK) return LYK_ERR_INVALID_ARG;
    const int grid = step_grid();
    if (grid < 1) return LYK_ERR_HIP;
    const Layout L = layout(*model, max_rows, grid);
    if (L.total > workspace_bytes) return LYK_ERR_WORKSPACE;
    WorkspaceTable& tab = workspaces();
    std::lock_guard<std::mutex> lock(tab.mu);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (hipMemsetAsync(d_workspace, 0, workspace_bytes, st) != hipSuccess) return LYK_ERR_HIP;
    // every workgroup's counter; the host copy is synchronous (pageable
    // source), so the vector may go out of scope afterwards
    std::vector<uint32_t> seq((size_t)grid, (uint32_t)launches);
    if (hipStreamSynchronize(st) != hipSuccess ||
        hipMemcpy(static_cast<char*>(d_workspace) + L.seq, seq.data(), seq.size() * 4, hipMemcpyHostToDevice) !=
            hipSuccess)
        return LYK_ERR_HIP;
    tab.by_ws[d_workspace] = WorkspaceState{};
    tab.by_ws[d_workspace].launches = launches;
    return LYK_OK;
}

int lyk_hip_step_error(const void* d_workspace, int32_t* error_out, void* stream) {
    if (!d_workspace || !error_out) return LYK_ERR_INVALID_ARG;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (hipMemcpyAsync(error_out, d_workspace, 4, hipMemcpyDeviceToHost, st) != hipSuccess) return LYK_ERR_HIP;
    if (hipStreamSynchronize(st) != hipSuccess) return LYK_ERR_HIP;
    return LYK_OK;
}

}  // extern "C"
