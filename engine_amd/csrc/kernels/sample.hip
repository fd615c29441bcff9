// Temperature / top-k / top-p sampling of logits on the device.
//
// Reference: Sampler::Sample (core/generation/sampler.cpp:35-106). The rule,
// restated: non-finite logits fail the row; temperature 0 takes the first
// index of the maximum; otherwise the indices are stably sorted by logit,
// descending, and cut to top_k; p_i = exp(double(l_i - l_max) * inv_temp) with
// inv_temp = 1.0f / temperature (float); the nucleus is the shortest prefix
// whose running sum of p_i / denom reaches top_p (denom = the sum of the
// candidates' p_i, in sorted order); r = u * mass (mass = the nucleus's sum),
// u the draw generate_canonical<double, 53> of the caller's mt19937_64 (what
// uniform_real_distribution<double>(0, mass) computes); the token is the
// first of the nucleus whose running sum reaches r.
//
// One workgroup per row:
//   1. scan: non-finite check and the first maximum;
//   2. with top_k, the k-th largest logit by a radix select over the order
//      bits (four 8-bit digits, LDS histograms), so that only logits at or
//      above it are kept;
//      candidates: every kept index whose p_i >= 2^-54, as 64-bit sort keys
//      (inverted order-preserving logit bits, index) -- a prefix of the
//      sorted order, and the only terms that can change a running sum that
//      starts at p_0 = 1: a smaller term is below half an ulp of every sum
//      the rule forms (each is >= 1, or for the top-p sums >= 1/denom with
//      the terms divided by denom alike), so adding it rounds back;
//   3. sort of the keys: bitonic in LDS when they fit, else a stable radix
//      sort in global memory;
//   4. p_i in parallel, then the rule's three running sums in order (by
//      wave 0, all lanes carrying the same sums), in double, as the
//      reference forms them.
// The result equals the reference's draw for draw; the one difference is
// the device's double exp, within an ulp of the host's, which moves a token
// only when r lies within about 1e-16 of a boundary.
#include <cmath>
#include <mutex>
#include <random>

#include "common.h"

namespace lyk {
namespace {

constexpr int kMaxRows = 4;            // rows per call, at most (the decode batch)
constexpr int kSampleThreads = 1024;
constexpr int kLdsKeys = 8192;        // keys sorted in LDS (64 KiB); more go through global memory
constexpr double kMinTerm = 0x1p-54;  // terms below this never change a running sum

struct Draws {
    double u[kMaxRows];
};

__device__ __forceinline__ uint32_t order_bits(float x) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);   // ascending with x
}

__device__ __forceinline__ int wave_of(int tid) { return tid >> 6; }

// Whether a term exp(d) reaches kMinTerm (ln 2^-54 = -37.4299...): exp is
// evaluated only near the cut.
__device__ __forceinline__ bool significant(double d) {
    if (d < -37.45) return false;
    if (d > -37.41) return true;
    return exp(d) >= kMinTerm;
}

// Sum over the workgroup of an int, every thread gets it.
__device__ int block_count(int v, int* scratch) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    if (lane == 0) scratch[wave] = v;
    __syncthreads();
    int s = 0;
    for (int w = 0; w < kSampleThreads / 64; ++w) s += scratch[w];
    __syncthreads();
    return s;
}

// Exclusive prefix of v over the threads in thread order, and the total.
__device__ int block_prefix(int v, int* scratch, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) scratch[wave] = x;
    __syncthreads();
    int base = 0;
    total = 0;
    for (int w = 0; w < kSampleThreads / 64; ++w) {
        if (w < wave) base += scratch[w];
        total += scratch[w];
    }
    __syncthreads();
    return base + x - v;
}

// Ascending bitonic sort of a[0..n2) (n2 a power of two) by the workgroup.
template <class T>
__device__ void bitonic_sort(T* a, int n2) {
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n2; i += kSampleThreads) {
                const int p = i ^ j;
                if (p > i) {
                    const bool up = (i & k) == 0;
                    const T x = a[i], y = a[p];
                    if ((x > y) == up) {
                        a[i] = y;
                        a[p] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Stable LSD radix sort of keys[0..n) by their upper 32 bits, 4 bits a pass
// (8 passes), through tmp; equal upper halves keep their input order, and
// the result ends in keys. Each pass: digit histogram, bases, then tiles of
// one key per thread scattered in order (rank within the tile from wave
// ballots and per-wave counts).
__device__ void radix_sort_hi(uint64_t* keys, uint64_t* tmp, int n, int* sh) {
    constexpr int W = kSampleThreads / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int* hist = sh;        // [16]
    int* base = sh + 16;   // [16] next output slot per digit
    int* wcnt = sh + 32;   // [W][16] keys per digit in each wave of the tile
    uint64_t* src = keys;
    uint64_t* dst = tmp;
    const uint64_t lt = (1ull << lane) - 1;
    for (int pass = 0; pass < 8; ++pass) {
        const int shift = 32 + 4 * pass;
        if (tid < 16) hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += kSampleThreads) atomicAdd(&hist[(int)(src[i] >> shift) & 15], 1);
        __syncthreads();
        if (tid == 0) {
            int acc = 0;
            for (int d = 0; d < 16; ++d) {
                base[d] = acc;
                acc += hist[d];
            }
        }
        __syncthreads();
        for (int t0 = 0; t0 < n; t0 += kSampleThreads) {
            const int i = t0 + tid;
            const bool live = i < n;
            const uint64_t key = live ? src[i] : 0ull;
            const int d = live ? (int)(key >> shift) & 15 : -1;
            int rank = 0;
            for (int dv = 0; dv < 16; ++dv) {
                const uint64_t m = __ballot(d == dv);
                if (d == dv) rank = __popcll(m & lt);
                if (lane == 0) wcnt[wave * 16 + dv] = __popcll(m);
            }
            __syncthreads();
            if (live) {
                int off = base[d] + rank;
                for (int w = 0; w < wave; ++w) off += wcnt[w * 16 + d];
                dst[off] = key;
            }
            __syncthreads();
            if (tid < 16) {
                int c = 0;
                for (int w = 0; w < W; ++w) c += wcnt[w * 16 + tid];
                base[tid] += c;
            }
            __syncthreads();
        }
        uint64_t* sw = src;
        src = dst;
        dst = sw;
    }
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(const float* __restrict__ logits, int ldl, int n,
                                                                float temperature, int top_k, float top_p,
                                                                Draws draws, uint64_t* __restrict__ keys_all,
                                                                double* __restrict__ probs_all, int cap,
                                                                int32_t* __restrict__ tokens) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int scratch[kSampleThreads / 64];
    __shared__ int sort_sh[32 + 16 * (kSampleThreads / 64)];
    __shared__ float bmax[kSampleThreads / 64];
    __shared__ int bidx[kSampleThreads / 64];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* l = logits + (size_t)row * ldl;
    uint64_t* keys = keys_all + (size_t)row * cap;
    double* probs = probs_all + (size_t)row * cap;

    // 1. non-finite count and the first maximum
    float mv = -INFINITY;
    int mi = 0x7fffffff, bad = 0;
    for (int i = tid; i < n; i += kSampleThreads) {
        const float x = l[i];
        if (!isfinite(x)) {
            bad = 1;
            continue;
        }
        if (x > mv || (x == mv && i < mi)) {
            mv = x;
            mi = i;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float v2 = __shfl_xor(mv, o, 64);
        const int i2 = __shfl_xor(mi, o, 64);
        if (v2 > mv || (v2 == mv && i2 < mi)) {
            mv = v2;
            mi = i2;
        }
    }
    if ((tid & 63) == 0) {
        bmax[tid >> 6] = mv;
        bidx[tid >> 6] = mi;
    }
    bad = block_count(bad, scratch);   // its barriers publish bmax / bidx too
    if (bad) {
        if (tid == 0) tokens[row] = -1;
        return;
    }
    mv = bmax[0];
    mi = bidx[0];
    for (int w = 1; w < kSampleThreads / 64; ++w)
        if (bmax[w] > mv || (bmax[w] == mv && bidx[w] < mi)) {
            mv = bmax[w];
            mi = bidx[w];
        }
    if (temperature == 0.0f) {
        if (tid == 0) tokens[row] = mi;
        return;
    }

    // 2. top_k: the order bits of the k-th largest logit (ties counted
    //    whole: the sort below cuts them by index)
    uint32_t floor_bits = 0;
    if (top_k > 0 && top_k < n) {
        int* hist = reinterpret_cast<int*>(smem);
        __shared__ int pick, left;
        uint32_t prefix = 0, mask = 0;
        if (tid == 0) left = top_k;
        for (int d = 3; d >= 0; --d) {
            for (int b = tid; b < 256; b += kSampleThreads) hist[b] = 0;
            __syncthreads();
            for (int i = tid; i < n; i += kSampleThreads) {
                const uint32_t ob = order_bits(l[i]);
                if ((ob & mask) == prefix) atomicAdd(&hist[(ob >> (8 * d)) & 255], 1);
            }
            __syncthreads();
            if (tid == 0) {
                int cum = 0, b = 255;
                for (; b > 0; --b) {
                    if (cum + hist[b] >= left) break;
                    cum += hist[b];
                }
                pick = b;
                left -= cum;
            }
            __syncthreads();
            prefix |= (uint32_t)pick << (8 * d);
            mask |= 255u << (8 * d);
        }
        floor_bits = prefix;
    }
    // candidates: kept and p_i >= 2^-54, keys (inverted logit order bits, index)
    const float inv_temp = 1.0f / temperature;
    auto keep = [&](float x) {
        return order_bits(x) >= floor_bits && significant((double)(x - mv) * inv_temp);
    };
    // each thread a contiguous index range, so the keys come out in index
    // order (the radix sort below is stable)
    const int per = (n + kSampleThreads - 1) / kSampleThreads;
    const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
    int mine = 0;
    for (int i = i0; i < i1; ++i)
        if (keep(l[i])) ++mine;
    int total;
    int at = block_prefix(mine, scratch, total);
    for (int i = i0; i < i1; ++i)
        if (keep(l[i])) keys[at++] = ((uint64_t)~order_bits(l[i]) << 32) | (uint32_t)i;
    const int nc = total;   // >= 1: the maximum's term is 1

    // 3. sort ascending: logits descending, equal logits by index
    int n2 = 1;
    while (n2 < nc) n2 <<= 1;
    __syncthreads();
    if (n2 <= kLdsKeys) {
        uint64_t* s = reinterpret_cast<uint64_t*>(smem);
        for (int i = tid; i < n2; i += kSampleThreads) s[i] = i < nc ? keys[i] : ~0ull;
        __syncthreads();
        bitonic_sort(s, n2);
        for (int i = tid; i < nc; i += kSampleThreads) keys[i] = s[i];
    } else {
        // by logit only: the keys are in index order and the sort is stable
        radix_sort_hi(keys, reinterpret_cast<uint64_t*>(probs), nc, sort_sh);
    }
    __syncthreads();

    // 4. terms in parallel; the running sums in order by wave 0: a batch of
    //    64 terms comes in one coalesced load, and every lane adds the batch's
    //    terms one by one (read across lanes in order), so all lanes carry the
    //    sequential sum; a term past the end reads 0, which changes no sum
    const int cand = top_k > 0 && top_k < nc ? top_k : nc;
    for (int i = tid; i < cand; i += kSampleThreads)
        probs[i] = exp((double)(l[(uint32_t)keys[i]] - mv) * inv_temp);
    __syncthreads();
    if (wave_of(tid) != 0) return;
    const int lane = tid & 63;
    auto term = [&](int i, int end) { return i < end ? probs[i] : 0.0; };
    double denom = 0.0;
    for (int i0 = 0; i0 < cand; i0 += 64) {
        const double v = term(i0 + lane, cand);
#pragma unroll
        for (int j = 0; j < 64; ++j) denom += __shfl(v, j, 64);
    }
    int nucleus = cand;
    if (top_p < 1.0f) {
        double cum = 0.0;
        bool found = false;
        for (int i0 = 0; i0 < cand && !found; i0 += 64) {
            const double q = term(i0 + lane, cand) / denom;
#pragma unroll
            for (int j = 0; j < 64; ++j) {
                cum += __shfl(q, j, 64);
                if (!found && i0 + j < cand && cum >= (double)top_p) {
                    nucleus = i0 + j + 1;
                    found = true;
                }
            }
        }
    }
    double mass = 0.0;
    for (int i0 = 0; i0 < nucleus; i0 += 64) {
        const double v = term(i0 + lane, nucleus);
#pragma unroll
        for (int j = 0; j < 64; ++j) mass += __shfl(v, j, 64);
    }
    const double r = draws.u[row] * (mass - 0.0) + 0.0;
    double acc = 0.0;
    int pick = nucleus - 1;
    bool found = false;
    for (int i0 = 0; i0 < nucleus && !found; i0 += 64) {
        const double v = term(i0 + lane, nucleus);
#pragma unroll
        for (int j = 0; j < 64; ++j) {
            acc += __shfl(v, j, 64);
            if (!found && i0 + j < nucleus && r <= acc) {
                pick = i0 + j;
                found = true;
            }
        }
    }
    const int tok = (int)(uint32_t)keys[pick];
    if (lane != 0) return;
    tokens[row] = tok;
}

// Launches sample_kernel over rows [0, m) with the scratch at `ws` (keys,
// then probabilities, m * cap 8-byte entries each; every entry a row uses
// is written before it is read, so the scratch needs no clearing).
int launch_sample(const float* d_logits, int64_t ldl, int m, int64_t n, float temperature, int32_t top_k,
                  float top_p, const double* u, int32_t* d_tokens, void* ws, hipStream_t stream) {
    Draws d{};
    for (int r = 0; r < m; ++r) {
        if (!(u[r] >= 0.0 && u[r] < 1.0)) return LYK_ERR_INVALID_ARG;
        d.u[r] = u[r];
    }
    int cap = 1;
    while (cap < n) cap <<= 1;
    char* base = static_cast<char*>(ws);
    uint64_t* keys = reinterpret_cast<uint64_t*>(base);
    double* probs = reinterpret_cast<double*>(base + (size_t)m * cap * 8);
    static std::once_flag lds_once;
    static bool lds_ok = false;
    std::call_once(lds_once, [] {
        lds_ok = hipFuncSetAttribute((const void*)sample_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     kLdsKeys * 8) == hipSuccess;
    });
    if (!lds_ok) return LYK_ERR_HIP;
    hipLaunchKernelGGL(sample_kernel, dim3(m), dim3(kSampleThreads), kLdsKeys * 8, stream, d_logits, (int)ldl,
                       (int)n, temperature, top_k, top_p, d, keys, probs, cap, d_tokens);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

int check_sample_args(const float* d_logits, int64_t ldl, int m, int64_t n, float temperature, int32_t top_k,
                      float top_p, const double* u, const int32_t* d_tokens) {
    if (!d_logits || !d_tokens || !u || m < 1 || n < 1 || ldl < n || n > (1 << 30)) return LYK_ERR_INVALID_ARG;
    if (m > kMaxRows) return LYK_ERR_SHAPE;
    if (!(temperature >= 0.0f) || !std::isfinite(temperature) || !(top_p > 0.0f) || top_p > 1.0f || top_k < 0)
        return LYK_ERR_INVALID_ARG;
    return LYK_OK;
}

// ---------------------------------------------------------- static scratch
// The allocation-free variant's scratch: a file-scope device array, one copy
// per GPU the library is loaded on, held until the process ends. Its size
// covers kMaxRows rows of up to kStaticLogits logits (2^18 >= every Qwen2
// vocabulary). Host code never passes the array's name to a kernel (on the
// host it is a stand-in, not a device address): it passes the address
// hipGetSymbolAddress gave for the current device.
constexpr int64_t kStaticLogits = 1 << 18;
constexpr size_t kStaticScratchBytes = (size_t)kMaxRows * kStaticLogits * 16;   // 16 MiB
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices];   // per device, from hipGetSymbolAddress

// The current device's address of `scratch`, looked up on the device's
// first call; nullptr when the lookup fails.
void* device_scratch() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (!scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        scratch_ptr[dev] = p;
    }
    return scratch_ptr[dev];
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

uint64_t lyk_hip_sample_workspace_bytes(int m, int64_t n) {
    if (m < 1 || n < 1) return 0;
    int64_t cap = 1;
    while (cap < n) cap <<= 1;
    return (uint64_t)m * (uint64_t)cap * 16;
}

int lyk_hip_sample(const float* d_logits, int64_t ldl, int m, int64_t n, float temperature, int32_t top_k,
                   float top_p, const double* u, int32_t* d_tokens, void* d_workspace, uint64_t workspace_bytes,
                   void* stream) {
    const int rc = check_sample_args(d_logits, ldl, m, n, temperature, top_k, top_p, u, d_tokens);
    if (rc != LYK_OK) return rc;
    if (!d_workspace || workspace_bytes < lyk_hip_sample_workspace_bytes(m, n)) return LYK_ERR_WORKSPACE;
    return launch_sample(d_logits, ldl, m, n, temperature, top_k, top_p, u, d_tokens, d_workspace,
                         static_cast<hipStream_t>(stream));
}

int lyk_hip_sample_static(const float* d_logits, int64_t ldl, int m, int64_t n, float temperature, int32_t top_k,
                          float top_p, const double* u, int32_t* d_tokens, void* stream) {
    const int rc = check_sample_args(d_logits, ldl, m, n, temperature, top_k, top_p, u, d_tokens);
    if (rc != LYK_OK) return rc;
    if (n > kStaticLogits) return LYK_ERR_SHAPE;   // beyond the static scratch
    void* ws = device_scratch();
    if (!ws) return LYK_ERR_HIP;
    return launch_sample(d_logits, ldl, m, n, temperature, top_k, top_p, u, d_tokens, ws,
                         static_cast<hipStream_t>(stream));
}

// The draws Sampler takes from its generator: std::mt19937_64 seeded with
// the request's seed (sampler.cpp:32-33), one generate_canonical<double, 53>
// per non-greedy token (what uniform_real_distribution<double>(0, mass)
// draws before scaling by mass).
void* lyk_rng_new(uint64_t seed) { return new std::mt19937_64(seed); }
void lyk_rng_free(void* g) { delete static_cast<std::mt19937_64*>(g); }
double lyk_rng_canonical(void* g) {
    return std::generate_canonical<double, 53>(*static_cast<std::mt19937_64*>(g));
}

}  // extern "C"
