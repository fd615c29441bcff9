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
//
// Without top_k (or with top_k past what LDS sorts) and more logits than LDS
// holds, lyk_hip_sample runs the same rule in three launches so the sort
// uses the whole GPU: sample_prep_kernel (steps 1-2: every index with its
// key, the inverted order bits for a candidate and all ones for the rest),
// a stable device-wide radix sort of (key, index) pairs per row (rocPRIM),
// and sample_finish_kernel (step 4 over the sorted candidates, a prefix of
// the sorted row). Keys compare as the single-kernel path's do (logits
// descending, equal logits by index), so both paths give the same token.
#include <cmath>
#include <cstring>
#include <mutex>
#include <random>

#include <rocprim/device/device_radix_sort.hpp>

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

// Steps 1-2 of a row by its workgroup: the non-finite check, the first
// maximum (value, index) and, with top_k, the order bits of the k-th largest
// logit (ties counted whole: the sort cuts them by index; 0 without top_k).
// hist: 256 ints of LDS.
struct RowHead {
    float mv;
    int mi;
    bool bad;
    uint32_t floor_bits;
};
__device__ RowHead row_head(const float* l, int n, int top_k, int* scratch, float* bmax, int* bidx, int* hist) {
    const int tid = threadIdx.x;
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
    if (bad) return RowHead{0.0f, 0, true, 0u};
    mv = bmax[0];
    mi = bidx[0];
    for (int w = 1; w < kSampleThreads / 64; ++w)
        if (bmax[w] > mv || (bmax[w] == mv && bidx[w] < mi)) {
            mv = bmax[w];
            mi = bidx[w];
        }

    // 2. top_k: the order bits of the k-th largest logit (ties counted
    //    whole: the sort below cuts them by index)
    uint32_t floor_bits = 0;
    if (top_k > 0 && top_k < n) {
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
    return RowHead{mv, mi, false, floor_bits};
}

// 4. the rule's running sums over the candidates' terms probs[0..cand) in
//    sorted order, by wave 0, in double as the reference forms them:
//    * denom, the sum of every term: a batch of 64 terms comes in one
//      coalesced load (the next batch's load is issued before this batch is
//      added), and every lane adds the batch's terms one by one (read across
//      lanes in order), so all lanes carry the sequential sum; lane j keeps
//      the running sum after term j: prefix[i] = the running sum through
//      term i;
//    * with top_p < 1, the running sum of term / denom up to the first that
//      reaches top_p (the nucleus);
//    * mass, the sum of the nucleus's terms: the same additions as denom's
//      first `nucleus` ones, so prefix[nucleus - 1];
//    * the pick, the first term whose running sum reaches r = u * mass: the
//      same running sums again, stored and non-decreasing, so a search (64
//      probes a round) finds it.
//    index(i) is candidate i's token.
// The rule's sequential sums run on one wave with every lane carrying the
// same sum. A batch of 64 terms (one coalesced load, issued a batch ahead)
// goes through a wave-private LDS stage that every lane then reads whole
// (the same addresses for all lanes: broadcast reads), so each add takes its
// operand from a register and the chain of dependent adds is all that
// serializes; lane 0 writes the running sums to `run`. Only the one wave
// that calls these touches `stage` and `run`, and its LDS accesses complete
// in order.
__device__ __forceinline__ double add_batch(double acc, double v, int lane, double* stage, double* run) {
    stage[lane] = v;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int c = 0; c < 64; c += 16) {
        double t[16], r[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) t[j] = stage[c + j];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            acc += t[j];
            r[j] = acc;
        }
        if (lane == 0)
#pragma unroll
            for (int j = 0; j < 16; ++j) run[c + j] = r[j];
    }
    __builtin_amdgcn_wave_barrier();
    return acc;
}

// denom = p[0] + p[1] + ... in order; prefix[i] = the running sum through p[i].
__device__ double running_sums(const double* p, double* prefix, int cand, int lane, double* stage, double* run) {
    double acc = 0.0;
    double v = lane < cand ? p[lane] : 0.0;
    for (int i0 = 0; i0 < cand; i0 += 64) {
        const double next = i0 + 64 + lane < cand ? p[i0 + 64 + lane] : 0.0;
        acc = add_batch(acc, v, lane, stage, run);
        if (i0 + lane < cand) prefix[i0 + lane] = run[lane];
        v = next;
    }
    return acc;
}

// The count of leading terms q[0..] whose running sum first reaches target
// (the nucleus), cand when it never does.
__device__ int first_reaching(const double* q, int cand, double target, int lane, double* stage, double* run) {
    double acc = 0.0;
    double v = lane < cand ? q[lane] : 0.0;
    for (int i0 = 0; i0 < cand; i0 += 64) {
        const double next = i0 + 64 + lane < cand ? q[i0 + 64 + lane] : 0.0;
        acc = add_batch(acc, v, lane, stage, run);
        if (acc >= target) {   // within this batch (the sums only grow)
            const uint64_t hit = __ballot(i0 + lane < cand && run[lane] >= target);
            if (hit) return i0 + __ffsll((unsigned long long)hit);
        }
        v = next;
    }
    return cand;
}

// 4. the rule's running sums over the candidates' terms probs[0..cand) in
//    sorted order, by wave 0, in double as the reference forms them:
//    * denom, the sum of every term: a batch of 64 terms comes in one
//      coalesced load (the next batch's load is issued before this batch is
//      added), and every lane adds the batch's terms one by one (read across
//      lanes in order), so all lanes carry the sequential sum; lane j keeps
//      the running sum after term j: prefix[i] = the running sum through
//      term i;
//    * with top_p < 1, the running sum of term / denom up to the first that
//      reaches top_p (the nucleus);
//    * mass, the sum of the nucleus's terms: the same additions as denom's
//      first `nucleus` ones, so prefix[nucleus - 1];
//    * the pick, the first term whose running sum reaches r = u * mass: the
//      same running sums again, stored and non-decreasing, so a search (64
//      probes a round) finds it.
//    index(i) is candidate i's token.
// The rule's sequential sums run on one wave with every lane carrying the
// same sum: a batch of B terms is read by every lane from the same
// addresses (broadcast loads; the next batch's loads are issued before this
// batch's adds), so each add takes its operand from a register and the chain
// of dependent adds is all that serializes. The address goes through a
// register the compiler cannot see into, so the loads stay vector loads.
template <int B>
__device__ __forceinline__ void load_batch(double (&t)[B], const double* p, int i0, int end) {
#pragma unroll
    for (int j = 0; j < B; ++j) t[j] = i0 + j < end ? p[i0 + j] : 0.0;
}
__device__ __forceinline__ const double* vector_address(const double* p) {
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    return p + zero;
}

// denom = p[0] + p[1] + ... in order; prefix[i] = the running sum through p[i].
template <int B>
__device__ double running_sums(const double* probs, double* prefix, int cand, int lane) {
    const double* p = vector_address(probs);
    double acc = 0.0;
    double t[B];
    load_batch(t, p, 0, cand);
    for (int i0 = 0; i0 < cand; i0 += B) {
        double tn[B], r[B];
        load_batch(tn, p, i0 + B, cand);
#pragma unroll
        for (int j = 0; j < B; ++j) {
            acc += t[j];
            r[j] = acc;
        }
        if (lane == 0)
#pragma unroll
            for (int j = 0; j < B; ++j)
                if (i0 + j < cand) prefix[i0 + j] = r[j];
#pragma unroll
        for (int j = 0; j < B; ++j) t[j] = tn[j];
    }
    return acc;
}

// The count of leading terms q[0..] whose running sum first reaches target
// (the nucleus), cand when it never does.
template <int B>
__device__ int first_reaching(const double* q, int cand, double target) {
    const double* p = vector_address(q);
    double acc = 0.0;
    double t[B];
    load_batch(t, p, 0, cand);
    for (int i0 = 0; i0 < cand; i0 += B) {
        double tn[B], r[B];
        load_batch(tn, p, i0 + B, cand);
#pragma unroll
        for (int j = 0; j < B; ++j) {
            acc += t[j];
            r[j] = acc;
        }
        if (acc >= target) {   // within this batch (the sums only grow)
            int f = B;
#pragma unroll
            for (int j = B - 1; j >= 0; --j) f = i0 + j < cand && r[j] >= target ? j : f;
            if (f < B) return i0 + f + 1;
        }
#pragma unroll
        for (int j = 0; j < B; ++j) t[j] = tn[j];
    }
    return cand;
}

// 4. the rule's running sums over the candidates' terms probs[0..cand) in
//    sorted order, in double as the reference forms them (every thread of
//    the workgroup calls it; the sequential sums run on wave 0):
//    * denom, the sum of every term (running_sums), with prefix[i] = the
//      running sum through term i;
//    * with top_p < 1, q_i = term_i / denom (in parallel, in place), and the
//      running sum of the q_i up to the first that reaches top_p (the
//      nucleus);
//    * mass, the sum of the nucleus's terms: the same additions as denom's
//      first `nucleus` ones, so prefix[nucleus - 1];
//    * the pick, the first term whose running sum reaches r = u * mass: the
//      same running sums again, stored and non-decreasing, so a search (64
//      probes a round) finds it.
//    index(i) is candidate i's token.
template <class Index>
__device__ void pick_token(double* probs, double* prefix, int cand, float top_p, double u, Index index,
                           int32_t* token) {
    const int tid = threadIdx.x, nthreads = blockDim.x;
    const int lane = tid & 63;
    __shared__ double sh_denom, stage[64], run[64];
    __shared__ int sh_nucleus;
    if (wave_of(tid) == 0) {
        const double d = running_sums(probs, prefix, cand, lane, stage, run);
        if (lane == 0) sh_denom = d;
    }
    __syncthreads();
    const double denom = sh_denom;
    int nucleus = cand;
    if (top_p < 1.0f) {
        for (int i = tid; i < cand; i += nthreads) probs[i] = probs[i] / denom;
        __syncthreads();
        if (wave_of(tid) == 0) {
            const int nu = first_reaching(probs, cand, (double)top_p, lane, stage, run);
            if (lane == 0) sh_nucleus = nu;
        }
        __syncthreads();
        nucleus = sh_nucleus;
    }
    if (wave_of(tid) != 0) return;
    const double mass = prefix[nucleus - 1];
    const double r = u * (mass - 0.0) + 0.0;
    // the first i < nucleus with r <= prefix[i], in [lo, hi); none: nucleus - 1
    int lo = 0, hi = nucleus;
    while (hi - lo > 64) {
        const int step = (hi - lo + 63) / 64;
        const int i = lo + lane * step;
        const uint64_t m = __ballot(i < hi && r <= prefix[i < hi ? i : lo]);
        if (m == 0) {
            lo += (hi - 1 - lo) / step * step + 1;   // past the last probe below hi
        } else {
            const int f = __ffsll((unsigned long long)m) - 1;
            hi = lo + f * step + 1;
            lo = f == 0 ? lo : lo + (f - 1) * step + 1;
        }
    }
    const uint64_t m = __ballot(lo + lane < hi && r <= prefix[lo + lane < hi ? lo + lane : lo]);
    const int pick = m ? lo + __ffsll((unsigned long long)m) - 1 : nucleus - 1;
    const int tok = index(pick);
    if (lane != 0) return;
    *token = tok;
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(const float* __restrict__ logits, int ldl, int n,
                                                                float temperature, int top_k, float top_p,
                                                                Draws draws, uint64_t* __restrict__ keys_all,
                                                                double* __restrict__ probs_all,
                                                                double* __restrict__ prefix_all, int cap,
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
    double* prefix = prefix_all + (size_t)row * cap;

    const RowHead hd = row_head(l, n, top_k, scratch, bmax, bidx, reinterpret_cast<int*>(smem));
    if (hd.bad) {
        if (tid == 0) tokens[row] = -1;
        return;
    }
    const float mv = hd.mv;
    if (temperature == 0.0f) {
        if (tid == 0) tokens[row] = hd.mi;
        return;
    }
    const uint32_t floor_bits = hd.floor_bits;
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

    const int cand = top_k > 0 && top_k < nc ? top_k : nc;
    for (int i = tid; i < cand; i += kSampleThreads)
        probs[i] = exp((double)(l[(uint32_t)keys[i]] - mv) * inv_temp);
    __syncthreads();
    pick_token(probs, prefix, cand, top_p, draws.u[row], [&](int i) { return (int)(uint32_t)keys[i]; },
               tokens + row);
}


// ---------------------------------------------------------- wide rows
// Per-row state the prep kernel hands to the finish kernel.
struct RowState {
    float mv;    // the row's maximum logit
    int nc;      // candidates (they sort first)
    int done;    // the token is written already (non-finite row, temperature 0)
    int pad;
};

// Steps 1-2 for one row: keys_in[i] = the inverted order bits of logit i
// when it is a candidate (kept by top_k, p_i >= 2^-54), else all ones (never
// a candidate's key: that is the order bits of a negative NaN); vals_in[i] =
// i. The candidates then sort first, logits descending, equal logits by
// index (the sort is stable and the input is in index order).
__global__ __launch_bounds__(kSampleThreads) void sample_prep_kernel(const float* __restrict__ logits, int ldl, int n,
                                                                     float temperature, int top_k,
                                                                     uint32_t* __restrict__ keys_in,
                                                                     uint32_t* __restrict__ vals_in, int cap,
                                                                     RowState* __restrict__ state,
                                                                     int32_t* __restrict__ tokens) {
    __shared__ int scratch[kSampleThreads / 64];
    __shared__ float bmax[kSampleThreads / 64];
    __shared__ int bidx[kSampleThreads / 64];
    __shared__ int hist[256];
    const int row = blockIdx.x, tid = threadIdx.x;
    const float* l = logits + (size_t)row * ldl;
    const RowHead hd = row_head(l, n, top_k, scratch, bmax, bidx, hist);
    if (hd.bad || temperature == 0.0f) {
        if (tid == 0) {
            tokens[row] = hd.bad ? -1 : hd.mi;
            state[row] = RowState{0.0f, 0, 1, 0};
        }
        return;
    }
    const float inv_temp = 1.0f / temperature;
    uint32_t* ki = keys_in + (size_t)row * cap;
    uint32_t* vi = vals_in + (size_t)row * cap;
    int mine = 0;
    for (int i = tid; i < n; i += kSampleThreads) {
        const float x = l[i];
        const bool kept = order_bits(x) >= hd.floor_bits && significant((double)(x - hd.mv) * inv_temp);
        ki[i] = kept ? ~order_bits(x) : 0xffffffffu;
        vi[i] = (uint32_t)i;
        mine += kept ? 1 : 0;
    }
    const int nc = block_count(mine, scratch);
    if (tid == 0) state[row] = RowState{hd.mv, nc, 0, 0};
}

// Step 4 for one row over its sorted candidates (vals_out: their indices).
constexpr int kFinishThreads = 256;
__global__ __launch_bounds__(kFinishThreads) void sample_finish_kernel(const float* __restrict__ logits, int ldl,
                                                                       float temperature, int top_k, float top_p,
                                                                       Draws draws,
                                                                       const uint32_t* __restrict__ vals_out,
                                                                       double* __restrict__ probs_all,
                                                                       double* __restrict__ prefix_all, int cap,
                                                                       const RowState* __restrict__ state,
                                                                       int32_t* __restrict__ tokens) {
    const int row = blockIdx.x, tid = threadIdx.x;
    const RowState st = state[row];
    if (st.done) return;
    const float* l = logits + (size_t)row * ldl;
    const uint32_t* vo = vals_out + (size_t)row * cap;
    double* probs = probs_all + (size_t)row * cap;
    double* prefix = prefix_all + (size_t)row * cap;
    const float inv_temp = 1.0f / temperature;
    const int cand = top_k > 0 && top_k < st.nc ? top_k : st.nc;
    for (int i = tid; i < cand; i += kFinishThreads) probs[i] = exp((double)(l[vo[i]] - st.mv) * inv_temp);
    __syncthreads();
    pick_token(probs, prefix, cand, top_p, draws.u[row], [&](int i) { return (int)vo[i]; }, tokens + row);
}

// Workspace of the wide path for m rows of n logits: keys and indices in
// and out (4 B each; the ins hold the running sums once sorted), the terms
// (8 B), row states, then the sort's scratch.
struct WideLayout {
    size_t keys_in, vals_in, keys_out, vals_out, probs, state, temp, temp_bytes, total;
};
WideLayout wide_layout(int m, int64_t n) {
    int64_t cap = 1;
    while (cap < n) cap <<= 1;
    WideLayout w{};
    const size_t e = (size_t)m * cap;
    w.keys_in = 0;
    w.vals_in = w.keys_in + e * 4;
    w.keys_out = w.vals_in + e * 4;
    w.vals_out = w.keys_out + e * 4;
    w.probs = w.vals_out + e * 4;
    w.state = w.probs + e * 8;
    w.temp = (w.state + (size_t)m * sizeof(RowState) + 255) / 256 * 256;
    size_t tb = 0;
    if (rocprim::radix_sort_pairs(nullptr, tb, (const uint32_t*)nullptr, (uint32_t*)nullptr, (const uint32_t*)nullptr,
                                  (uint32_t*)nullptr, (unsigned int)n, 0, 32) != hipSuccess)
        tb = 0;
    w.temp_bytes = tb;
    w.total = tb ? w.temp + tb : 0;
    return w;
}

// Whether lyk_hip_sample takes the wide path: more logits than LDS sorts,
// and a cut (top_k) that leaves more than that.
bool wide_path(int64_t n, float temperature, int32_t top_k) {
    return temperature != 0.0f && n > kLdsKeys && (top_k == 0 || top_k >= kLdsKeys);
}

int launch_sample_wide(const float* d_logits, int64_t ldl, int m, int64_t n, float temperature, int32_t top_k,
                       float top_p, const double* u, int32_t* d_tokens, void* ws, hipStream_t stream) {
    Draws d{};
    for (int r = 0; r < m; ++r) {
        if (!(u[r] >= 0.0 && u[r] < 1.0)) return LYK_ERR_INVALID_ARG;
        d.u[r] = u[r];
    }
    const WideLayout w = wide_layout(m, n);
    if (!w.total) return LYK_ERR_HIP;
    int cap = 1;
    while (cap < n) cap <<= 1;
    char* base = static_cast<char*>(ws);
    uint32_t* ki = reinterpret_cast<uint32_t*>(base + w.keys_in);
    uint32_t* vi = reinterpret_cast<uint32_t*>(base + w.vals_in);
    uint32_t* ko = reinterpret_cast<uint32_t*>(base + w.keys_out);
    uint32_t* vo = reinterpret_cast<uint32_t*>(base + w.vals_out);
    double* probs = reinterpret_cast<double*>(base + w.probs);
    RowState* state = reinterpret_cast<RowState*>(base + w.state);
    hipLaunchKernelGGL(sample_prep_kernel, dim3(m), dim3(kSampleThreads), 0, stream, d_logits, (int)ldl, (int)n,
                       temperature, top_k, ki, vi, cap, state, d_tokens);
    LYK_LAUNCH_CHECK();
    for (int r = 0; r < m; ++r) {
        size_t tb = w.temp_bytes;
        if (rocprim::radix_sort_pairs(base + w.temp, tb, ki + (size_t)r * cap, ko + (size_t)r * cap,
                                      vi + (size_t)r * cap, vo + (size_t)r * cap, (unsigned int)n, 0, 32, stream) !=
            hipSuccess)
            return LYK_ERR_LAUNCH;
    }
    hipLaunchKernelGGL(sample_finish_kernel, dim3(m), dim3(kFinishThreads), 0, stream, d_logits, (int)ldl,
                       temperature, top_k, top_p, d, vo, probs, reinterpret_cast<double*>(base + w.keys_in), cap,
                       state, d_tokens);
    LYK_LAUNCH_CHECK();
    return LYK_OK;
}

// Launches sample_kernel over rows [0, m) with the scratch at `ws` (keys,
// then terms, then running sums, m * cap 8-byte entries each; every entry a
// row uses is written before it is read, so the scratch needs no clearing).
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
    double* prefix = reinterpret_cast<double*>(base + (size_t)m * cap * 16);
    static std::once_flag lds_once;
    static bool lds_ok = false;
    std::call_once(lds_once, [] {
        lds_ok = hipFuncSetAttribute((const void*)sample_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     kLdsKeys * 8) == hipSuccess;
    });
    if (!lds_ok) return LYK_ERR_HIP;
    hipLaunchKernelGGL(sample_kernel, dim3(m), dim3(kSampleThreads), kLdsKeys * 8, stream, d_logits, (int)ldl,
                       (int)n, temperature, top_k, top_p, d, keys, probs, prefix, cap, d_tokens);
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
constexpr size_t kStaticScratchBytes = (size_t)kMaxRows * kStaticLogits * 24;   // 24 MiB
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
    if (m < 1 || n < 1 || m > kMaxRows || n > (1 << 30)) return 0;
    int64_t cap = 1;
    while (cap < n) cap <<= 1;
    const uint64_t one = (uint64_t)m * (uint64_t)cap * 24;   // the one-launch path
    if (n <= kLdsKeys) return one;
    const WideLayout w = wide_layout(m, n);
    return w.total > one ? w.total : one;
}

int lyk_hip_sample(const float* d_logits, int64_t ldl, int m, int64_t n, float temperature, int32_t top_k,
                   float top_p, const double* u, int32_t* d_tokens, void* d_workspace, uint64_t workspace_bytes,
                   void* stream) {
    const int rc = check_sample_args(d_logits, ldl, m, n, temperature, top_k, top_p, u, d_tokens);
    if (rc != LYK_OK) return rc;
    if (!d_workspace || workspace_bytes < lyk_hip_sample_workspace_bytes(m, n)) return LYK_ERR_WORKSPACE;
    if (wide_path(n, temperature, top_k))
        return launch_sample_wide(d_logits, ldl, m, n, temperature, top_k, top_p, u, d_tokens, d_workspace,
                                  static_cast<hipStream_t>(stream));
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
