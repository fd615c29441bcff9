// Load-time weight quantization and repacking into the device layouts
// declared in include/lykuro_hip.h. This is the "model/loader" step of the
// hip backend: the reference quantizes at load on the host too
// (WeightBuffer::Quantize, backends/cuda/qwen_cuda_model.cu:1133-1210) but
// keeps plain row-major storage; here rows are tiled 64 to a wave and codes
// reordered so that one 16-byte load per lane feeds one 32-weight group.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "fp16.h"
#include "lykuro_hip.h"

namespace lyk {
namespace {

int worker_count(int64_t rows) {
    unsigned hw = std::thread::hardware_concurrency();
    int n = int(std::min<unsigned>(hw == 0 ? 1u : hw, 16u));
    return int(std::max<int64_t>(1, std::min<int64_t>(n, rows / 64)));
}

// Runs fn(r0, r1) over [0, rows) split across worker threads.
template <class Fn>
void parallel_rows(int64_t rows, Fn fn) {
    const int workers = worker_count(rows);
    if (workers <= 1) {
        fn(int64_t(0), rows);
        return;
    }
    std::vector<std::thread> pool;
    for (int t = 1; t < workers; ++t)
        pool.emplace_back(fn, rows * t / workers, rows * (t + 1) / workers);
    fn(int64_t(0), rows / workers);
    for (auto& th : pool) th.join();
}

int8_t quant_code(float w, float s, float lo, float hi) {
    float r = std::round(w / s);  // ties away from zero
    return int8_t(std::clamp(r, lo, hi));
}

int64_t tiles_of(int64_t n, int paired) {
    return paired ? (n + 31) / 32 : (n + 63) / 64;
}

// Source of packed row `lane` of tile `t`: (matrix 0/1, row), or -1 if padding.
inline int64_t src_row(int64_t t, int lane, int64_t n, int paired, int* which) {
    if (paired) {
        *which = lane >= 32;
        int64_t r = t * 32 + (lane & 31);
        return r < n ? r : -1;
    }
    *which = 0;
    int64_t r = t * 64 + lane;
    return r < n ? r : -1;
}

// Bit position of code j (0..7) within a 32-bit word of the q4 layout.
constexpr int kNibblePos[8] = {0, 16, 4, 20, 8, 24, 12, 28};

// Geometry of the tiled ("step") layouts: tiles of tr rows (paired: tr/2 rows
// of each matrix), lane l of a block holding row l % tr and sub-block l / tr,
// 4 blocks per chunk. unit = k values of one lane's block (32 q4, 16 q8).
struct Tiled {
    int64_t tiles, nb, nc;   // tiles; valid blocks and chunks per tile
    int tr, lpr;
};
constexpr int kChunkBlocks = 4;

bool tiled_of(int64_t n, int64_t k, int paired, int tr, int unit, Tiled* g) {
    if (n <= 0 || k <= 0 || (tr != 16 && tr != 32 && tr != 64)) return false;
    g->tr = tr;
    g->lpr = 64 / tr;
    g->tiles = paired ? (n + tr / 2 - 1) / (tr / 2) : (n + tr - 1) / tr;
    const int64_t units = (k + unit - 1) / unit;
    g->nb = (units + g->lpr - 1) / g->lpr;
    g->nc = (g->nb + kChunkBlocks - 1) / kChunkBlocks;
    return true;
}

// Source row of lane `lane` in tile t: (matrix 0/1, row) or -1 for padding.
inline int64_t tiled_row(const Tiled& g, int64_t t, int lane, int64_t n, int paired, int* which) {
    const int r = lane % g.tr;
    if (paired) {
        *which = r >= g.tr / 2;
        const int64_t row = t * (g.tr / 2) + (r % (g.tr / 2));
        return row < n ? row : -1;
    }
    *which = 0;
    const int64_t row = t * g.tr + r;
    return row < n ? row : -1;
}

}  // namespace
}  // namespace lyk

using namespace lyk;

extern "C" {

int lyk_abi_version(void) { return LYK_ABI_VERSION; }

int lyk_q4_layout(int64_t n, int64_t k, int paired, uint64_t* weight_bytes,
                  uint64_t* scale_bytes) {
    if (n <= 0 || k <= 0 || !weight_bytes || !scale_bytes) return LYK_ERR_INVALID_ARG;
    const int64_t t = tiles_of(n, paired);
    const int64_t chunks = ((k + 31) / 32 + 7) / 8;
    *weight_bytes = uint64_t(t * chunks * 8 * 64 * 16);
    *scale_bytes = uint64_t(t * chunks * 64 * 16);
    return LYK_OK;
}

int lyk_q8_layout(int64_t n, int64_t k, int paired, uint64_t* weight_bytes,
                  uint64_t* scale_bytes) {
    if (n <= 0 || k <= 0 || !weight_bytes || !scale_bytes) return LYK_ERR_INVALID_ARG;
    const int64_t t = tiles_of(n, paired);
    const int64_t chunks = ((k + 15) / 16 + 7) / 8;
    *weight_bytes = uint64_t(t * chunks * 8 * 64 * 16);
    *scale_bytes = uint64_t(t * 64 * 2);
    return LYK_OK;
}

int lyk_q4_quantize(const float* w, int64_t n, int64_t k, int8_t* codes,
                    uint16_t* scales) {
    if (!w || !codes || !scales || n <= 0 || k <= 0) return LYK_ERR_INVALID_ARG;
    const int64_t groups = (k + 31) / 32;
    parallel_rows(n, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            const float* row = w + r * k;
            for (int64_t g = 0; g < groups; ++g) {
                const int64_t k0 = g * 32, k1 = std::min(k, k0 + 32);
                float absmax = 0.0f;
                for (int64_t i = k0; i < k1; ++i) absmax = std::max(absmax, std::fabs(row[i]));
                const uint16_t sh = quant_scale_f16(absmax, 7.0f);
                scales[r * groups + g] = sh;
                const float s = f16_to_f32(sh);
                for (int64_t i = k0; i < k1; ++i)
                    codes[r * k + i] = quant_code(row[i], s, -8.0f, 7.0f);
            }
        }
    });
    return LYK_OK;
}

int lyk_q8_quantize(const float* w, int64_t n, int64_t k, int8_t* codes,
                    uint16_t* scales) {
    if (!w || !codes || !scales || n <= 0 || k <= 0) return LYK_ERR_INVALID_ARG;
    parallel_rows(n, [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; ++r) {
            const float* row = w + r * k;
            float absmax = 0.0f;
            for (int64_t i = 0; i < k; ++i) absmax = std::max(absmax, std::fabs(row[i]));
            const uint16_t sh = quant_scale_f16(absmax, 127.0f);
            scales[r] = sh;
            const float s = f16_to_f32(sh);
            for (int64_t i = 0; i < k; ++i) codes[r * k + i] = quant_code(row[i], s, -127.0f, 127.0f);
        }
    });
    return LYK_OK;
}

int lyk_q4_pack(const int8_t* codes, const uint16_t* scales,
                const int8_t* b_codes, const uint16_t* b_scales, int64_t n,
                int64_t k, void* qw, void* qs) {
    const int paired = b_codes != nullptr;
    if (!codes || !scales || !qw || !qs || n <= 0 || k <= 0) return LYK_ERR_INVALID_ARG;
    if (paired && !b_scales) return LYK_ERR_INVALID_ARG;
    const int64_t T = tiles_of(n, paired);
    const int64_t groups = (k + 31) / 32;
    const int64_t chunks = (groups + 7) / 8, Gp = chunks * 8;
    uint32_t* wout = static_cast<uint32_t*>(qw);
    uint16_t* sout = static_cast<uint16_t*>(qs);
    parallel_rows(T, [&](int64_t t0, int64_t t1) {
        for (int64_t t = t0; t < t1; ++t) {
            for (int lane = 0; lane < 64; ++lane) {
                int which = 0;
                const int64_t r = src_row(t, lane, n, paired, &which);
                const int8_t* crow = r < 0 ? nullptr : (which ? b_codes : codes) + r * k;
                const uint16_t* srow = r < 0 ? nullptr : (which ? b_scales : scales) + r * groups;
                for (int64_t g = 0; g < Gp; ++g) {
                    uint32_t* dst = wout + ((t * Gp + g) * 64 + lane) * 4;
                    for (int d = 0; d < 4; ++d) {
                        uint32_t word = 0;
                        for (int j = 0; j < 8; ++j) {
                            const int64_t kk = g * 32 + d * 8 + j;
                            const int q = (crow && kk < k) ? crow[kk] : 0;
                            word |= uint32_t(q + 8) << kNibblePos[j];
                        }
                        dst[d] = word;
                    }
                }
                for (int64_t c = 0; c < chunks; ++c)
                    for (int j = 0; j < 8; ++j) {
                        const int64_t g = c * 8 + j;
                        sout[((t * chunks + c) * 64 + lane) * 8 + j] =
                            (srow && g < groups) ? srow[g] : uint16_t(0);
                    }
            }
        }
    });
    return LYK_OK;
}

int lyk_q8_pack(const int8_t* codes, const uint16_t* scales,
                const int8_t* b_codes, const uint16_t* b_scales, int64_t n,
                int64_t k, void* qw, void* qs) {
    const int paired = b_codes != nullptr;
    if (!codes || !scales || !qw || !qs || n <= 0 || k <= 0) return LYK_ERR_INVALID_ARG;
    if (paired && !b_scales) return LYK_ERR_INVALID_ARG;
    const int64_t T = tiles_of(n, paired);
    const int64_t blocks = (k + 15) / 16;
    const int64_t Bp = (blocks + 7) / 8 * 8;
    uint8_t* wout = static_cast<uint8_t*>(qw);
    uint16_t* sout = static_cast<uint16_t*>(qs);
    parallel_rows(T, [&](int64_t t0, int64_t t1) {
        for (int64_t t = t0; t < t1; ++t) {
            for (int lane = 0; lane < 64; ++lane) {
                int which = 0;
                const int64_t r = src_row(t, lane, n, paired, &which);
                const int8_t* crow = r < 0 ? nullptr : (which ? b_codes : codes) + r * k;
                for (int64_t b = 0; b < Bp; ++b) {
                    uint8_t* dst = wout + ((t * Bp + b) * 64 + lane) * 16;
                    for (int j = 0; j < 16; ++j) {
                        const int64_t kk = b * 16 + j;
                        const int q = (crow && kk < k) ? crow[kk] : 0;
                        dst[j] = uint8_t(q + 128);
                    }
                }
                sout[t * 64 + lane] = r < 0 ? uint16_t(0) : (which ? b_scales : scales)[r];
            }
        }
    });
    return LYK_OK;
}

int lyk_q4_layout_tiled(int64_t n, int64_t k, int paired, int tile_rows,
                        uint64_t* weight_bytes, uint64_t* scale_bytes) {
    Tiled g;
    if (!weight_bytes || !scale_bytes || !tiled_of(n, k, paired, tile_rows, 32, &g)) return LYK_ERR_INVALID_ARG;
    *weight_bytes = uint64_t(g.tiles * g.nc * kChunkBlocks * 64 * 16);
    *scale_bytes = uint64_t(g.tiles * g.nc * 64 * kChunkBlocks * 2);
    return LYK_OK;
}

int lyk_q8_layout_tiled(int64_t n, int64_t k, int paired, int tile_rows,
                        uint64_t* weight_bytes, uint64_t* scale_bytes) {
    Tiled g;
    if (!weight_bytes || !scale_bytes || !tiled_of(n, k, paired, tile_rows, 16, &g)) return LYK_ERR_INVALID_ARG;
    *weight_bytes = uint64_t(g.tiles * g.nc * kChunkBlocks * 64 * 16);
    *scale_bytes = uint64_t(g.tiles * 64 * 2);
    return LYK_OK;
}

int lyk_q4_pack_tiled(const int8_t* codes, const uint16_t* scales,
                      const int8_t* b_codes, const uint16_t* b_scales, int64_t n,
                      int64_t k, int tile_rows, void* qw, void* qs) {
    const int paired = b_codes != nullptr;
    Tiled g;
    if (!codes || !scales || !qw || !qs || !tiled_of(n, k, paired, tile_rows, 32, &g)) return LYK_ERR_INVALID_ARG;
    if (paired && !b_scales) return LYK_ERR_INVALID_ARG;
    const int64_t groups = (k + 31) / 32, NBp = g.nc * kChunkBlocks;
    uint32_t* wout = static_cast<uint32_t*>(qw);
    uint16_t* sout = static_cast<uint16_t*>(qs);
    parallel_rows(g.tiles * 64, [&](int64_t i0, int64_t i1) {
        for (int64_t i = i0; i < i1; ++i) {
            const int64_t t = i / 64;
            const int lane = int(i % 64), sub = lane / g.tr;
            int which = 0;
            const int64_t r = tiled_row(g, t, lane, n, paired, &which);
            const int8_t* crow = r < 0 ? nullptr : (which ? b_codes : codes) + r * k;
            const uint16_t* srow = r < 0 ? nullptr : (which ? b_scales : scales) + r * groups;
            for (int64_t b = 0; b < NBp; ++b) {
                const int64_t grp = b * g.lpr + sub;   // this lane's group in block b
                uint32_t* dst = wout + ((t * NBp + b) * 64 + lane) * 4;
                for (int d = 0; d < 4; ++d) {
                    uint32_t word = 0;
                    for (int j = 0; j < 8; ++j) {
                        const int64_t kk = grp * 32 + d * 8 + j;
                        const int q = (crow && kk < k) ? crow[kk] : 0;
                        word |= uint32_t(q + 8) << kNibblePos[j];
                    }
                    dst[d] = word;
                }
                sout[((t * g.nc + b / kChunkBlocks) * 64 + lane) * kChunkBlocks + b % kChunkBlocks] =
                    (srow && grp < groups) ? srow[grp] : uint16_t(0);
            }
        }
    });
    return LYK_OK;
}

int lyk_q8_pack_tiled(const int8_t* codes, const uint16_t* scales,
                      const int8_t* b_codes, const uint16_t* b_scales, int64_t n,
                      int64_t k, int tile_rows, void* qw, void* qs) {
    const int paired = b_codes != nullptr;
    Tiled g;
    if (!codes || !scales || !qw || !qs || !tiled_of(n, k, paired, tile_rows, 16, &g)) return LYK_ERR_INVALID_ARG;
    if (paired && !b_scales) return LYK_ERR_INVALID_ARG;
    const int64_t NBp = g.nc * kChunkBlocks;
    uint8_t* wout = static_cast<uint8_t*>(qw);
    uint16_t* sout = static_cast<uint16_t*>(qs);
    parallel_rows(g.tiles * 64, [&](int64_t i0, int64_t i1) {
        for (int64_t i = i0; i < i1; ++i) {
            const int64_t t = i / 64;
            const int lane = int(i % 64), sub = lane / g.tr;
            int which = 0;
            const int64_t r = tiled_row(g, t, lane, n, paired, &which);
            const int8_t* crow = r < 0 ? nullptr : (which ? b_codes : codes) + r * k;
            for (int64_t b = 0; b < NBp; ++b) {
                const int64_t kb = b * g.lpr + sub;   // this lane's 16-k block
                uint8_t* dst = wout + ((t * NBp + b) * 64 + lane) * 16;
                for (int j = 0; j < 16; ++j) {
                    const int64_t kk = kb * 16 + j;
                    const int q = (crow && kk < k) ? crow[kk] : 0;
                    dst[j] = uint8_t(q + 128);
                }
            }
            sout[t * 64 + lane] = r < 0 ? uint16_t(0) : (which ? b_scales : scales)[r];
        }
    });
    return LYK_OK;
}

int lyk_q4_unpack_tiled(const void* qw, const void* qs, int64_t n, int64_t k, int paired,
                        int tile_rows, int8_t* codes, uint16_t* scales) {
    Tiled g;
    if (!qw || !qs || !codes || !scales || !tiled_of(n, k, paired, tile_rows, 32, &g)) return LYK_ERR_INVALID_ARG;
    const int64_t groups = (k + 31) / 32, NBp = g.nc * kChunkBlocks;
    const uint32_t* win = static_cast<const uint32_t*>(qw);
    const uint16_t* sin = static_cast<const uint16_t*>(qs);
    for (int64_t t = 0; t < g.tiles; ++t)
        for (int lane = 0; lane < 64; ++lane) {
            int which = 0;
            const int64_t r = tiled_row(g, t, lane, n, paired, &which);
            if (r < 0) continue;
            const int64_t row = r + (which ? n : 0), sub = lane / g.tr;
            for (int64_t b = 0; b < NBp; ++b) {
                const int64_t grp = b * g.lpr + sub;
                if (grp >= groups) continue;
                const uint32_t* src = win + ((t * NBp + b) * 64 + lane) * 4;
                for (int d = 0; d < 4; ++d)
                    for (int j = 0; j < 8; ++j) {
                        const int64_t kk = grp * 32 + d * 8 + j;
                        if (kk < k) codes[row * k + kk] = int8_t(int((src[d] >> kNibblePos[j]) & 15u) - 8);
                    }
                scales[row * groups + grp] = sin[((t * g.nc + b / kChunkBlocks) * 64 + lane) * kChunkBlocks + b % kChunkBlocks];
            }
        }
    return LYK_OK;
}

int lyk_q8_unpack_tiled(const void* qw, const void* qs, int64_t n, int64_t k, int paired,
                        int tile_rows, int8_t* codes, uint16_t* scales) {
    Tiled g;
    if (!qw || !qs || !codes || !scales || !tiled_of(n, k, paired, tile_rows, 16, &g)) return LYK_ERR_INVALID_ARG;
    const int64_t NBp = g.nc * kChunkBlocks, kblocks = (k + 15) / 16;
    const uint8_t* win = static_cast<const uint8_t*>(qw);
    const uint16_t* sin = static_cast<const uint16_t*>(qs);
    for (int64_t t = 0; t < g.tiles; ++t)
        for (int lane = 0; lane < 64; ++lane) {
            int which = 0;
            const int64_t r = tiled_row(g, t, lane, n, paired, &which);
            if (r < 0) continue;
            const int64_t row = r + (which ? n : 0), sub = lane / g.tr;
            for (int64_t b = 0; b < NBp; ++b) {
                const int64_t kb = b * g.lpr + sub;
                if (kb >= kblocks) continue;
                const uint8_t* src = win + ((t * NBp + b) * 64 + lane) * 16;
                for (int j = 0; j < 16; ++j) {
                    const int64_t kk = kb * 16 + j;
                    if (kk < k) codes[row * k + kk] = int8_t(int(src[j]) - 128);
                }
            }
            scales[row] = sin[t * 64 + lane];
        }
    return LYK_OK;
}

}  // extern "C"
