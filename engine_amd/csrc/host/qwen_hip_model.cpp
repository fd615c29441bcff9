// QwenHipModel: host side of the MI355X hip backend (C++20). Owns device
// memory, the paged KV pool and the decode step; every device computation is
// a call into the gfx950 kernel library through include/lykuro_hip.h.
//
// Contract followed (reference paths): GenerativeModel
// (model/architectures/generative_model.h:40-105); error semantics of
// QwenModel / QwenCudaModel Prefill, Decode, DecodeBatch and GreedyRun
// (model/architectures/qwen/qwen_model.cpp:333-412,
// backends/cuda/qwen_cuda_model.cu:2518-2660, 2641-2776, 2778-3102); paged
// pool and prefix cache (qwen_cuda_model.cu:1623-1749, 1913-2008,
// 2545-2608).
#include "qwen_hip_model.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <thread>
#include <unordered_map>

#include "fp16.h"
#include "kv_pool.h"
#include "lykuro_hip.h"
#include "lykuro_hip_model.h"

namespace lykuro::nie {

namespace {

constexpr const char kComponent[] = "qwen_hip";
constexpr int kMaxBatch = 4;          // rows per fused step (lyk_hip_decode_step limit)
// prompt rows per prefill chunk pass by default: a 2048-token prompt in one
// pass fills the grid in every GEMM (measured at 7B: 256 rows 320 ms, 1024
// rows 110 ms, 2048 rows 79 ms to the first token); chunk sizes do not change
// the results (no row's arithmetic depends on its chunk)
constexpr uint32_t kDefaultChunkRows = 2048;
constexpr uint32_t kGreedyMax = 256;  // greedy steps per GreedyRun call

Status HipFail(hipError_t err, const char* what) {
    if (err == hipErrorOutOfMemory || err == hipErrorMemoryAllocation)
        return Status(ErrorCode::kGpuOom, what, kComponent);
    return Status(ErrorCode::kGpuUnhealthy, what, kComponent);
}

Status KernelFail(int rc, const char* what) {
    if (rc == LYK_ERR_SHAPE) return Status(ErrorCode::kUnsupportedModel, what, kComponent);
    return Status(ErrorCode::kGpuUnhealthy, what, kComponent).WithDetail("lyk_status", rc);
}

#define HIP_OK(expr, what)                                \
    do {                                                  \
        hipError_t e_ = (expr);                           \
        if (e_ != hipSuccess) return HipFail(e_, what);   \
    } while (0)

#define LYK_OK_OR(expr, what)                          \
    do {                                               \
        int rc_ = (expr);                              \
        if (rc_ != LYK_OK) return KernelFail(rc_, what); \
    } while (0)

int64_t RoundUp(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) {
        o.p = nullptr;
        o.bytes = 0;
    }
    DevBuf& operator=(DevBuf&& o) noexcept {
        if (this != &o) {
            Free();
            p = o.p;
            bytes = o.bytes;
            o.p = nullptr;
            o.bytes = 0;
        }
        return *this;
    }
    ~DevBuf() { Free(); }
    void Free() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    Status Alloc(size_t n, bool zero = true) {
        Free();
        HIP_OK(hipMalloc(&p, n ? n : 1), "device allocation failed");
        bytes = n;
        if (zero) HIP_OK(hipMemset(p, 0, n ? n : 1), "device memset failed");
        return Status::Ok();
    }
    Status Upload(const void* src, size_t n) {
        Status s = Alloc(n, false);
        if (!s.ok()) return s;
        HIP_OK(hipMemcpy(p, src, n, hipMemcpyHostToDevice), "weight upload failed");
        return Status::Ok();
    }
    template <class T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

struct PinnedBuf {
    void* p = nullptr;
    ~PinnedBuf() {
        if (p) (void)hipHostFree(p);
    }
    Status Alloc(size_t n) {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        HIP_OK(hipHostMalloc(&p, n ? n : 1, hipHostMallocDefault), "pinned allocation failed");
        return Status::Ok();
    }
    template <class T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

struct PackedMat {
    DevBuf qw, qs;
    int64_t n = 0, k = 0;
    bool paired = false;
    int tile_rows = 64;   // tiled layout height (lyk_q*_pack_tiled)
};

// A sequence's KV blocks and length. It shares ownership of the pool, so a
// sequence may outlive its model; its blocks go back to the pool when it is
// destroyed or cleared.
class HipSequenceState final : public SequenceState {
public:
    HipSequenceState(std::shared_ptr<hip::KvBlockPool> pool, uint32_t max_tokens, SequenceOptions options)
        : pool_(std::move(pool)), max_tokens_(max_tokens), options_(std::move(options)) {}
    ~HipSequenceState() override { Clear(); }
    uint32_t length() const override { return length_; }
    uint32_t capacity() const override { return max_tokens_; }
    const SequenceOptions& options() const { return options_; }
    const std::vector<int32_t>& blocks() const { return blocks_; }

    // Blocks for the first `tokens` positions (capacity_exhausted when the
    // pool has none left; blocks taken so far are kept).
    Status Reserve(uint32_t tokens) {
        const uint32_t bt = pool_->block_tokens();
        while (size_t(blocks_.size()) * bt < tokens) {
            const std::optional<int32_t> b = pool_->Take();
            if (!b) return Status(ErrorCode::kCapacityExhausted, "kv block pool exhausted", kComponent);
            blocks_.push_back(*b);
        }
        return Status::Ok();
    }
    // Starts from cached blocks (each already holding a reference for this
    // sequence) that cover the first `tokens` positions.
    void Adopt(std::vector<int32_t> cached, uint32_t tokens) {
        Clear();
        blocks_ = std::move(cached);
        length_ = tokens;
    }
    // Back to an empty sequence.
    void Clear() {
        for (int32_t b : blocks_) pool_->Drop(b);
        blocks_.clear();
        length_ = 0;
    }
    void Advance(uint32_t n) { length_ += n; }

private:
    std::shared_ptr<hip::KvBlockPool> pool_;
    uint32_t max_tokens_;
    uint32_t length_ = 0;
    SequenceOptions options_;
    std::vector<int32_t> blocks_;
};

// Tensor kinds of the synthetic generator's stream ids (kind*1000 + layer).
enum Kind {
    kEmbed = 0, kInputNorm, kQW, kQB, kKW, kKB, kVW, kVB, kOW, kPostNorm, kGateW, kUpW, kDownW,
    kFinalNorm, kLmHead
};

std::string LayerName(uint32_t l, const char* suffix) {
    return "model.layers." + std::to_string(l) + "." + suffix;
}

}  // namespace

// ------------------------------------------------------------ weight sources

Status SafetensorsWeightSource::Read(const std::string& name, const std::vector<uint64_t>& shape,
                                     std::vector<float>& out) const {
    const TensorInfo* info = file_.FindTensor(name);
    const uint8_t* data = file_.TensorData(name);
    if (info == nullptr || data == nullptr)
        return Status(ErrorCode::kArtifactVerificationFailed, "expected weight tensor missing", kComponent);
    if (info->shape != shape)
        return Status(ErrorCode::kArtifactVerificationFailed, "weight tensor shape mismatch", kComponent);
    out.resize(info->element_count);
    const uint16_t* h = reinterpret_cast<const uint16_t*>(data);
    switch (info->dtype) {
        case Dtype::kF32: std::memcpy(out.data(), data, info->data_size); break;
        case Dtype::kF16:
            for (uint64_t i = 0; i < info->element_count; ++i) out[i] = lyk::f16_to_f32(h[i]);
            break;
        case Dtype::kBf16:
            for (uint64_t i = 0; i < info->element_count; ++i) out[i] = lyk::bf16_to_f32(h[i]);
            break;
        default:
            return Status(ErrorCode::kArtifactVerificationFailed, "weight tensor is not floating point", kComponent);
    }
    return Status::Ok();
}

Status SafetensorsWeightSource::ReadQuantized(const std::string& base, bool q8, int64_t n, int64_t k,
                                              std::vector<int8_t>& codes, std::vector<uint16_t>& scales,
                                              bool& found) const {
    found = false;
    const TensorInfo* w = file_.FindTensor(base + ".qweight");
    const TensorInfo* s = file_.FindTensor(base + ".qscale");
    if (w == nullptr && s == nullptr) return Status::Ok();
    if (w == nullptr || s == nullptr)
        return Status(ErrorCode::kArtifactVerificationFailed, "quantized weight without its scales", kComponent);
    // int4: U8 [n][ceil(k/2)], code + 8 per nibble, even k in the low nibble,
    // fp16 scales [n][ceil(k/32)]; int8: I8 [n][k], fp16 scales [n]
    const bool is_q8 = w->dtype == Dtype::kI8;
    if ((w->dtype != Dtype::kU8 && w->dtype != Dtype::kI8) || s->dtype != Dtype::kF16)
        return Status(ErrorCode::kArtifactVerificationFailed, "quantized weight dtypes invalid", kComponent);
    if (is_q8 != q8)
        return Status(ErrorCode::kUnsupportedModel, "artifact quantization differs from the model options", kComponent);
    const std::vector<uint64_t> wshape = {uint64_t(n), uint64_t(q8 ? k : (k + 1) / 2)};
    const std::vector<uint64_t> sshape = q8 ? std::vector<uint64_t>{uint64_t(n)}
                                            : std::vector<uint64_t>{uint64_t(n), uint64_t((k + 31) / 32)};
    if (w->shape != wshape || s->shape != sshape)
        return Status(ErrorCode::kArtifactVerificationFailed, "quantized weight shape mismatch", kComponent);
    const uint8_t* wd = file_.TensorData(base + ".qweight");
    const uint8_t* sd = file_.TensorData(base + ".qscale");
    codes.resize(size_t(n * k));
    scales.resize(s->element_count);
    std::memcpy(scales.data(), sd, s->data_size);
    if (q8) {
        std::memcpy(codes.data(), wd, size_t(n * k));
    } else {
        const int64_t kb = (k + 1) / 2;
        for (int64_t r = 0; r < n; ++r)
            for (int64_t i = 0; i < k; ++i) {
                const uint8_t byte = wd[r * kb + i / 2];
                codes[size_t(r * k + i)] = int8_t(int((i & 1) ? byte >> 4 : byte & 15) - 8);
            }
    }
    found = true;
    return Status::Ok();
}

Status SyntheticWeightSource::Read(const std::string& name, const std::vector<uint64_t>& shape,
                                   std::vector<float>& out) const {
    uint64_t count = 1;
    for (uint64_t d : shape) count *= d;
    out.resize(count);
    if (name.find("norm") != std::string::npos) {
        std::fill(out.begin(), out.end(), 1.0f);
        return Status::Ok();
    }
    int kind = -1;
    uint32_t layer = 0;
    if (name == "model.embed_tokens.weight") kind = kEmbed;
    else if (name == "lm_head.weight") kind = kLmHead;
    else {
        static const std::pair<const char*, int> kLayer[] = {
            {"self_attn.q_proj.weight", kQW}, {"self_attn.q_proj.bias", kQB},
            {"self_attn.k_proj.weight", kKW}, {"self_attn.k_proj.bias", kKB},
            {"self_attn.v_proj.weight", kVW}, {"self_attn.v_proj.bias", kVB},
            {"self_attn.o_proj.weight", kOW}, {"mlp.gate_proj.weight", kGateW},
            {"mlp.up_proj.weight", kUpW},     {"mlp.down_proj.weight", kDownW}};
        const std::string prefix = "model.layers.";
        if (name.rfind(prefix, 0) == 0) {
            const size_t dot = name.find('.', prefix.size());
            layer = uint32_t(std::stoul(name.substr(prefix.size(), dot - prefix.size())));
            const std::string suffix = name.substr(dot + 1);
            for (const auto& [s, k] : kLayer)
                if (suffix == s) kind = k;
        }
    }
    if (kind < 0)
        return Status(ErrorCode::kArtifactVerificationFailed, "expected weight tensor missing", kComponent);
    const uint64_t stream = uint64_t(kind) * 1000 + layer;
    const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    const uint64_t workers = count < (1u << 20) ? 1 : hw;
    std::vector<std::thread> pool;
    for (uint64_t t = 1; t < workers; ++t) {
        const uint64_t a = count * t / workers, b = count * (t + 1) / workers;
        pool.emplace_back([this, stream, a, b, &out] { lyk_synth_normal(seed_, stream, a, b - a, sigma_, out.data() + a); });
    }
    lyk_synth_normal(seed_, stream, 0, count / workers, sigma_, out.data());
    for (auto& th : pool) th.join();
    return Status::Ok();
}

// ------------------------------------------------------------------- config

Status HipQwenConfig::FromManifest(const ModelManifest& m, HipQwenConfig& out) {
    auto fail = [](const char* msg) {
        return Status(ErrorCode::kArtifactVerificationFailed, msg, kComponent);
    };
    out.vocab_size = m.vocab_size;
    out.hidden_size = m.hidden_size;
    out.num_layers = m.num_layers;
    out.num_heads = m.num_attention_heads;
    out.num_kv_heads = m.num_key_value_heads;
    out.head_dim = m.head_dim;
    out.intermediate_size = m.intermediate_size;
    out.max_context_tokens = m.max_context_tokens;
    out.rms_norm_eps = m.rms_norm_eps > 0 ? float(m.rms_norm_eps) : 1e-6f;
    out.rope_theta = m.rope_theta > 0 ? float(m.rope_theta) : 10000.0f;
    out.tie_word_embeddings = m.tie_word_embeddings;
    out.eos_token_ids = m.eos_token_ids;
    if (out.intermediate_size == 0) return fail("manifest missing intermediate_size");
    if (out.head_dim % 2 != 0) return fail("head_dim must be even for RoPE");
    if (out.num_kv_heads == 0 || out.num_heads % out.num_kv_heads != 0)
        return fail("attention head configuration inconsistent");
    if (out.eos_token_ids.empty()) return fail("manifest missing eos_token_ids");
    for (uint32_t id : out.eos_token_ids)
        if (id >= out.vocab_size) return fail("eos token id out of vocab range");
    return Status::Ok();
}

// --------------------------------------------------------------------- impl

struct QwenHipModel::Impl {
    struct Layer {
        DevBuf input_norm, post_norm, qkv_bias;
        PackedMat qkv, o, gateup, down;
    };

    HipModelOptions opt;
    HipQwenConfig c;
    hipStream_t stream = nullptr;
    bool q8 = false;

    DevBuf embed, final_norm;
    PackedMat lm_head;
    std::vector<Layer> layers;

    std::shared_ptr<hip::KvBlockPool> pool;
    DevBuf kv;  // [layer][K|V][num_blocks][nkv][bt][hd] fp16
    size_t kv_layer_elems = 0;

    DevBuf rcos, rsin;
    uint32_t rope_cap = 0, table_stride = 0;

    // fused step: model description, its device layer table and workspace
    lyk_step_model md{};
    DevBuf d_layers, d_step_ws;
    uint64_t step_ws_bytes = 0;

    // per-step rows (kMaxBatch)
    DevBuf d_tokens, d_pos, d_tables, d_logits, d_history, d_step, d_nonfinite, d_prompt;
    PinnedBuf h_tokens, h_pos, h_tables, h_logits, h_history, h_nonfinite, h_prompt;
    size_t prompt_cap = 0;

    // chunk prefill: prompt rows per pass (0: off) and the pass's buffers
    uint32_t chunk_rows = 0;
    DevBuf pf_x, pf_xn, pf_qkv, pf_q, pf_attn, pf_act;

    uint64_t prefix_hits = 0;
    uint64_t gemv_bytes = 0;
    bool tracing = false;
    DevBuf d_trace;  // phase timestamps of the last step (when tracing)

    ~Impl() {
        if (stream) (void)hipStreamDestroy(stream);
    }

    uint16_t* kcache(uint32_t l) const { return kv.as<uint16_t>() + (size_t)l * 2 * kv_layer_elems; }
    uint16_t* vcache(uint32_t l) const { return kcache(l) + kv_layer_elems; }

    // cos/sin tables and block-table stride for positions < cap; rebuilt
    // when a longer sequence is created.
    Status EnsureRope(uint32_t cap) {
        if (cap <= rope_cap) return Status::Ok();
        const uint32_t half = c.head_dim / 2;
        std::vector<float> cs((size_t)cap * half), sn((size_t)cap * half);
        for (uint32_t i = 0; i < half; ++i) {
            // the CPU reference's expressions (qwen_model.cpp:45-48), in float
            const float freq = std::pow(c.rope_theta, -2.0f * float(i) / float(c.head_dim));
            for (uint32_t p = 0; p < cap; ++p) {
                const float angle = float(p) * freq;
                cs[(size_t)p * half + i] = std::cos(angle);
                sn[(size_t)p * half + i] = std::sin(angle);
            }
        }
        HIP_OK(hipStreamSynchronize(stream), "device execution failed");
        Status s = rcos.Upload(cs.data(), cs.size() * 4);
        if (!s.ok()) return s;
        s = rsin.Upload(sn.data(), sn.size() * 4);
        if (!s.ok()) return s;
        rope_cap = cap;
        md.rope_cos = rcos.as<float>();
        md.rope_sin = rsin.as<float>();
        md.rope_positions = int32_t(cap);
        table_stride = std::max<uint32_t>(1, (cap + pool->block_tokens() - 1) / pool->block_tokens());
        s = d_tables.Alloc((size_t)kMaxBatch * table_stride * 4);
        if (!s.ok()) return s;
        return h_tables.Alloc((size_t)kMaxBatch * table_stride * 4);
    }

    // One fused decode step for rows 0..m-1 whose token, position and block
    // table are already on the device.
    Status LaunchStep(int m, int mode) {
        lyk_step_io io{};
        io.m = m;
        io.mode = mode;
        io.tokens = d_tokens.as<int32_t>();
        io.positions = d_pos.as<int32_t>();
        io.block_tables = d_tables.as<int32_t>();
        io.table_stride = int32_t(table_stride);
        io.logits = d_logits.as<float>();
        io.ld_logits = c.vocab_size;
        if (tracing) io.trace = d_trace.as<uint64_t>();
        if (mode == LYK_STEP_GREEDY) {
            io.nonfinite = d_nonfinite.as<int32_t>();
            io.history = d_history.as<int32_t>();
            io.step = d_step.as<int32_t>();
        }
        LYK_OK_OR(lyk_hip_decode_step(&md, &io, d_step_ws.p, step_ws_bytes, kMaxBatch, stream),
                  "decode step launch failed");
        return Status::Ok();
    }

    // After a stream synchronization: a step that could not complete leaves
    // an error word in the workspace; reset it so later steps can run.
    Status CheckSteps() {
        int32_t err = 0;
        LYK_OK_OR(lyk_hip_step_error(d_step_ws.p, &err, stream), "decode step status read failed");
        if (err != 0) {
            (void)lyk_hip_step_reset(d_step_ws.p, step_ws_bytes, stream);
            (void)hipStreamSynchronize(stream);
            return Status(ErrorCode::kGpuUnhealthy, "decode step did not complete on the device", kComponent);
        }
        return Status::Ok();
    }

    // One chunk pass over T prompt rows of one sequence (token ids on the
    // device at d_tok, positions pos0..pos0+T-1, its block table in row 0 of
    // d_tables, table_len blocks): per layer RMSNorm, the QKV GEMM (+ bias),
    // RoPE with the K/V append, causal chunk attention, the o GEMM into the
    // residual, RMSNorm, the gate/up GEMM with SiLU, the down GEMM into the
    // residual (ForwardChunk, qwen_cuda_model.cu:2398-2516). The last layer
    // stops after its K/V append: only the prompt's last token, which the
    // fused step runs, needs the hidden state past it.
    Status ChunkPass(const int32_t* d_tok, int T, int pos0, int table_len) {
        const int H = int(c.hidden_size), nq = int(c.num_heads), nkv = int(c.num_kv_heads), hd = int(c.head_dim);
        const int In = int(c.intermediate_size), kq = nq * hd, rows = (nq + 2 * nkv) * hd;
        const int bt = int(pool->block_tokens()), nb = int(pool->num_blocks()), qi = q8 ? 1 : 0;
        const float eps = c.rms_norm_eps;
        float* X = pf_x.as<float>();
        uint16_t* Xn = pf_xn.as<uint16_t>();
        LYK_OK_OR(lyk_hip_embed_rmsnorm(embed.as<float>(), c.vocab_size, d_tok, T, H, X, H,
                                        layers[0].input_norm.as<float>(), eps, Xn, H, stream),
                  "prefill embedding failed");
        for (uint32_t l = 0; l < c.num_layers; ++l) {
            const Layer& L = layers[l];
            if (l > 0)
                LYK_OK_OR(lyk_hip_rmsnorm_f16(X, H, L.input_norm.as<float>(), eps, T, H, Xn, H, stream),
                          "prefill norm failed");
            LYK_OK_OR(lyk_hip_gemm_q(Xn, H, T, H, L.qkv.qw.p, L.qkv.qs.p, rows, L.qkv.tile_rows, qi, LYK_GEMM_STORE,
                                     L.qkv_bias.as<float>(), pf_qkv.p, rows, stream),
                      "prefill qkv GEMM failed");
            LYK_OK_OR(lyk_hip_chunk_rope_kv(pf_qkv.as<float>(), rows, T, pos0, nq, nkv, hd, rcos.as<float>(),
                                            rsin.as<float>(), int(rope_cap), pf_q.as<float>(), kcache(l), vcache(l),
                                            d_tables.as<int32_t>(), table_len, bt, nb, stream),
                      "prefill RoPE / KV append failed");
            if (l + 1 == c.num_layers) break;
            LYK_OK_OR(lyk_hip_chunk_attention(pf_q.as<float>(), kcache(l), vcache(l), d_tables.as<int32_t>(),
                                              table_len, T, pos0, nq, nkv, hd, bt, nb, pf_attn.as<uint16_t>(), kq,
                                              stream),
                      "prefill attention failed");
            LYK_OK_OR(lyk_hip_gemm_q(pf_attn.as<uint16_t>(), kq, T, kq, L.o.qw.p, L.o.qs.p, H, L.o.tile_rows, qi,
                                     LYK_GEMM_ADD, nullptr, X, H, stream),
                      "prefill o GEMM failed");
            LYK_OK_OR(lyk_hip_rmsnorm_f16(X, H, L.post_norm.as<float>(), eps, T, H, Xn, H, stream),
                      "prefill norm failed");
            LYK_OK_OR(lyk_hip_gemm_q(Xn, H, T, H, L.gateup.qw.p, L.gateup.qs.p, In, L.gateup.tile_rows, qi,
                                     LYK_GEMM_SILU_PAIRS, nullptr, pf_act.p, In, stream),
                      "prefill gate/up GEMM failed");
            LYK_OK_OR(lyk_hip_gemm_q(pf_act.as<uint16_t>(), In, T, In, L.down.qw.p, L.down.qs.p, H, L.down.tile_rows,
                                     qi, LYK_GEMM_ADD, nullptr, X, H, stream),
                      "prefill down GEMM failed");
        }
        return Status::Ok();
    }

    // Uploads tokens, positions and block tables of up to kMaxBatch rows.
    Status UploadRows(const std::vector<HipSequenceState*>& seqs, const std::vector<uint32_t>& tokens,
                      const std::vector<uint32_t>& positions) {
        const size_t m = seqs.size();
        int32_t* ht = h_tokens.as<int32_t>();
        int32_t* hp = h_pos.as<int32_t>();
        int32_t* tb = h_tables.as<int32_t>();
        for (size_t i = 0; i < m; ++i) {
            ht[i] = int32_t(tokens[i]);
            hp[i] = int32_t(positions[i]);
            const auto& blocks = seqs[i]->blocks();
            std::copy(blocks.begin(), blocks.end(), tb + i * table_stride);
        }
        HIP_OK(hipMemcpyAsync(d_tokens.p, ht, m * 4, hipMemcpyHostToDevice, stream), "token upload failed");
        HIP_OK(hipMemcpyAsync(d_pos.p, hp, m * 4, hipMemcpyHostToDevice, stream), "position upload failed");
        HIP_OK(hipMemcpyAsync(d_tables.p, tb, m * table_stride * 4, hipMemcpyHostToDevice, stream),
               "block table upload failed");
        return Status::Ok();
    }
};

// --------------------------------------------------------------------- load

namespace {

// Codes and fp16 scales of an [n, k] fp32 matrix by the load-time quantizer
// (int4: groups of 32 along k; int8: per row).
Status Quantize(bool q8, const std::vector<float>& w, int64_t n, int64_t k, std::vector<int8_t>& codes,
                std::vector<uint16_t>& scales) {
    codes.resize(size_t(n * k));
    scales.resize(size_t(n * (q8 ? 1 : (k + 31) / 32)));
    const int rc = q8 ? lyk_q8_quantize(w.data(), n, k, codes.data(), scales.data())
                      : lyk_q4_quantize(w.data(), n, k, codes.data(), scales.data());
    if (rc != LYK_OK) return Status(ErrorCode::kUnsupportedModel, "weight quantization failed", kComponent);
    return Status::Ok();
}

// Packs codes and scales (paired: b beside a, gate and up) into the fused
// step's tiled layout and uploads them.
Status PackUpload(bool q8, const std::vector<int8_t>& ca, const std::vector<uint16_t>& sa,
                  const std::vector<int8_t>* cbp, const std::vector<uint16_t>* sbp, int64_t n, int64_t k,
                  bool normed_input, int tile_rows, PackedMat& out, uint64_t& bytes) {
    const bool paired = cbp != nullptr;
    int rc;
    // the tile height the fused step streams this shape best with on this device
    const int tr = tile_rows ? tile_rows : lyk_hip_step_tile_rows(n, k, paired, q8 ? 1 : 0, normed_input ? 1 : 0);
    if (tr == 0) return Status(ErrorCode::kGpuUnhealthy, "hip device properties unavailable", kComponent);
    if (tr != 16 && tr != 32 && tr != 64) return Status(ErrorCode::kUnsupportedModel, "tile height must be 16, 32 or 64", kComponent);
    uint64_t wb = 0, sbytes = 0;
    rc = q8 ? lyk_q8_layout_tiled(n, k, paired, tr, &wb, &sbytes)
            : lyk_q4_layout_tiled(n, k, paired, tr, &wb, &sbytes);
    if (rc != LYK_OK) return Status(ErrorCode::kUnsupportedModel, "weight shape unsupported", kComponent);
    std::vector<uint8_t> qw(wb), qs(sbytes);
    const int8_t* cb = paired ? cbp->data() : nullptr;
    const uint16_t* sb = paired ? sbp->data() : nullptr;
    rc = q8 ? lyk_q8_pack_tiled(ca.data(), sa.data(), cb, sb, n, k, tr, qw.data(), qs.data())
            : lyk_q4_pack_tiled(ca.data(), sa.data(), cb, sb, n, k, tr, qw.data(), qs.data());
    if (rc != LYK_OK) return Status(ErrorCode::kUnsupportedModel, "weight packing failed", kComponent);
    Status s = out.qw.Upload(qw.data(), qw.size());
    if (!s.ok()) return s;
    s = out.qs.Upload(qs.data(), qs.size());
    if (!s.ok()) return s;
    out.n = n;
    out.k = k;
    out.paired = paired;
    out.tile_rows = tr;
    // bytes a step reads: codes and scales of the real rows (no tile padding)
    const int64_t rows = n * (paired ? 2 : 1);
    bytes += q8 ? uint64_t(rows * k + rows * 2) : uint64_t(rows * ((k + 1) / 2) + rows * ((k + 31) / 32) * 2);
    return Status::Ok();
}

Status UploadF32(const std::vector<float>& v, DevBuf& out) { return out.Upload(v.data(), v.size() * 4); }

}  // namespace

QwenHipModel::LoadResult QwenHipModel::Load(const ModelManifest& manifest, const SafetensorsFile& weights,
                                            const HipModelOptions& options) {
    SafetensorsWeightSource src(weights);
    return Load(manifest, src, options);
}

QwenHipModel::LoadResult QwenHipModel::Load(const ModelManifest& manifest, const WeightSource& src,
                                            const HipModelOptions& options) {
    LoadResult r;
    std::unique_ptr<QwenHipModel> model(new QwenHipModel());
    r.status = HipQwenConfig::FromManifest(manifest, model->config_);
    if (!r.status.ok()) return r;
    const HipQwenConfig& c = model->config_;
    model->limits_.vocab_size = c.vocab_size;
    model->limits_.max_context_tokens = c.max_context_tokens;
    model->limits_.eos_token_ids = c.eos_token_ids;
    model->device_id_ = options.device_id;
    if (options.kv_block_tokens == 0) {
        r.status = Status(ErrorCode::kUnsupportedModel, "kv block size must be positive", kComponent);
        return r;
    }

    int devices = 0;
    if (hipGetDeviceCount(&devices) != hipSuccess || options.device_id < 0 || options.device_id >= devices) {
        r.status = Status(ErrorCode::kGpuUnhealthy, "hip device not available", kComponent);
        return r;
    }
    if (hipSetDevice(options.device_id) != hipSuccess) {
        r.status = Status(ErrorCode::kGpuUnhealthy, "hip device not usable", kComponent);
        return r;
    }

    auto impl = std::make_unique<Impl>();
    Impl& I = *impl;
    I.opt = options;
    I.c = c;
    I.q8 = options.quantization == HipWeightQuant::kInt8;
    if (hipStreamCreateWithFlags(&I.stream, hipStreamNonBlocking) != hipSuccess) {
        r.status = Status(ErrorCode::kGpuUnhealthy, "stream creation failed", kComponent);
        return r;
    }

    const uint64_t H = c.hidden_size, qd = uint64_t(c.num_heads) * c.head_dim,
                   kvd = uint64_t(c.num_kv_heads) * c.head_dim, In = c.intermediate_size, V = c.vocab_size;
    size_t expected = 0;
    std::vector<float> a, b, cbuf;
    auto read = [&](const std::string& name, std::vector<uint64_t> shape, std::vector<float>& out) {
        ++expected;
        return src.Read(name, shape, out);
    };
    // An [n, k] GEMV matrix as codes and scales: offline-quantized in the
    // source (`base`.qweight / .qscale), else `base`.weight quantized here.
    auto codes_of = [&](const std::string& base, uint64_t n, uint64_t k, std::vector<int8_t>& codes,
                        std::vector<uint16_t>& scales) -> Status {
        bool found = false;
        Status s = src.ReadQuantized(base, I.q8, int64_t(n), int64_t(k), codes, scales, found);
        if (!s.ok()) return s;
        if (found) {
            expected += 2;
            return Status::Ok();
        }
        std::vector<float> w;
        s = read(base + ".weight", {n, k}, w);
        if (!s.ok()) return s;
        return Quantize(I.q8, w, int64_t(n), int64_t(k), codes, scales);
    };
    std::vector<int8_t> ca, cb, ct;
    std::vector<uint16_t> sa, sb, st;
#define LOAD_OR_RETURN(expr)         \
    do {                             \
        Status s_ = (expr);          \
        if (!s_.ok()) {              \
            r.status = s_;           \
            return r;                \
        }                            \
    } while (0)

    std::vector<float> embed;
    LOAD_OR_RETURN(read("model.embed_tokens.weight", {V, H}, embed));
    LOAD_OR_RETURN(UploadF32(embed, I.embed));
    I.layers.resize(c.num_layers);
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        Impl::Layer& L = I.layers[l];
        LOAD_OR_RETURN(read(LayerName(l, "input_layernorm.weight"), {H}, a));
        LOAD_OR_RETURN(UploadF32(a, L.input_norm));
        LOAD_OR_RETURN(read(LayerName(l, "post_attention_layernorm.weight"), {H}, a));
        LOAD_OR_RETURN(UploadF32(a, L.post_norm));
        // fused qkv: rows [q | k | v] (codes and per-row scales
        // concatenated), bias concatenated the same way
        std::vector<float> bias, t;
        ca.clear();
        sa.clear();
        for (const char* nm : {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"}) {
            LOAD_OR_RETURN(codes_of(LayerName(l, nm), std::string(nm) == "self_attn.q_proj" ? qd : kvd, H, ct, st));
            ca.insert(ca.end(), ct.begin(), ct.end());
            sa.insert(sa.end(), st.begin(), st.end());
        }
        for (const char* nm : {"self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias"}) {
            LOAD_OR_RETURN(read(LayerName(l, nm), {std::string(nm).find("q_proj") != std::string::npos ? qd : kvd}, t));
            bias.insert(bias.end(), t.begin(), t.end());
        }
        LOAD_OR_RETURN(PackUpload(I.q8, ca, sa, nullptr, nullptr, int64_t(qd + 2 * kvd), int64_t(H), true,
                                  options.tile_rows[0], L.qkv, I.gemv_bytes));
        LOAD_OR_RETURN(UploadF32(bias, L.qkv_bias));
        LOAD_OR_RETURN(codes_of(LayerName(l, "self_attn.o_proj"), H, qd, ca, sa));
        LOAD_OR_RETURN(PackUpload(I.q8, ca, sa, nullptr, nullptr, int64_t(H), int64_t(qd), false, options.tile_rows[1],
                                  L.o, I.gemv_bytes));
        LOAD_OR_RETURN(codes_of(LayerName(l, "mlp.gate_proj"), In, H, ca, sa));
        LOAD_OR_RETURN(codes_of(LayerName(l, "mlp.up_proj"), In, H, cb, sb));
        LOAD_OR_RETURN(PackUpload(I.q8, ca, sa, &cb, &sb, int64_t(In), int64_t(H), true, options.tile_rows[2],
                                  L.gateup, I.gemv_bytes));
        LOAD_OR_RETURN(codes_of(LayerName(l, "mlp.down_proj"), H, In, ca, sa));
        LOAD_OR_RETURN(PackUpload(I.q8, ca, sa, nullptr, nullptr, int64_t(H), int64_t(In), false, options.tile_rows[3],
                                  L.down, I.gemv_bytes));
    }
    LOAD_OR_RETURN(read("model.norm.weight", {H}, a));
    LOAD_OR_RETURN(UploadF32(a, I.final_norm));
    if (c.tie_word_embeddings) {
        // the head is the embedding; an offline-quantized artifact may carry
        // its quantized form as lm_head.qweight / .qscale
        bool found = false;
        LOAD_OR_RETURN(src.ReadQuantized("lm_head", I.q8, int64_t(V), int64_t(H), ca, sa, found));
        if (found) expected += 2;
        else LOAD_OR_RETURN(Quantize(I.q8, embed, int64_t(V), int64_t(H), ca, sa));
    } else {
        LOAD_OR_RETURN(codes_of("lm_head", V, H, ca, sa));
    }
    LOAD_OR_RETURN(PackUpload(I.q8, ca, sa, nullptr, nullptr, int64_t(V), int64_t(H), true, options.tile_rows[4],
                              I.lm_head, I.gemv_bytes));
    if (src.tensor_count() != expected) {
        r.status = Status(ErrorCode::kArtifactVerificationFailed, "weight file contains unexpected tensors",
                          kComponent);
        return r;
    }
    embed.clear();
    embed.shrink_to_fit();

    // paged KV pool
    const uint32_t bt = options.kv_block_tokens;
    const uint64_t pool_tokens =
        options.kv_pool_tokens ? options.kv_pool_tokens : uint64_t(std::max(1u, c.max_context_tokens)) * 4;
    const uint32_t nblocks = uint32_t(std::max<uint64_t>(1, (pool_tokens + bt - 1) / bt));
    I.pool = std::make_shared<hip::KvBlockPool>(nblocks, bt);
    I.kv_layer_elems = (size_t)nblocks * c.num_kv_heads * bt * c.head_dim;
    LOAD_OR_RETURN(I.kv.Alloc(I.kv_layer_elems * 2 * 2 * c.num_layers));

    // step rows
    const size_t B = kMaxBatch;
    LOAD_OR_RETURN(I.d_tokens.Alloc(B * 4));
    LOAD_OR_RETURN(I.d_pos.Alloc(B * 4));
    LOAD_OR_RETURN(I.d_logits.Alloc(B * V * 4));
    LOAD_OR_RETURN(I.d_history.Alloc(kGreedyMax * 4));
    LOAD_OR_RETURN(I.d_step.Alloc(4));
    LOAD_OR_RETURN(I.d_nonfinite.Alloc(B * 4));
    LOAD_OR_RETURN(I.h_tokens.Alloc(B * 4));
    LOAD_OR_RETURN(I.h_pos.Alloc(B * 4));
    LOAD_OR_RETURN(I.h_logits.Alloc(B * V * 4));
    LOAD_OR_RETURN(I.h_history.Alloc(kGreedyMax * 4));
    LOAD_OR_RETURN(I.h_nonfinite.Alloc(B * 4));

    // fused step: model description, device layer table, workspace
    std::vector<lyk_step_layer> table(c.num_layers);
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        const Impl::Layer& L = I.layers[l];
        lyk_step_layer& e = table[l];
        e.qkv_w = L.qkv.qw.p;
        e.qkv_s = L.qkv.qs.p;
        e.qkv_bias = L.qkv_bias.as<float>();
        e.o_w = L.o.qw.p;
        e.o_s = L.o.qs.p;
        e.gateup_w = L.gateup.qw.p;
        e.gateup_s = L.gateup.qs.p;
        e.down_w = L.down.qw.p;
        e.down_s = L.down.qs.p;
        e.input_norm = L.input_norm.as<float>();
        e.post_norm = L.post_norm.as<float>();
        e.k_cache = I.kcache(l);
        e.v_cache = I.vcache(l);
    }
    LOAD_OR_RETURN(I.d_layers.Upload(table.data(), table.size() * sizeof(lyk_step_layer)));
    lyk_step_model& md = I.md;
    md.vocab_size = int32_t(V);
    md.hidden_size = int32_t(H);
    md.num_layers = int32_t(c.num_layers);
    md.num_heads = int32_t(c.num_heads);
    md.num_kv_heads = int32_t(c.num_kv_heads);
    md.head_dim = int32_t(c.head_dim);
    md.intermediate_size = int32_t(In);
    md.q8 = I.q8 ? 1 : 0;
    md.rms_norm_eps = c.rms_norm_eps;
    md.block_tokens = int32_t(bt);
    md.num_blocks = int32_t(nblocks);
    md.attn_split_tokens = options.attn_split_tokens;
    md.attn_max_splits = options.attn_max_splits;
    md.lds_prefetch = options.lds_prefetch;
    md.tile_rows[0] = I.layers[0].qkv.tile_rows;
    md.tile_rows[1] = I.layers[0].o.tile_rows;
    md.tile_rows[2] = I.layers[0].gateup.tile_rows;
    md.tile_rows[3] = I.layers[0].down.tile_rows;
    md.tile_rows[4] = I.lm_head.tile_rows;
    md.embed = I.embed.as<float>();
    md.final_norm = I.final_norm.as<float>();
    md.lm_head_w = I.lm_head.qw.p;
    md.lm_head_s = I.lm_head.qs.p;
    md.layers = I.d_layers.as<lyk_step_layer>();
    LOAD_OR_RETURN(I.EnsureRope(std::max(1u, c.max_context_tokens)));
    I.step_ws_bytes = lyk_hip_step_workspace_bytes(&md, kMaxBatch);
    if (I.step_ws_bytes == 0) {
        r.status = Status(ErrorCode::kUnsupportedModel, "model geometry unsupported by the hip kernels",
                          kComponent);
        return r;
    }
    LOAD_OR_RETURN(I.d_step_ws.Alloc(I.step_ws_bytes, false));
    // chunk prefill where its kernels take the geometry (head dim 64 or 128,
    // GEMM rows a multiple of 8)
    {
        const uint32_t kq = c.num_heads * c.head_dim;
        const bool fits = (c.head_dim == 64 || c.head_dim == 128) && H % 8 == 0 && kq % 8 == 0 && In % 8 == 0;
        const int want = options.prefill_chunk;
        if (want < -1) {
            r.status = Status(ErrorCode::kInvalidRequest, "prefill_chunk must be -1, 0 or positive", kComponent);
            return r;
        }
        I.chunk_rows = want == -1 || !fits ? 0u : want == 0 ? kDefaultChunkRows : uint32_t(want);
        if (I.chunk_rows) {
            const size_t C = I.chunk_rows, rows = size_t(c.num_heads + 2 * c.num_kv_heads) * c.head_dim;
            LOAD_OR_RETURN(I.pf_x.Alloc(C * H * 4, false));
            LOAD_OR_RETURN(I.pf_xn.Alloc(C * H * 2, false));
            LOAD_OR_RETURN(I.pf_qkv.Alloc(C * rows * 4, false));
            LOAD_OR_RETURN(I.pf_q.Alloc(C * kq * 4, false));
            LOAD_OR_RETURN(I.pf_attn.Alloc(C * kq * 2, false));
            LOAD_OR_RETURN(I.pf_act.Alloc(C * In * 2, false));
        }
    }
    if (lyk_hip_step_reset(I.d_step_ws.p, I.step_ws_bytes, I.stream) != LYK_OK) {
        r.status = Status(ErrorCode::kGpuUnhealthy, "workspace reset failed", kComponent);
        return r;
    }
    if (hipDeviceSynchronize() != hipSuccess) {
        r.status = Status(ErrorCode::kGpuUnhealthy, "device initialisation failed", kComponent);
        return r;
    }
#undef LOAD_OR_RETURN
    model->impl_ = std::move(impl);
    r.model = std::move(model);
    return r;
}

QwenHipModel::~QwenHipModel() {
    if (impl_) (void)hipSetDevice(device_id_);
}

void* QwenHipModel::stream() const { return impl_->stream; }

Status QwenHipModel::SetStepTracing(bool on) {
    HIP_OK(hipSetDevice(device_id_), "hip device not usable");
    Impl& I = *impl_;
    if (on && !I.d_trace.p) {
        Status s = I.d_trace.Alloc((size_t)lyk_hip_step_grid() *
                                   (4 * (size_t)lyk_hip_step_phases(&I.md, LYK_STEP_GREEDY) + 2) * 8);
        if (!s.ok()) return s;
    }
    I.tracing = on;
    return Status::Ok();
}

Status QwenHipModel::StepTrace(std::vector<uint64_t>& ticks) {
    Impl& I = *impl_;
    ticks.clear();
    if (!I.d_trace.p) return Status(ErrorCode::kInvalidRequest, "step tracing is off", kComponent);
    HIP_OK(hipSetDevice(device_id_), "hip device not usable");
    HIP_OK(hipStreamSynchronize(I.stream), "device execution failed");
    ticks.resize(I.d_trace.bytes / 8);
    HIP_OK(hipMemcpy(ticks.data(), I.d_trace.p, I.d_trace.bytes, hipMemcpyDeviceToHost), "trace download failed");
    return Status::Ok();
}

uint64_t QwenHipModel::step_launches() const { return lyk_hip_step_launches(impl_->d_step_ws.p); }

Status QwenHipModel::SetStepLaunches(uint64_t launches) {
    HIP_OK(hipSetDevice(device_id_), "hip device not usable");
    Impl& I = *impl_;
    HIP_OK(hipStreamSynchronize(I.stream), "device execution failed");
    LYK_OK_OR(lyk_hip_step_set_launches(&I.md, kMaxBatch, I.d_step_ws.p, I.step_ws_bytes, launches, I.stream),
              "step launch count update failed");
    return Status::Ok();
}

void QwenHipModel::SetWaitLimit(uint32_t microseconds) { impl_->md.wait_limit_us = microseconds; }

uint32_t QwenHipModel::kv_blocks_total() const { return impl_->pool->num_blocks(); }
uint32_t QwenHipModel::kv_blocks_free() const { return impl_->pool->available(); }
uint64_t QwenHipModel::prefix_cache_hit_tokens() const { return impl_->prefix_hits; }
uint64_t QwenHipModel::gemv_weight_bytes() const { return impl_->gemv_bytes; }

// ---------------------------------------------------------------- sequences

Status QwenHipModel::CreateSequence(uint32_t max_tokens, std::unique_ptr<SequenceState>& out) {
    return CreateSequenceEx(max_tokens, SequenceOptions{}, out);
}

Status QwenHipModel::CreateSequenceEx(uint32_t max_tokens, const SequenceOptions& options,
                                      std::unique_ptr<SequenceState>& out) {
    HIP_OK(hipSetDevice(device_id_), "hip device not usable");
    Status s = impl_->EnsureRope(std::max(1u, max_tokens));
    if (!s.ok()) return s;
    out = std::make_unique<HipSequenceState>(impl_->pool, max_tokens, options);
    return Status::Ok();
}

Status QwenHipModel::Prefill(SequenceState& state, const std::vector<uint32_t>& tokens,
                             std::vector<float>& logits) {
    auto& seq = static_cast<HipSequenceState&>(state);
    if (tokens.empty()) return Status(ErrorCode::kInvalidRequest, "empty prompt", kComponent);
    if (seq.length() != 0) return Status(ErrorCode::kInternalError, "prefill requires an empty cache", kComponent);
    if (tokens.size() > seq.capacity())
        return Status(ErrorCode::kContextLengthExceeded, "prompt exceeds cache capacity", kComponent);
    for (uint32_t t : tokens)
        if (t >= config_.vocab_size) return Status(ErrorCode::kInvalidRequest, "token id out of vocab range", kComponent);
    HIP_OK(hipSetDevice(device_id_), "hip device not usable");
    Impl& I = *impl_;
    const uint32_t bt = I.pool->block_tokens();
    const uint32_t n = uint32_t(tokens.size());

    // Prefix cache: blocks published under the same scope-seeded chain keys
    // are adopted from the start of the prompt; the block holding the last
    // token is always recomputed, so its logits come out.
    std::vector<uint64_t> keys;
    uint32_t start = 0;
    if (seq.options().allow_prefix_cache) {
        keys = hip::PrefixChainKeys(seq.options().scope_key, tokens.data(), n, bt);
        std::vector<int32_t> hit;
        for (uint32_t b = 0; b < (n - 1) / bt; ++b) {
            const std::optional<int32_t> blk = I.pool->Find(keys[b]);
            if (!blk) break;
            hit.push_back(*blk);
        }
        start = uint32_t(hit.size()) * bt;
        if (!hit.empty()) seq.Adopt(std::move(hit), start);
    }
    // Any failure from here leaves the sequence empty again, with nothing
    // published, so the caller may retry or drop it.
    auto fail = [&seq](Status s) {
        seq.Clear();
        return s;
    };

    Status s = seq.Reserve(n);
    if (!s.ok()) return fail(s);
    // Tokens and then positions of the uncached part go up in one copy
    // (rows tokens, rows positions); the chunk passes read the tokens in
    // place, and each fused step takes its row with device-to-device
    // copies, so no host staging buffer is rewritten while a copy from it
    // may be pending.
    const size_t rows = n - start;
    if (rows * 2 > I.prompt_cap) {
        HIP_OK(hipStreamSynchronize(I.stream), "device execution failed");
        I.prompt_cap = std::max<size_t>(rows * 2, 1024);
        if (!(s = I.d_prompt.Alloc(I.prompt_cap * 4)).ok()) return fail(s);
        if (!(s = I.h_prompt.Alloc(I.prompt_cap * 4)).ok()) return fail(s);
    }
    int32_t* hp = I.h_prompt.as<int32_t>();
    for (size_t r = 0; r < rows; ++r) {
        hp[r] = int32_t(tokens[start + r]);
        hp[rows + r] = int32_t(start + r);
    }
    if (hipMemcpyAsync(I.d_prompt.p, hp, rows * 8, hipMemcpyHostToDevice, I.stream) != hipSuccess)
        return fail(Status(ErrorCode::kGpuUnhealthy, "prompt upload failed", kComponent));
    if (!(s = I.UploadRows({&seq}, {tokens[start]}, {start})).ok()) return fail(s);
    const int32_t* d_tok = I.d_prompt.as<int32_t>();
    const int32_t* d_pos = d_tok + rows;
    // Every token but the last in chunk passes on the matrix cores, the
    // last through the fused step, which gives the logits; without chunk
    // passes every token goes through the step (HIDDEN mode but the last).
    uint32_t first_step = start;
    if (I.chunk_rows && n - 1 > start) {
        const int table_len = int(seq.blocks().size());
        for (uint32_t c0 = start; c0 < n - 1; c0 += I.chunk_rows) {
            const uint32_t T = std::min(I.chunk_rows, n - 1 - c0);
            if (!(s = I.ChunkPass(d_tok + (c0 - start), int(T), int(c0), table_len)).ok()) return fail(s);
        }
        first_step = n - 1;
    }
    for (uint32_t i = first_step; i < n; ++i) {
        const size_t r = i - start;
        if (hipMemcpyAsync(I.d_tokens.p, d_tok + r, 4, hipMemcpyDeviceToDevice, I.stream) != hipSuccess ||
            hipMemcpyAsync(I.d_pos.p, d_pos + r, 4, hipMemcpyDeviceToDevice, I.stream) != hipSuccess)
            return fail(Status(ErrorCode::kGpuUnhealthy, "prompt row copy failed", kComponent));
        if (!(s = I.LaunchStep(1, i + 1 == n ? LYK_STEP_LOGITS : LYK_STEP_HIDDEN)).ok()) return fail(s);
    }
    logits.resize(config_.vocab_size);
    if (hipMemcpyAsync(I.h_logits.p, I.d_logits.p, logits.size() * 4, hipMemcpyDeviceToHost, I.stream) !=
            hipSuccess ||
        hipStreamSynchronize(I.stream) != hipSuccess)
        return fail(Status(ErrorCode::kGpuUnhealthy, "device execution failed", kComponent));
    if (!(s = I.CheckSteps()).ok()) return fail(s);
    std::memcpy(logits.data(), I.h_logits.p, logits.size() * 4);
    for (float v : logits)
        if (!std::isfinite(v))
            return fail(Status(ErrorCode::kInferenceFailed, "logits contain non-finite values", kComponent));

    seq.Advance(n - start);
    I.prefix_hits += start;
    for (size_t b = 0; b < keys.size() && b < seq.blocks().size(); ++b) I.pool->Publish(keys[b], seq.blocks()[b]);
    return Status::Ok();
}

Status QwenHipModel::Decode(SequenceState& state, uint32_t token, std::vector<float>& logits) {
    std::vector<DecodeBatchItem> items = {{&state, token, &logits}};
    std::vector<Status> per_item;
    Status s = DecodeBatch(items, per_item);
    if (!s.ok()) return s;
    return per_item[0];
}

Status QwenHipModel::DecodeBatch(std::vector<DecodeBatchItem>& items, std::vector<Status>& per_item) {
    per_item.assign(items.size(), Status::Ok());
    HIP_OK(hipSetDevice(device_id_), "hip device not usable");
    Impl& I = *impl_;
    std::vector<size_t> valid;
    for (size_t i = 0; i < items.size(); ++i) {
        auto* st = static_cast<HipSequenceState*>(items[i].state);
        if (items[i].token >= config_.vocab_size) {
            per_item[i] = Status(ErrorCode::kInvalidRequest, "token id out of vocab range", kComponent);
        } else if (st->length() >= st->capacity()) {
            per_item[i] = Status(ErrorCode::kContextLengthExceeded, "kv cache capacity exhausted", kComponent);
        } else {
            Status cap = st->Reserve(st->length() + 1);
            if (!cap.ok()) per_item[i] = cap;
            else valid.push_back(i);
        }
    }
    // Every group of rows runs before any sequence advances: a device
    // failure in a later group returns with no sequence advanced (the K/V
    // rows already written sit past each sequence's length and are
    // rewritten by its next step).
    const size_t V = config_.vocab_size;
    for (size_t g0 = 0; g0 < valid.size(); g0 += kMaxBatch) {
        const size_t m = std::min<size_t>(kMaxBatch, valid.size() - g0);
        std::vector<HipSequenceState*> seqs;
        std::vector<uint32_t> toks, pos;
        for (size_t i = 0; i < m; ++i) {
            const size_t idx = valid[g0 + i];
            auto* st = static_cast<HipSequenceState*>(items[idx].state);
            seqs.push_back(st);
            toks.push_back(items[idx].token);
            pos.push_back(st->length());
        }
        Status s = I.UploadRows(seqs, toks, pos);
        if (!s.ok()) return s;
        s = I.LaunchStep(int(m), LYK_STEP_LOGITS);
        if (!s.ok()) return s;
        HIP_OK(hipMemcpyAsync(I.h_logits.p, I.d_logits.p, m * V * 4, hipMemcpyDeviceToHost, I.stream),
               "logits download failed");
        HIP_OK(hipStreamSynchronize(I.stream), "device execution failed");
        s = I.CheckSteps();
        if (!s.ok()) return s;
        const float* hl = I.h_logits.as<float>();
        for (size_t i = 0; i < m; ++i) items[valid[g0 + i]].logits->assign(hl + i * V, hl + (i + 1) * V);
    }
    for (size_t idx : valid) {
        const std::vector<float>& out = *items[idx].logits;
        if (std::all_of(out.begin(), out.end(), [](float v) { return std::isfinite(v); }))
            static_cast<HipSequenceState*>(items[idx].state)->Advance(1);
        else
            per_item[idx] = Status(ErrorCode::kInferenceFailed, "logits contain non-finite values", kComponent);
    }
    return Status::Ok();
}

Status QwenHipModel::GreedyRun(SequenceState& state, uint32_t token, uint32_t max_new,
                               std::vector<uint32_t>& out_tokens) {
    auto& seq = static_cast<HipSequenceState&>(state);
    out_tokens.clear();
    if (token >= config_.vocab_size)
        return Status(ErrorCode::kInvalidRequest, "token id out of vocab range", kComponent);
    if (max_new == 0) return Status(ErrorCode::kInvalidRequest, "max_new must be > 0", kComponent);
    if (seq.length() >= seq.capacity())
        return Status(ErrorCode::kContextLengthExceeded, "kv cache capacity exhausted", kComponent);
    HIP_OK(hipSetDevice(device_id_), "hip device not usable");
    Impl& I = *impl_;
    const uint32_t len = seq.length();
    const uint32_t steps = std::min({max_new, kGreedyMax, seq.capacity() - len});
    Status s = seq.Reserve(len + steps);
    if (!s.ok()) return s;
    s = I.UploadRows({&seq}, {token}, {len});
    if (!s.ok()) return s;
    HIP_OK(hipMemsetAsync(I.d_step.p, 0, 4, I.stream), "step reset failed");
    HIP_OK(hipMemsetAsync(I.d_nonfinite.p, 0, 4, I.stream), "flag reset failed");
    for (uint32_t i = 0; i < steps; ++i) {
        s = I.LaunchStep(1, LYK_STEP_GREEDY);
        if (!s.ok()) return s;
    }
    HIP_OK(hipMemcpyAsync(I.h_history.p, I.d_history.p, steps * 4, hipMemcpyDeviceToHost, I.stream),
           "token download failed");
    HIP_OK(hipMemcpyAsync(I.h_nonfinite.p, I.d_nonfinite.p, 4, hipMemcpyDeviceToHost, I.stream),
           "flag download failed");
    HIP_OK(hipStreamSynchronize(I.stream), "device execution failed");
    s = I.CheckSteps();
    if (!s.ok()) return s;
    if (I.h_nonfinite.as<int32_t>()[0] != 0)
        return Status(ErrorCode::kInferenceFailed, "logits contain non-finite values", kComponent);
    const int32_t* hist = I.h_history.as<int32_t>();
    out_tokens.assign(hist, hist + steps);
    seq.Advance(steps);
    return Status::Ok();
}

}  // namespace lykuro::nie
