// plugins.cpp — the inference-engine plugins of the LLM operator path:
// plugin_rms_norm, plugin_rms_norm_add, plugin_reshape_and_cache,
// plugin_causal_conv1d_fn and plugin_flash_attention.
//
// Names, inputs, attributes (with their defaults), output shapes and the
// zero-then-compute semantics follow the reference plugins
// (teco/plugin/pluginRmsNorm/plugin_rms_norm.cc:52-149,
//  pluginReshapeAndCache/plugin_reshape_and_cache.cc:38-130,
//  pluginCausalConv1d/plugin_causal_conv1d.cc:38-186,
//  pluginFlashAttention/plugin_flash_attention.cc:38-160).
// Differences, each toward the reference's documented intent:
//   * every tecoops status is checked; a failure throws PluginError (the
//     reference ignores the returned status);
//   * one tecoops handle per plugin instance, rebound to the engine stream on
//     each Enqueue (the reference creates and destroys one per call, which on
//     this library would also drop flash attention's split-KV scratch);
//   * the element type comes from the engine's input type (fp16 when the
//     engine gives none, as the reference assumes);
//   * flash attention passes the block table's real shape and differences
//     cu_seqlens_q on the device (the reference leaves bt_shape empty and
//     passes cumulative offsets where per-batch lengths are expected,
//     plugin_flash_attention.cc:79, :98, :108); on a stream being captured
//     into a graph it calls the allocation-free entry point;
//   * causal_conv1d treats the stride attributes' default 0 as "packed"
//     (dim for x / out rows, (width-1)*dim for conv_state entries), and
//     copies the updated state on the engine stream instead of a blocking
//     copy (plugin_causal_conv1d.cc:153);
//   * no progress printing to stdout.
#include <algorithm>
#include <cmath>
#include <numeric>

#include "tecoops_plugin.h"

namespace TECO_INFER {

namespace {

void check(tecoopsStatus_t st, const char *what) {
    if (st != TECOOPS_STATUS_SUCCESS)
        throw PluginError(st, std::string(what) + ": " + tecoopsGetErrorString(st));
}

void check_hip(hipError_t e, const char *what) {
    if (e != hipSuccess)
        throw PluginError(TECOOPS_STATUS_INTERNAL_ERROR,
                          std::string(what) + ": " + hipGetErrorString(e));
}

void require(bool ok, const std::string &msg) {
    if (!ok) throw PluginError(TECOOPS_STATUS_BAD_PARAM, msg);
}

int64_t numel(const std::vector<int> &s) {
    return std::accumulate(s.begin(), s.end(), int64_t{1},
                           [](int64_t a, int b) { return a * b; });
}

size_t elem_bytes(tecoopsDataType_t t) {
    switch (t) {
        case TECOOPS_DATA_HALF:
        case TECOOPS_DATA_BFLOAT16:
        case TECOOPS_DATA_INT16:
            return 2;
        case TECOOPS_DATA_INT8:
        case TECOOPS_DATA_UINT8:
        case TECOOPS_DATA_BOOL:
            return 1;
        case TECOOPS_DATA_INT64:
        case TECOOPS_DATA_DOUBLE:
            return 8;
        default:
            return 4;
    }
}

// A tecoops handle owned by one plugin instance.
class PluginHandle {
 public:
    PluginHandle() = default;
    PluginHandle(const PluginHandle &) = delete;
    PluginHandle &operator=(const PluginHandle &) = delete;
    ~PluginHandle() {
        if (h_ != nullptr) tecoopsDestroy(h_);
    }
    tecoopsHandle_t bind(hipStream_t stream) {
        if (h_ == nullptr) check(tecoopsCreate(&h_), "tecoopsCreate");
        check(tecoopsSetStream(h_, stream), "tecoopsSetStream");
        return h_;
    }

 private:
    tecoopsHandle_t h_ = nullptr;
};

// Tensor descriptor freed on scope exit.
class Desc {
 public:
    Desc(tecoopsDataType_t t, const std::vector<int> &shape) {
        check(tecoopsCreateTensorDescriptor(&d_), "tecoopsCreateTensorDescriptor");
        const tecoopsStatus_t st = tecoopsSetTensorNdDescriptor(
            d_, t, static_cast<int>(shape.size()), shape.data(), nullptr);
        if (st != TECOOPS_STATUS_SUCCESS) {
            tecoopsDestroyTensorDescriptor(d_);
            d_ = nullptr;
            check(st, "tecoopsSetTensorNdDescriptor");
        }
    }
    ~Desc() {
        if (d_ != nullptr) tecoopsDestroyTensorDescriptor(d_);
    }
    operator tecoopsTensorDescriptor_t() const { return d_; }

 private:
    tecoopsTensorDescriptor_t d_ = nullptr;
};

// ------------------------------------------------------------------ rms_norm

struct plugin_rms_normAttrs {
    static void Declare(AttrDecl &d) { d.Field("eps", 1e-5, "Epsilon for numerical stability"); }
};
using plugin_rms_norm_addAttrs = plugin_rms_normAttrs;

// [..., hidden] rows: every leading dimension counts as tokens.
void rms_rows(const std::vector<int> &shape, int &tokens, int &hidden) {
    require(shape.size() >= 2, "rms_norm input must be [num_tokens, hidden_size]");
    hidden = shape.back();
    const int64_t n = numel(shape) / std::max(hidden, 1);
    require(n <= INT32_MAX, "rms_norm: too many rows");
    tokens = static_cast<int>(n);
}

class PluginRmsNormImpl : public AbstractPluginOp {
 public:
    void InferOutputShape(const std::vector<std::vector<int>> &in, int, std::vector<std::vector<int>> &out,
                          int, const OpAttr &) override {
        out[0] = in[0];
    }
    void Enqueue(std::shared_ptr<ComputeContext> &ctx) override {
        std::vector<int> shape;
        ctx->GetInputShape(0, shape);
        int tokens, hidden;
        rms_rows(shape, tokens, hidden);
        double eps;
        ctx->GetAttr("eps", eps);
        check(tecoopsRmsNormEx(handle_.bind(ctx->GetStream()), ctx->GetInputDataPtr(0),
                               ctx->GetInputDataPtr(1), nullptr, ctx->GetOutputDataPtr(0), nullptr,
                               tokens, hidden, static_cast<float>(eps), ctx->GetInputDataType(0)),
              "plugin_rms_norm");
    }

 private:
    PluginHandle handle_;
};

class PluginRmsNormAddImpl : public AbstractPluginOp {
 public:
    void InferOutputShape(const std::vector<std::vector<int>> &in, int, std::vector<std::vector<int>> &out,
                          int, const OpAttr &) override {
        out[0] = in[0];
        out[1] = in[0];
    }
    void Enqueue(std::shared_ptr<ComputeContext> &ctx) override {
        std::vector<int> shape, rshape;
        ctx->GetInputShape(0, shape);
        ctx->GetInputShape(2, rshape);
        require(numel(shape) == numel(rshape), "rms_norm_add: residual shape differs from input");
        int tokens, hidden;
        rms_rows(shape, tokens, hidden);
        double eps;
        ctx->GetAttr("eps", eps);
        check(tecoopsRmsNormEx(handle_.bind(ctx->GetStream()), ctx->GetInputDataPtr(0),
                               ctx->GetInputDataPtr(1), ctx->GetInputDataPtr(2),
                               ctx->GetOutputDataPtr(0), ctx->GetOutputDataPtr(1), tokens, hidden,
                               static_cast<float>(eps), ctx->GetInputDataType(0)),
              "plugin_rms_norm_add");
    }

 private:
    PluginHandle handle_;
};

// ---------------------------------------------------------- reshape_and_cache

struct plugin_reshape_and_cacheAttrs {
    static void Declare(AttrDecl &d) {
        d.Field("num_blocks", int64_t{0}, "Number of KV cache blocks")
            .Field("block_size", int64_t{0}, "Block size (tokens per block)");
    }
};

// One output [2*num_blocks, Hkv, block_size, D]: key cache, then value cache.
class PluginReshapeAndCacheImpl : public AbstractPluginOp {
 public:
    void InferOutputShape(const std::vector<std::vector<int>> &in, int, std::vector<std::vector<int>> &out,
                          int, const OpAttr &attr) override {
        require(in[0].size() == 3, "key must be [num_tokens, num_kv_heads, head_size]");
        const int64_t nb = attr.GetAttr<int64_t>("num_blocks");
        const int64_t bs = attr.GetAttr<int64_t>("block_size");
        require(nb > 0 && bs > 0 && 2 * nb <= INT32_MAX, "num_blocks and block_size must be > 0");
        out[0] = {static_cast<int>(2 * nb), in[0][1], static_cast<int>(bs), in[0][2]};
    }
    void Enqueue(std::shared_ptr<ComputeContext> &ctx) override {
        std::vector<int> ks;
        ctx->GetInputShape("key", ks);
        require(ks.size() == 3, "key must be [num_tokens, num_kv_heads, head_size]");
        int64_t nb, bs;
        ctx->GetAttr("num_blocks", nb);
        ctx->GetAttr("block_size", bs);
        require(nb > 0 && bs > 0 && nb <= INT32_MAX && bs <= INT32_MAX,
                "num_blocks and block_size must be > 0");
        const tecoopsDataType_t t = ctx->GetInputDataType("key");
        const size_t cache_bytes =
            static_cast<size_t>(nb) * bs * ks[1] * ks[2] * elem_bytes(t);
        char *base = static_cast<char *>(ctx->GetOutputDataPtr(0));
        tecoopsHandle_t h = handle_.bind(ctx->GetStream());
        check(tecoopsMemset(h, base, 0, 2 * cache_bytes), "plugin_reshape_and_cache memset");
        check(tecoopsReshapeAndCacheEx(h, ctx->GetInputDataPtr("key"), ctx->GetInputDataPtr("value"),
                                       static_cast<const int64_t *>(ctx->GetInputDataPtr("slot_mapping")),
                                       base, base + cache_bytes, ks[0], ks[1], ks[2],
                                       static_cast<int>(nb), static_cast<int>(bs), t),
              "plugin_reshape_and_cache");
    }

 private:
    PluginHandle handle_;
};

// ------------------------------------------------------------- causal_conv1d

struct plugin_causal_conv1d_fnAttrs {
    static void Declare(AttrDecl &d) {
        d.Field("pad_slot_id", int64_t{-1}, "Padding slot ID")
            .Field("conv_state_stride", int64_t{0}, "Stride between conv state entries (elements)")
            .Field("x_seq_stride", int64_t{0}, "Stride between tokens of x (elements)")
            .Field("out_seq_stride", int64_t{0}, "Stride between tokens of out (elements)")
            .Field("api_mode", int64_t{0}, "API mode (0 = respect hasInitialState)")
            .Field("act_mode", int64_t{0}, "Activation mode");
    }
};

// Outputs (out like x, conv_state_out like convState), both zeroed first.
class PluginCausalConv1dFnImpl : public AbstractPluginOp {
 public:
    void InferOutputShape(const std::vector<std::vector<int>> &in, int, std::vector<std::vector<int>> &out,
                          int, const OpAttr &) override {
        out[0] = in[0];
        out[1] = in[5];
    }
    void Enqueue(std::shared_ptr<ComputeContext> &ctx) override {
        std::vector<int> xs, ws, qs, ss;
        ctx->GetInputShape("x", xs);
        ctx->GetInputShape("weight", ws);
        ctx->GetInputShape("queryStartLoc", qs);
        ctx->GetInputShape("convState", ss);
        require(xs.size() == 2, "x must be [total_seqlen, dim]");
        require(ws.size() == 2 && ws[1] == xs[1], "weight must be [width, dim]");
        require(qs.size() == 1 && qs[0] >= 2, "queryStartLoc must be [batch + 1]");
        require(ss.size() == 3, "convState must be [num_entries, width - 1, dim]");
        int64_t pad, css, xss, oss, api, act;
        ctx->GetAttr("pad_slot_id", pad);
        ctx->GetAttr("conv_state_stride", css);
        ctx->GetAttr("x_seq_stride", xss);
        ctx->GetAttr("out_seq_stride", oss);
        ctx->GetAttr("api_mode", api);
        ctx->GetAttr("act_mode", act);
        const int total = xs[0], dim = xs[1], width = ws[0], batch = qs[0] - 1;
        if (css == 0) css = static_cast<int64_t>(width - 1) * dim;
        if (xss == 0) xss = dim;
        if (oss == 0) oss = dim;
        const tecoopsDataType_t t = ctx->GetInputDataType("x");
        require(t == TECOOPS_DATA_HALF, "plugin_causal_conv1d_fn computes in fp16");
        const size_t out_bytes = static_cast<size_t>(total) * dim * 2;
        const size_t state_bytes = static_cast<size_t>(numel(ss)) * 2;
        void *state = ctx->GetInputDataPtr("convState");
        void *state_out = ctx->GetOutputDataPtr(1);
        hipStream_t stream = ctx->GetStream();
        tecoopsHandle_t h = handle_.bind(stream);
        check(tecoopsMemset(h, ctx->GetOutputDataPtr(0), 0, out_bytes), "conv1d memset out");
        check(tecoopsMemset(h, state_out, 0, state_bytes), "conv1d memset state");
        check(tecoopsCausalConv1d(h, batch, total, dim, width, static_cast<int>(css),
                                  static_cast<int>(xss), static_cast<int>(oss), static_cast<int>(pad),
                                  static_cast<int>(api), static_cast<int>(act), ctx->GetInputDataPtr("x"),
                                  state, ctx->GetInputDataPtr("weight"), ctx->GetOutputDataPtr(0),
                                  static_cast<const int *>(ctx->GetInputDataPtr("queryStartLoc")),
                                  static_cast<const int *>(ctx->GetInputDataPtr("convStateIndices")),
                                  static_cast<const int8_t *>(ctx->GetInputDataPtr("hasInitialState"))),
              "plugin_causal_conv1d_fn");
        if (state_bytes != 0 && state_out != state)
            check_hip(hipMemcpyAsync(state_out, state, state_bytes, hipMemcpyDeviceToDevice, stream),
                      "conv1d state copy");
    }

 private:
    PluginHandle handle_;
};

// ----------------------------------------------------------- flash_attention

struct plugin_flash_attentionAttrs {
    static void Declare(AttrDecl &d) {
        d.Field("max_seqlen_q", int64_t{0}, "Max Q length")
            .Field("max_seqlen_k", int64_t{0}, "Max K length")
            .Field("max_block_num", int64_t{0}, "Max number of blocks in cache")
            // Extensions (the reference has neither): <= 0 means 1/sqrt(head_size).
            .Field("softmax_scale", -1.0, "Softmax scale")
            .Field("causal", int64_t{1}, "Bottom-right causal mask");
    }
};

class PluginFlashAttentionImpl : public AbstractPluginOp {
 public:
    void InferOutputShape(const std::vector<std::vector<int>> &in, int, std::vector<std::vector<int>> &out,
                          int, const OpAttr &) override {
        out[0] = in[0];
    }
    void Enqueue(std::shared_ptr<ComputeContext> &ctx) override {
        std::vector<int> qs, ks, vs, bts, cus;
        ctx->GetInputShape("q", qs);
        ctx->GetInputShape("k_cache", ks);
        ctx->GetInputShape("v_cache", vs);
        ctx->GetInputShape("block_table", bts);
        ctx->GetInputShape("cu_seqlens_q", cus);
        require(qs.size() == 3, "q must be [total_tokens, num_heads, head_size]");
        require(ks.size() == 4 && vs == ks, "caches must be [num_blocks, kv_heads, block_size, head_size]");
        require(bts.size() == 2, "block_table must be [batch, max_blocks]");
        require(cus.size() == 1 && cus[0] == bts[0] + 1, "cu_seqlens_q must be [batch + 1]");
        int64_t max_q, max_k;
        double scale;
        int64_t causal;
        ctx->GetAttr("max_seqlen_q", max_q);
        ctx->GetAttr("max_seqlen_k", max_k);
        ctx->GetAttr("softmax_scale", scale);
        ctx->GetAttr("causal", causal);
        // Unset bounds (<= 0) go through as they are: the library derives them
        // from the shapes (the mean q length, the block-table width * block
        // size).  The reference sets neither.
        require(max_q <= INT32_MAX && max_k <= INT32_MAX, "max_seqlen out of range");
        const tecoopsDataType_t t = ctx->GetInputDataType("q");
        Desc bt_d(TECOOPS_DATA_INT32, bts), q_d(t, qs), k_d(t, ks), v_d(t, vs), o_d(t, qs);
        hipStream_t stream = ctx->GetStream();
        tecoopsHandle_t h = handle_.bind(stream);
        const auto *cu = static_cast<const int *>(ctx->GetInputDataPtr("cu_seqlens_q"));
        const auto *kv = static_cast<const int *>(ctx->GetInputDataPtr("seqused_k"));
        // An engine capturing its stream into a graph gets the allocation-free
        // entry point: the handle's split-KV scratch can be freed by a later
        // call while the graph still holds its address.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
            (void)hipGetLastError();
            cs = hipStreamCaptureStatusNone;
        }
        if (cs != hipStreamCaptureStatusNone)
            check(tecoopsFlashAttentionNoAlloc(
                      h, static_cast<int>(max_q), static_cast<int>(max_k), nullptr, cu, kv, bt_d,
                      ctx->GetInputDataPtr("block_table"), q_d, ctx->GetInputDataPtr("q"), k_d,
                      ctx->GetInputDataPtr("k_cache"), v_d, ctx->GetInputDataPtr("v_cache"), o_d,
                      ctx->GetOutputDataPtr(0), static_cast<float>(scale), static_cast<int>(causal != 0)),
                  "plugin_flash_attention");
        else
            check(tecoopsFlashAttentionEx(
                      h, static_cast<int>(max_q), static_cast<int>(max_k), nullptr, cu, kv, bt_d,
                      ctx->GetInputDataPtr("block_table"), q_d, ctx->GetInputDataPtr("q"), k_d,
                      ctx->GetInputDataPtr("k_cache"), v_d, ctx->GetInputDataPtr("v_cache"), o_d,
                      ctx->GetOutputDataPtr(0), static_cast<float>(scale), static_cast<int>(causal != 0),
                      nullptr),
                  "plugin_flash_attention");
    }

 private:
    PluginHandle handle_;
};

}  // namespace

REGISTER_PLUGIN_OP_IMPL(plugin_rms_norm, PluginRmsNormImpl)
PLUGIN_REGISTER_OP("plugin_rms_norm")
    .Input("input").Type("Tensor").Desc("Input tensor [num_tokens, hidden_size]")
    .Input("weight").Type("Tensor").Desc("Weight tensor [hidden_size]")
    .AttrType<plugin_rms_normAttrs>()
    .Register();

REGISTER_PLUGIN_OP_IMPL(plugin_rms_norm_add, PluginRmsNormAddImpl)
PLUGIN_REGISTER_OP("plugin_rms_norm_add")
    .Input("input").Type("Tensor").Desc("Input tensor [num_tokens, hidden_size]")
    .Input("weight").Type("Tensor").Desc("Weight tensor [hidden_size]")
    .Input("residual").Type("Tensor").Desc("Residual tensor [num_tokens, hidden_size]")
    .AttrType<plugin_rms_norm_addAttrs>()
    .NumOfOut(2)
    .Register();

REGISTER_PLUGIN_OP_IMPL(plugin_reshape_and_cache, PluginReshapeAndCacheImpl)
PLUGIN_REGISTER_OP("plugin_reshape_and_cache")
    .Input("key").Type("Tensor").Desc("Key input with shape [num_tokens, num_kv_heads, head_size]")
    .Input("value").Type("Tensor").Desc("Value input with shape [num_tokens, num_kv_heads, head_size]")
    .Input("slot_mapping").Type("Tensor").Desc("Slot mapping with shape [num_tokens]")
    .AttrType<plugin_reshape_and_cacheAttrs>()
    .Register();

REGISTER_PLUGIN_OP_IMPL(plugin_causal_conv1d_fn, PluginCausalConv1dFnImpl)
PLUGIN_REGISTER_OP("plugin_causal_conv1d_fn")
    .Input("x").Type("Tensor").Desc("Input tensor [total_seqlen, dim]")
    .Input("weight").Type("Tensor").Desc("Weight tensor [width, dim]")
    .Input("queryStartLoc").Type("Tensor").Desc("Query start locations [batch + 1] int32")
    .Input("convStateIndices").Type("Tensor").Desc("Conv state cache indices [batch] int32")
    .Input("hasInitialState").Type("Tensor").Desc("Whether each batch has an initial state [batch] int8")
    .Input("convState").Type("Tensor").Desc("Conv state cache [num_entries, width-1, dim]")
    .AttrType<plugin_causal_conv1d_fnAttrs>()
    .NumOfOut(2)
    .Register();

REGISTER_PLUGIN_OP_IMPL(plugin_flash_attention, PluginFlashAttentionImpl)
PLUGIN_REGISTER_OP("plugin_flash_attention")
    .Input("q").Type("Tensor").Desc("Query: [total_tokens, num_heads, head_size]")
    .Input("k_cache").Type("Tensor").Desc("K cache: [num_blocks, kv_heads, block_size, head_size]")
    .Input("v_cache").Type("Tensor").Desc("V cache: [num_blocks, kv_heads, block_size, head_size]")
    .Input("block_table").Type("Tensor").Desc("Block table: [batch_size, block_table_dim]")
    .Input("cu_seqlens_q").Type("Tensor").Desc("Cumulative Q seq lens: [batch_size + 1]")
    .Input("seqused_k").Type("Tensor").Desc("KV seq used per batch: [batch_size]")
    .AttrType<plugin_flash_attentionAttrs>()
    .Register();

}  // namespace TECO_INFER
