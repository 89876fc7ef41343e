// torch_ext.cpp — TORCH_LIBRARY(tecoops) registration of the operator path.
//
// Replaces the reference's pybind11 module api/torch_ext.cpp:208-215 (whose
// README claims a TORCH_LIBRARY registration it does not have) with real
// torch op schemas: the same op names and positional arguments
// (torch_ext.cpp:61-206), outputs mutated in place and annotated Tensor(a!),
// returning nothing.  Every op binds the current HIP stream of the calling
// thread (the reference never sets a stream, torch_ext.cpp:35-42) and calls
// the C ABI of libtecoops.so; a non-success status raises.
//
// Differences from the reference wrappers: flash_attn_varlen_func keeps
// cu_seqlens_q on the device (no host copy, torch_ext.cpp:119-126), honours
// softmax_scale / causal and takes the element type (fp16 or bf16) from q;
// causal_conv1d_fn_torch reads the [dim, tokens] layout in place instead of
// two transposing copies (torch_ext.cpp:186-205).
#include <c10/hip/HIPStream.h>
#include <torch/library.h>
#include <ATen/ATen.h>
#include <ATen/Tensor.h>

#include <algorithm>
#include <unordered_map>

#include "tecoops.h"

namespace {

using at::Tensor;

// One handle per (thread, device), bound to that thread's current stream of
// the device on every call: threads never share a handle, so concurrent
// callers cannot race on its stream.
struct HandleCache {
    std::unordered_map<int, tecoopsHandle_t> by_device;
    ~HandleCache() {
        for (auto &kv : by_device) tecoopsDestroy(kv.second);
    }
};

tecoopsHandle_t handle_for(const Tensor &t) {
    thread_local HandleCache cache;
    const int dev = t.get_device();
    auto it = cache.by_device.find(dev);
    tecoopsHandle_t h;
    if (it == cache.by_device.end()) {
        TORCH_CHECK(tecoopsCreate(&h) == TECOOPS_STATUS_SUCCESS, "tecoopsCreate failed");
        cache.by_device.emplace(dev, h);
    } else {
        h = it->second;
    }
    tecoopsSetStream(h, c10::hip::getCurrentHIPStream(dev).stream());
    return h;
}

void check(tecoopsStatus_t st, const char *what) {
    TORCH_CHECK(st == TECOOPS_STATUS_SUCCESS, what, ": ", tecoopsGetErrorString(st));
}

tecoopsDataType_t dtype_of(const Tensor &t) {
    if (t.scalar_type() == at::kHalf) return TECOOPS_DATA_HALF;
    if (t.scalar_type() == at::kBFloat16) return TECOOPS_DATA_BFLOAT16;
    TORCH_CHECK(false, "tecoops: unsupported dtype ", t.scalar_type(), " (float16 or bfloat16)");
}

void need_cuda(std::initializer_list<const Tensor *> ts) {
    for (const Tensor *t : ts)
        if (t && t->defined()) TORCH_CHECK(t->is_cuda(), "tecoops: tensors must be on the GPU");
}

// The C ABI takes plain pointers with packed row-major extents.
void need_contiguous(std::initializer_list<const Tensor *> ts) {
    for (const Tensor *t : ts)
        if (t && t->defined())
            TORCH_CHECK(t->is_contiguous(), "tecoops: tensors must be contiguous");
}

void need_dtype(const Tensor &t, at::ScalarType st, const char *name) {
    TORCH_CHECK(t.scalar_type() == st, "tecoops: ", name, " must be ", st, ", got ",
                t.scalar_type());
}

struct Desc {
    tecoopsTensorDescriptor_t d = nullptr;
    Desc(const Tensor &t, tecoopsDataType_t dt) {
        check(tecoopsCreateTensorDescriptor(&d), "tecoopsCreateTensorDescriptor");
        std::vector<int> dims(t.dim()), strides(t.dim());
        for (int i = 0; i < t.dim(); ++i) {
            dims[i] = static_cast<int>(t.size(i));
            strides[i] = static_cast<int>(t.stride(i));
        }
        check(tecoopsSetTensorNdDescriptor(d, dt, t.dim(), dims.data(), strides.data()),
              "tecoopsSetTensorNdDescriptor");
    }
    ~Desc() { tecoopsDestroyTensorDescriptor(d); }
};

// reference torch_ext.cpp:61-79
void reshape_and_cache(const Tensor &key, const Tensor &value, const Tensor &slot_mapping,
                       Tensor &key_cache, Tensor &value_cache) {
    need_cuda({&key, &value, &slot_mapping, &key_cache, &value_cache});
    need_contiguous({&key, &value, &slot_mapping, &key_cache, &value_cache});
    TORCH_CHECK(slot_mapping.scalar_type() == at::kLong, "slot_mapping must be int64");
    TORCH_CHECK(key.dim() == 3 && key_cache.dim() == 4 && value.sizes() == key.sizes() &&
                    value_cache.sizes() == key_cache.sizes() &&
                    slot_mapping.numel() == key.size(0),
                "reshape_and_cache: key/value [T, Hkv, D], caches [blocks, Hkv, bs, D], "
                "slot_mapping [T]");
    check(tecoopsReshapeAndCacheEx(handle_for(key), key.data_ptr(), value.data_ptr(),
                                   slot_mapping.data_ptr<int64_t>(), key_cache.data_ptr(),
                                   value_cache.data_ptr(), key.size(0), key.size(1), key.size(2),
                                   key_cache.size(0), key_cache.size(2), dtype_of(key)),
          "reshape_and_cache");
}

// reference torch_ext.cpp:81-97
void rms_norm(const Tensor &input, const Tensor &weight, const c10::optional<Tensor> &residual,
              Tensor &output, const c10::optional<Tensor> &residual_out, double eps) {
    need_cuda({&input, &weight, &output});
    const Tensor *res = residual.has_value() ? &*residual : nullptr;
    const Tensor *res_out = residual_out.has_value() ? &*residual_out : nullptr;
    need_contiguous({&input, &weight, &output, res, res_out});
    // leading dimensions are rows, as in the plugin
    const int64_t D = input.size(-1);
    const int64_t N = D ? input.numel() / D : 0;
    const at::ScalarType st = input.scalar_type();
    need_dtype(weight, st, "weight");
    need_dtype(output, st, "output");
    TORCH_CHECK(weight.numel() == D && output.numel() == input.numel(),
                "rms_norm: weight must hold hidden_size elements and output match input");
    for (const Tensor *t : {res, res_out})
        if (t) {
            need_dtype(*t, st, "residual");
            TORCH_CHECK(t->numel() == input.numel(), "rms_norm: residual tensors must match input");
        }
    check(tecoopsRmsNormEx(handle_for(input), input.data_ptr(), weight.data_ptr(),
                           res ? res->data_ptr() : nullptr, output.data_ptr(),
                           res_out ? res_out->data_ptr() : nullptr, N, D,
                           static_cast<float>(eps), dtype_of(input)),
          "rms_norm");
}

// reference torch_ext.cpp:99-165
void flash_attn_varlen_func(const Tensor &q, const Tensor &k, const Tensor &v,
                            int64_t max_seqlen_q, const Tensor &cu_seqlens_q,
                            int64_t max_seqlen_k, const c10::optional<Tensor> &cu_seqlens_k,
                            const Tensor &seqused_k, double softmax_scale, bool causal,
                            const c10::optional<Tensor> &window_size, const Tensor &block_table,
                            bool return_softmax_lse, Tensor &out) {
    (void)cu_seqlens_k;
    (void)window_size;
    (void)return_softmax_lse;  // accepted and ignored, as in the reference
    need_cuda({&q, &k, &v, &cu_seqlens_q, &seqused_k, &block_table, &out});
    const tecoopsDataType_t dt = dtype_of(q);
    Desc bt(block_table, TECOOPS_DATA_INT32), qd(q, dt), kd(k, dt), vd(v, dt), od(out, dt);
    // The split-KV workspace comes from torch's allocator: stream-ordered like
    // any tensor, and taken from the graph's pool under CUDA-graph capture,
    // where the handle's own scratch (hipMalloc on a stream's first use) could
    // not be allocated.  The launch hints are the ones the library derives
    // without a workspace (mean q length; max_seqlen_k capped by the
    // block-table width * block size), so the plan and results are unchanged:
    // max_seqlen_q raised to the mean q length, max_seqlen_k capped by (or,
    // when <= 0, taken as) the block-table width * block size.
    int q_hint = static_cast<int>(max_seqlen_q), k_hint = static_cast<int>(max_seqlen_k);
    Tensor ws;
    if (q.dim() == 3 && k.dim() == 4 && block_table.dim() == 2 && block_table.size(0) > 0) {
        const int64_t batch = block_table.size(0);
        const int64_t cap = std::min<int64_t>(block_table.size(1) * k.size(2), 0x7fffffff);
        const int64_t q_mean = std::max<int64_t>(1, (q.size(0) + batch - 1) / batch);
        q_hint = static_cast<int>(std::min<int64_t>(std::max(max_seqlen_q, q_mean), 0x7fffffff));
        k_hint = static_cast<int>(max_seqlen_k > 0 ? std::min<int64_t>(max_seqlen_k, cap) : cap);
        size_t bytes = 0;
        if (k_hint > 0 &&
            tecoopsGetFlashAttentionWorkspaceSize(static_cast<int>(batch), static_cast<int>(q.size(1)),
                                                  static_cast<int>(q.size(2)), q_hint, k_hint,
                                                  &bytes) == TECOOPS_STATUS_SUCCESS &&
            bytes > 0)
            ws = at::empty({static_cast<int64_t>(bytes)}, q.options().dtype(at::kByte));
    }
    if (!ws.defined()) {
        q_hint = static_cast<int>(max_seqlen_q);
        k_hint = static_cast<int>(max_seqlen_k);
    }
    check(tecoopsFlashAttentionEx(handle_for(q), q_hint, k_hint, nullptr,
                                  cu_seqlens_q.data_ptr<int>(), seqused_k.data_ptr<int>(), bt.d,
                                  block_table.data_ptr(), qd.d, q.data_ptr(), kd.d, k.data_ptr(),
                                  vd.d, v.data_ptr(), od.d, out.data_ptr(),
                                  softmax_scale > 0 ? static_cast<float>(softmax_scale) : -1.0f,
                                  causal ? 1 : 0, ws.defined() ? ws.data_ptr() : nullptr),
          "flash_attn_varlen_func");
}

// reference torch_ext.cpp:167-206; x / out [dim, tokens], weight [width, dim]
void causal_conv1d_fn_torch(Tensor &out, Tensor &conv_states, const Tensor &x,
                            const Tensor &weight, const Tensor &query_start_loc,
                            const Tensor &cache_indices, const Tensor &has_initial_state,
                            int64_t pad_slot_id) {
    need_cuda({&out, &conv_states, &x, &weight, &query_start_loc, &cache_indices,
               &has_initial_state});
    const int dim = x.size(0), total = x.size(1);
    check(tecoopsCausalConv1dEx(handle_for(x), query_start_loc.size(0) - 1, total, dim,
                                weight.size(0), x.data_ptr(), 0, x.stride(1), x.stride(0),
                                out.data_ptr(), 0, out.stride(1), out.stride(0),
                                weight.data_ptr(), weight.stride(1), weight.stride(0), nullptr,
                                conv_states.data_ptr(), conv_states.stride(0),
                                query_start_loc.data_ptr<int>(), cache_indices.data_ptr<int>(),
                                has_initial_state.data_ptr<int8_t>(),
                                static_cast<int>(pad_slot_id), 0, 1),
          "causal_conv1d_fn_torch");
}

// ------------------------------------------------------------ extensions

void causal_conv1d(const Tensor &x, const Tensor &weight, const c10::optional<Tensor> &bias,
                   Tensor &out, const c10::optional<Tensor> &conv_states, bool silu) {
    need_cuda({&x, &weight, &out});
    check(tecoopsCausalConv1dEx(handle_for(x), x.size(0), x.size(2), x.size(1), weight.size(1),
                                x.data_ptr(), x.stride(0), x.stride(2), x.stride(1),
                                out.data_ptr(), out.stride(0), out.stride(2), out.stride(1),
                                weight.data_ptr(), weight.stride(0), weight.stride(1),
                                bias.has_value() ? bias->data_ptr() : nullptr,
                                conv_states.has_value() ? conv_states->data_ptr() : nullptr,
                                conv_states.has_value() ? conv_states->stride(0) : 0, nullptr,
                                nullptr, nullptr, -1, 0, silu ? 1 : 0),
          "causal_conv1d");
}

void rotary_embedding(const Tensor &positions, Tensor &query, const c10::optional<Tensor> &key,
                      int64_t head_size, const c10::optional<Tensor> &cos_sin_cache,
                      bool is_neox, double base, int64_t rot_dim) {
    need_cuda({&positions, &query});
    const int64_t T = positions.numel();
    const int H = query.numel() / (T * head_size);
    const int Hkv = key.has_value() ? key->numel() / (T * head_size) : 0;
    const int rd = rot_dim > 0 ? rot_dim
                               : (cos_sin_cache.has_value() ? cos_sin_cache->size(1) : head_size);
    check(tecoopsRotaryEmbedding(handle_for(query), positions.data_ptr<int64_t>(),
                                 query.data_ptr(), key.has_value() ? key->data_ptr() : nullptr,
                                 T, H, Hkv, head_size, rd, query.stride(0),
                                 key.has_value() ? key->stride(0) : 0,
                                 cos_sin_cache.has_value() ? cos_sin_cache->data_ptr<float>()
                                                           : nullptr,
                                 cos_sin_cache.has_value() ? cos_sin_cache->size(0) : 0,
                                 static_cast<float>(base), is_neox ? 1 : 0, dtype_of(query)),
          "rotary_embedding");
}

void rotary_reshape_and_cache(const Tensor &positions, Tensor &query, Tensor &key,
                              const Tensor &value, const Tensor &slot_mapping, Tensor &key_cache,
                              Tensor &value_cache, int64_t head_size,
                              const c10::optional<Tensor> &cos_sin_cache, bool is_neox,
                              double base, int64_t rot_dim, bool write_key) {
    need_cuda({&positions, &query, &key, &value, &slot_mapping, &key_cache, &value_cache});
    const int64_t T = positions.numel();
    const int H = query.numel() / (T * head_size);
    const int Hkv = key.numel() / (T * head_size);
    const int rd = rot_dim > 0 ? rot_dim
                               : (cos_sin_cache.has_value() ? cos_sin_cache->size(1) : head_size);
    check(tecoopsRotaryReshapeAndCache(
              handle_for(query), positions.data_ptr<int64_t>(), query.data_ptr(), key.data_ptr(),
              value.data_ptr(), slot_mapping.data_ptr<int64_t>(), key_cache.data_ptr(),
              value_cache.data_ptr(), T, H, Hkv, head_size, rd, query.stride(0), key.stride(0),
              value.stride(0),
              cos_sin_cache.has_value() ? cos_sin_cache->data_ptr<float>() : nullptr,
              cos_sin_cache.has_value() ? cos_sin_cache->size(0) : 0, static_cast<float>(base),
              is_neox ? 1 : 0, key_cache.size(0), key_cache.size(2), write_key ? 1 : 0,
              dtype_of(query)),
          "rotary_reshape_and_cache");
}

void gemv(const Tensor &weight, const Tensor &x, Tensor &out) {
    need_cuda({&weight, &x, &out});
    need_contiguous({&weight, &x, &out});
    need_dtype(weight, x.scalar_type(), "weight");
    need_dtype(out, x.scalar_type(), "out");
    const int B = x.dim() == 2 ? x.size(0) : 1;
    TORCH_CHECK(weight.dim() == 2 && x.size(-1) == weight.size(1) &&
                    out.numel() == B * weight.size(0),
                "gemv: weight [N, K], x [B, K], out [B, N]");
    check(tecoopsGemv(handle_for(x), weight.data_ptr(), x.data_ptr(), out.data_ptr(), B,
                      weight.size(0), weight.size(1), dtype_of(x)),
          "gemv");
}

void gemv_int8(const Tensor &weight, const Tensor &scales, const Tensor &x, Tensor &out) {
    need_cuda({&weight, &scales, &x, &out});
    need_contiguous({&weight, &scales, &x, &out});
    need_dtype(weight, at::kChar, "weight");
    need_dtype(scales, at::kHalf, "scales");
    need_dtype(x, at::kHalf, "x");
    need_dtype(out, at::kHalf, "out");
    const int B = x.dim() == 2 ? x.size(0) : 1;
    TORCH_CHECK(weight.dim() == 2 && x.size(-1) == weight.size(1) &&
                    out.numel() == B * weight.size(0) && scales.numel() == weight.size(0),
                "gemv_int8: weight [N, K], scales [N], x [B, K], out [B, N]");
    check(tecoopsGemvInt8(handle_for(x), weight.data_ptr<int8_t>(), scales.data_ptr(),
                          x.data_ptr(), out.data_ptr(), B, weight.size(0), weight.size(1)),
          "gemv_int8");
}

void memset_(Tensor &t, int64_t value) {
    need_cuda({&t});
    check(tecoopsMemset(handle_for(t), t.data_ptr(), static_cast<int>(value),
                        t.numel() * t.element_size()),
          "memset");
}

}  // namespace

TORCH_LIBRARY(tecoops, m) {
    m.def("reshape_and_cache(Tensor key, Tensor value, Tensor slot_mapping, "
          "Tensor(a!) key_cache, Tensor(b!) value_cache) -> ()");
    m.def("rms_norm(Tensor input, Tensor weight, Tensor? residual, Tensor(a!) output, "
          "Tensor(b!)? residual_out, float eps) -> ()");
    m.def("flash_attn_varlen_func(Tensor q, Tensor k, Tensor v, int max_seqlen_q, "
          "Tensor cu_seqlens_q, int max_seqlen_k, Tensor? cu_seqlens_k, Tensor seqused_k, "
          "float softmax_scale, bool causal, Tensor? window_size, Tensor block_table, "
          "bool return_softmax_lse, Tensor(a!) out) -> ()");
    m.def("causal_conv1d_fn_torch(Tensor(a!) out, Tensor(b!) conv_states, Tensor x, "
          "Tensor weight, Tensor query_start_loc, Tensor cache_indices, "
          "Tensor has_initial_state, int pad_slot_id) -> ()");
    m.def("causal_conv1d(Tensor x, Tensor weight, Tensor? bias, Tensor(a!) out, "
          "Tensor(b!)? conv_states, bool silu) -> ()");
    m.def("rotary_embedding(Tensor positions, Tensor(a!) query, Tensor(b!)? key, int head_size, "
          "Tensor? cos_sin_cache, bool is_neox, float base, int rot_dim) -> ()");
    m.def("rotary_reshape_and_cache(Tensor positions, Tensor(a!) query, Tensor(b!) key, "
          "Tensor value, Tensor slot_mapping, Tensor(c!) key_cache, Tensor(d!) value_cache, "
          "int head_size, Tensor? cos_sin_cache, bool is_neox, float base, int rot_dim, "
          "bool write_key) -> ()");
    m.def("gemv(Tensor weight, Tensor x, Tensor(a!) out) -> ()");
    m.def("gemv_int8(Tensor weight, Tensor scales, Tensor x, Tensor(a!) out) -> ()");
    m.def("memset(Tensor(a!) t, int value) -> ()");
}

TORCH_LIBRARY_IMPL(tecoops, CUDA, m) {
    m.impl("reshape_and_cache", &reshape_and_cache);
    m.impl("rms_norm", &rms_norm);
    m.impl("flash_attn_varlen_func", &flash_attn_varlen_func);
    m.impl("causal_conv1d_fn_torch", &causal_conv1d_fn_torch);
    m.impl("causal_conv1d", &causal_conv1d);
    m.impl("rotary_embedding", &rotary_embedding);
    m.impl("rotary_reshape_and_cache", &rotary_reshape_and_cache);
    m.impl("gemv", &gemv);
    m.impl("gemv_int8", &gemv_int8);
    m.impl("memset", &memset_);
}
