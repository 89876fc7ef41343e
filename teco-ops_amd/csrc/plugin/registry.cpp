// registry.cpp — plugin registry and the C entry points that drive plugins
// the way an inference engine does (create an instance per graph node, infer
// output shapes, enqueue on a HIP stream).
//
// The registry plays the part of the engine-side tables that
// REGISTER_PLUGIN_OP_IMPL / PLUGIN_REGISTER_OP fill in the reference
// (doc/README_PLUGIN.md:103-141).  Host code only: no device calls here.
#include <cctype>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <sstream>

#include "tecoops_plugin.h"

namespace TECO_INFER {

PluginRegistry &PluginRegistry::Get() {
    static PluginRegistry r;
    return r;
}

void PluginRegistry::AddImpl(const std::string &name, PluginFactory f) {
    impls_[name] = std::move(f);
}

void PluginRegistry::AddSpec(const PluginOpSpec &spec) { specs_[spec.name] = spec; }

const PluginOpSpec *PluginRegistry::FindSpec(const std::string &name) const {
    auto it = specs_.find(name);
    return it == specs_.end() ? nullptr : &it->second;
}

std::unique_ptr<AbstractPluginOp> PluginRegistry::Create(const std::string &name) const {
    auto it = impls_.find(name);
    if (it == impls_.end()) return nullptr;
    return it->second();
}

std::vector<std::string> PluginRegistry::Names() const {
    std::vector<std::string> out;
    for (const auto &kv : impls_)
        if (specs_.count(kv.first)) out.push_back(kv.first);
    return out;
}

}  // namespace TECO_INFER

struct tecoopsPluginInstance {
    std::string name;
    const TECO_INFER::PluginOpSpec *spec;
    std::unique_ptr<TECO_INFER::AbstractPluginOp> op;
};

namespace {

using TECO_INFER::AttrValue;
using TECO_INFER::OpAttr;
using TECO_INFER::PluginError;

std::string trim(const std::string &s) {
    size_t a = 0, b = s.size();
    while (a < b && std::isspace(static_cast<unsigned char>(s[a]))) ++a;
    while (b > a && std::isspace(static_cast<unsigned char>(s[b - 1]))) --b;
    return s.substr(a, b - a);
}

AttrValue parse_value(const std::string &name, const std::string &text) {
    const std::string t = trim(text);
    if (t.empty()) throw PluginError(TECOOPS_STATUS_BAD_PARAM, "empty value for '" + name + "'");
    if (t.front() == '[') {
        if (t.back() != ']')
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "unterminated list for '" + name + "'");
        std::vector<int64_t> v;
        std::stringstream ss(t.substr(1, t.size() - 2));
        std::string item;
        while (std::getline(ss, item, ',')) {
            item = trim(item);
            if (item.empty()) continue;
            char *end = nullptr;
            const long long x = std::strtoll(item.c_str(), &end, 10);
            if (*end != '\0')
                throw PluginError(TECOOPS_STATUS_BAD_PARAM, "bad list item for '" + name + "'");
            v.push_back(x);
        }
        return AttrValue(v);
    }
    char *end = nullptr;
    const long long i = std::strtoll(t.c_str(), &end, 10);
    if (*end == '\0') return AttrValue(static_cast<int64_t>(i));
    const double d = std::strtod(t.c_str(), &end);
    if (*end == '\0') return AttrValue(d);
    return AttrValue(t);
}

// Registered defaults, then "name=value;..." overrides (unknown names are an error).
OpAttr make_attrs(const TECO_INFER::PluginOpSpec &spec, const char *text) {
    OpAttr attr;
    for (const auto &f : spec.attrs.fields()) attr.Set(f.name, f.def);
    if (text == nullptr) return attr;
    std::stringstream ss(text);
    std::string item;
    while (std::getline(ss, item, ';')) {
        if (trim(item).empty()) continue;
        const size_t eq = item.find('=');
        if (eq == std::string::npos)
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "attribute without '=': " + item);
        const std::string name = trim(item.substr(0, eq));
        bool known = false;
        for (const auto &f : spec.attrs.fields()) known = known || f.name == name;
        if (!known)
            throw PluginError(TECOOPS_STATUS_BAD_PARAM,
                              "unknown attribute '" + name + "' for " + spec.name);
        attr.Set(name, parse_value(name, item.substr(eq + 1)));
    }
    return attr;
}

std::vector<std::vector<int>> unpack_shapes(int n, const int *ndims, const int *dims) {
    if (n < 0 || (n > 0 && ndims == nullptr))
        throw PluginError(TECOOPS_STATUS_BAD_PARAM, "bad tensor count or shapes");
    std::vector<std::vector<int>> out(n);
    size_t pos = 0;
    for (int i = 0; i < n; ++i) {
        if (ndims[i] < 0 || ndims[i] > TECOOPS_DIM_MAX)
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "tensor rank out of range");
        if (ndims[i] > 0 && dims == nullptr)
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "missing dims");
        out[i].assign(dims + pos, dims + pos + ndims[i]);
        pos += ndims[i];
    }
    return out;
}

template <typename F>
tecoopsStatus_t guarded(const char *what, F &&f) {
    try {
        f();
        return TECOOPS_STATUS_SUCCESS;
    } catch (const PluginError &e) {
        std::fprintf(stderr, "tecoops plugin %s: %s\n", what, e.what());
        return e.status();
    } catch (const std::exception &e) {
        std::fprintf(stderr, "tecoops plugin %s: %s\n", what, e.what());
        return TECOOPS_STATUS_INTERNAL_ERROR;
    }
}

}  // namespace

extern "C" {

int tecoopsPluginCount(void) {
    return static_cast<int>(TECO_INFER::PluginRegistry::Get().Names().size());
}

const char *tecoopsPluginName(int index) {
    // Names are stable for the life of the process; keep them in static storage.
    static std::mutex mu;
    static std::vector<std::string> names;
    std::lock_guard<std::mutex> g(mu);
    names = TECO_INFER::PluginRegistry::Get().Names();
    if (index < 0 || index >= static_cast<int>(names.size())) return nullptr;
    return TECO_INFER::PluginRegistry::Get().FindSpec(names[index])->name.c_str();
}

int tecoopsPluginNumInputs(const char *op) {
    const auto *s = op ? TECO_INFER::PluginRegistry::Get().FindSpec(op) : nullptr;
    return s ? static_cast<int>(s->inputs.size()) : -1;
}

const char *tecoopsPluginInputName(const char *op, int index) {
    const auto *s = op ? TECO_INFER::PluginRegistry::Get().FindSpec(op) : nullptr;
    if (s == nullptr || index < 0 || index >= static_cast<int>(s->inputs.size())) return nullptr;
    return s->inputs[index].name.c_str();
}

int tecoopsPluginNumOutputs(const char *op) {
    const auto *s = op ? TECO_INFER::PluginRegistry::Get().FindSpec(op) : nullptr;
    return s ? s->num_outputs : -1;
}

tecoopsStatus_t tecoopsPluginCreate(const char *op, tecoopsPluginInstance_t *inst) {
    if (op == nullptr || inst == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    const auto &reg = TECO_INFER::PluginRegistry::Get();
    const auto *spec = reg.FindSpec(op);
    if (spec == nullptr) return TECOOPS_STATUS_NOT_SUPPORTED;
    auto impl = reg.Create(op);
    if (!impl) return TECOOPS_STATUS_NOT_SUPPORTED;
    *inst = new tecoopsPluginInstance{op, spec, std::move(impl)};
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsPluginDestroy(tecoopsPluginInstance_t inst) {
    if (inst == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    delete inst;
    return TECOOPS_STATUS_SUCCESS;
}

tecoopsStatus_t tecoopsPluginInferOutputShape(tecoopsPluginInstance_t inst, int n_input,
                                              const int *in_ndims, const int *in_dims,
                                              const char *attrs, int n_output,
                                              int *out_ndims, int *out_dims) {
    if (inst == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    if (out_ndims == nullptr || out_dims == nullptr) return TECOOPS_STATUS_BAD_PARAM;
    return guarded(inst->name.c_str(), [&] {
        if (n_input != static_cast<int>(inst->spec->inputs.size()) ||
            n_output != inst->spec->num_outputs)
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "input / output count mismatch");
        const auto in = unpack_shapes(n_input, in_ndims, in_dims);
        const OpAttr attr = make_attrs(*inst->spec, attrs);
        std::vector<std::vector<int>> out(n_output);
        inst->op->InferOutputShape(in, n_input, out, n_output, attr);
        for (int i = 0; i < n_output; ++i) {
            if (out[i].size() > TECOOPS_DIM_MAX)
                throw PluginError(TECOOPS_STATUS_INTERNAL_ERROR, "output rank out of range");
            out_ndims[i] = static_cast<int>(out[i].size());
            for (size_t d = 0; d < out[i].size(); ++d) out_dims[i * TECOOPS_DIM_MAX + d] = out[i][d];
        }
    });
}

tecoopsStatus_t tecoopsPluginEnqueue(tecoopsPluginInstance_t inst, int n_input,
                                     void *const *in_data, const int *in_dtypes,
                                     const int *in_ndims, const int *in_dims, int n_output,
                                     void *const *out_data, const int *out_dtypes,
                                     const int *out_ndims, const int *out_dims,
                                     const char *attrs, hipStream_t stream) {
    if (inst == nullptr) return TECOOPS_STATUS_NOT_INITIALIZED;
    return guarded(inst->name.c_str(), [&] {
        if (n_input != static_cast<int>(inst->spec->inputs.size()) ||
            n_output != inst->spec->num_outputs)
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "input / output count mismatch");
        if ((n_input > 0 && in_data == nullptr) || (n_output > 0 && out_data == nullptr))
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "missing data pointers");
        const auto ishape = unpack_shapes(n_input, in_ndims, in_dims);
        const auto oshape = unpack_shapes(n_output, out_ndims, out_dims);
        std::vector<TECO_INFER::ComputeContext::Tensor> in(n_input), out(n_output);
        for (int i = 0; i < n_input; ++i) {
            in[i].data = in_data[i];
            in[i].shape = ishape[i];
            if (in_dtypes) in[i].dtype = static_cast<tecoopsDataType_t>(in_dtypes[i]);
        }
        for (int i = 0; i < n_output; ++i) {
            out[i].data = out_data[i];
            out[i].shape = oshape[i];
            if (out_dtypes) out[i].dtype = static_cast<tecoopsDataType_t>(out_dtypes[i]);
        }
        auto ctx = std::make_shared<TECO_INFER::ComputeContext>(
            inst->spec, make_attrs(*inst->spec, attrs), std::move(in), std::move(out), stream);
        inst->op->Enqueue(ctx);
    });
}

}  // extern "C"
