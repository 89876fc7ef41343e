/*
 * tecoops_plugin.h — the inference-engine plugin contract for the tecoops
 * operators, backed by HIP streams.
 *
 * Interface followed: doc/README_PLUGIN.md:56-141 and :343-357 of the
 * reference (AbstractPluginOp::InferOutputShape / Enqueue, ComputeContext,
 * OpAttr::GetAttr<T>, REGISTER_PLUGIN_OP_IMPL and PLUGIN_REGISTER_OP inside
 * namespace TECO_INFER), as used by the reference's teco/plugin sources
 * (e.g. pluginRmsNorm/plugin_rms_norm.cc:52-131).  The engine
 * headers that define these classes upstream (Teco-Inference, TVM attrs) are
 * not part of the operator library, so this header supplies a self-contained
 * version of the contract:
 *
 *   - ComputeContext is a concrete record the engine fills: input / output
 *     device pointers, shapes and element types, the op's attributes and the
 *     hipStream_t to enqueue on.  Inputs are found by index or by the names
 *     the op's registration declares.
 *   - Attribute structs declare their fields with defaults through a static
 *     Declare(AttrDecl&) in place of TVM_DECLARE_ATTRS; .AttrType<T>() on the
 *     registration records them.
 *   - A plugin that cannot run throws PluginError carrying a tecoopsStatus_t;
 *     the C entry points at the end of this header return that status.
 *
 * The C entry points (exported by libtecoops_plugin.so) drive the registered
 * plugins the way an engine would: create an instance, infer output shapes,
 * enqueue on a stream.  ctypes front ends and host tests use them.
 */
#ifndef TECOOPS_PLUGIN_H_
#define TECOOPS_PLUGIN_H_

#include "tecoops.h"

#ifdef __cplusplus
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

namespace TECO_INFER {

/* One attribute value: integer, real, string or integer list. */
struct AttrValue {
    enum Kind { kInt, kReal, kString, kInts } kind = kInt;
    int64_t i = 0;
    double d = 0.0;
    std::string s;
    std::vector<int64_t> v;

    AttrValue() = default;
    AttrValue(int64_t x) : kind(kInt), i(x), d(static_cast<double>(x)) {}
    AttrValue(int x) : AttrValue(static_cast<int64_t>(x)) {}
    AttrValue(double x) : kind(kReal), i(static_cast<int64_t>(x)), d(x) {}
    AttrValue(const std::string &x) : kind(kString), s(x) {}
    AttrValue(const char *x) : kind(kString), s(x) {}
    AttrValue(const std::vector<int64_t> &x) : kind(kInts), v(x) {}
};

class PluginError : public std::runtime_error {
 public:
    PluginError(tecoopsStatus_t st, const std::string &what)
        : std::runtime_error(what), status_(st) {}
    tecoopsStatus_t status() const { return status_; }

 private:
    tecoopsStatus_t status_;
};

/* Attribute set of one op instance (OpAttr::GetAttr<T>(name), README_PLUGIN.md:355). */
class OpAttr {
 public:
    void Set(const std::string &name, const AttrValue &v) { values_[name] = v; }
    bool Has(const std::string &name) const { return values_.count(name) != 0; }

    template <typename T>
    T GetAttr(const std::string &name) const {
        auto it = values_.find(name);
        if (it == values_.end())
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "missing attribute '" + name + "'");
        const AttrValue &a = it->second;
        if constexpr (std::is_same_v<T, std::string>) {
            if (a.kind != AttrValue::kString)
                throw PluginError(TECOOPS_STATUS_BAD_PARAM, "attribute '" + name + "' is not a string");
            return a.s;
        } else if constexpr (std::is_same_v<T, std::vector<int64_t>>) {
            if (a.kind != AttrValue::kInts)
                throw PluginError(TECOOPS_STATUS_BAD_PARAM, "attribute '" + name + "' is not a list");
            return a.v;
        } else {
            static_assert(std::is_arithmetic_v<T>, "numeric, string or int64 list attributes");
            if (a.kind == AttrValue::kString || a.kind == AttrValue::kInts)
                throw PluginError(TECOOPS_STATUS_BAD_PARAM, "attribute '" + name + "' is not numeric");
            if constexpr (std::is_floating_point_v<T>)
                return static_cast<T>(a.kind == AttrValue::kReal ? a.d : static_cast<double>(a.i));
            else
                return static_cast<T>(a.kind == AttrValue::kInt ? a.i : static_cast<int64_t>(a.d));
        }
    }

    const std::map<std::string, AttrValue> &values() const { return values_; }

 private:
    std::map<std::string, AttrValue> values_;
};

/* Field list of an attribute struct: name, default and description. */
class AttrDecl {
 public:
    struct Entry {
        std::string name;
        AttrValue def;
        std::string desc;
    };
    AttrDecl &Field(const std::string &name, const AttrValue &def, const std::string &desc) {
        fields_.push_back({name, def, desc});
        return *this;
    }
    const std::vector<Entry> &fields() const { return fields_; }

 private:
    std::vector<Entry> fields_;
};

/* Declared interface of one plugin op (PLUGIN_REGISTER_OP, README_PLUGIN.md:120-136). */
struct PluginOpSpec {
    struct Port {
        std::string name, type, desc;
    };
    std::string name;
    std::vector<Port> inputs;
    AttrDecl attrs;
    int num_outputs = 1;

    int InputIndex(const std::string &n) const {
        for (size_t i = 0; i < inputs.size(); ++i)
            if (inputs[i].name == n) return static_cast<int>(i);
        return -1;
    }
};

/* Per-launch view the engine hands to Enqueue (README_PLUGIN.md:343-351). */
class ComputeContext {
 public:
    struct Tensor {
        void *data = nullptr;
        std::vector<int> shape;
        tecoopsDataType_t dtype = TECOOPS_DATA_HALF;
    };

    ComputeContext(const PluginOpSpec *spec, OpAttr attr, std::vector<Tensor> inputs,
                   std::vector<Tensor> outputs, hipStream_t stream)
        : spec_(spec), attr_(std::move(attr)), inputs_(std::move(inputs)),
          outputs_(std::move(outputs)), stream_(stream) {}

    void *GetInputDataPtr(int idx) const { return input(idx).data; }
    void *GetInputDataPtr(const std::string &name) const { return input(index(name)).data; }
    void *GetOutputDataPtr(int idx) const {
        if (idx < 0 || idx >= static_cast<int>(outputs_.size()))
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "output index out of range");
        return outputs_[idx].data;
    }
    void GetInputShape(int idx, std::vector<int> &shape) const { shape = input(idx).shape; }
    void GetInputShape(const std::string &name, std::vector<int> &shape) const {
        shape = input(index(name)).shape;
    }
    /* Element type of an input: an extension (the reference plugins assume fp16). */
    tecoopsDataType_t GetInputDataType(const std::string &name) const {
        return input(index(name)).dtype;
    }
    tecoopsDataType_t GetInputDataType(int idx) const { return input(idx).dtype; }
    int NumInputs() const { return static_cast<int>(inputs_.size()); }
    int NumOutputs() const { return static_cast<int>(outputs_.size()); }

    template <typename T>
    void GetAttr(const std::string &name, T &value) const {
        value = attr_.GetAttr<T>(name);
    }
    const OpAttr &Attr() const { return attr_; }
    hipStream_t GetStream() const { return stream_; }

 private:
    int index(const std::string &name) const {
        const int i = spec_ ? spec_->InputIndex(name) : -1;
        if (i < 0) throw PluginError(TECOOPS_STATUS_BAD_PARAM, "unknown input '" + name + "'");
        return i;
    }
    const Tensor &input(int idx) const {
        if (idx < 0 || idx >= static_cast<int>(inputs_.size()))
            throw PluginError(TECOOPS_STATUS_BAD_PARAM, "input index out of range");
        return inputs_[idx];
    }

    const PluginOpSpec *spec_;
    OpAttr attr_;
    std::vector<Tensor> inputs_, outputs_;
    hipStream_t stream_;
};

/* Base class of every plugin (README_PLUGIN.md:56-101). */
class AbstractPluginOp {
 public:
    virtual ~AbstractPluginOp() = default;
    virtual void InferOutputShape(const std::vector<std::vector<int>> &total_input_shape,
                                  int n_input,
                                  std::vector<std::vector<int>> &total_output_shape,
                                  int n_output, const OpAttr &attr) = 0;
    virtual void Enqueue(std::shared_ptr<ComputeContext> &ctx) = 0;
};

using PluginFactory = std::function<std::unique_ptr<AbstractPluginOp>()>;

/* Process-wide registry filled by the registration macros at load time. */
class PluginRegistry {
 public:
    static PluginRegistry &Get();
    void AddImpl(const std::string &name, PluginFactory f);
    void AddSpec(const PluginOpSpec &spec);
    const PluginOpSpec *FindSpec(const std::string &name) const;
    std::unique_ptr<AbstractPluginOp> Create(const std::string &name) const;
    std::vector<std::string> Names() const;

 private:
    std::map<std::string, PluginFactory> impls_;
    std::map<std::string, PluginOpSpec> specs_;
};

struct PluginImplRegistrar {
    PluginImplRegistrar(const char *name, PluginFactory f) {
        PluginRegistry::Get().AddImpl(name, std::move(f));
    }
};

struct PluginSpecRegistrar {
    explicit PluginSpecRegistrar(const PluginOpSpec &spec) { PluginRegistry::Get().AddSpec(spec); }
};

/* Builder behind PLUGIN_REGISTER_OP("name").Input(..).Type(..).Desc(..)... */
class PluginOpBuilder {
 public:
    explicit PluginOpBuilder(const char *name) { spec_.name = name; }
    PluginOpBuilder &Input(const std::string &n) {
        spec_.inputs.push_back({n, "Tensor", ""});
        return *this;
    }
    PluginOpBuilder &Type(const std::string &t) {
        if (!spec_.inputs.empty()) spec_.inputs.back().type = t;
        return *this;
    }
    PluginOpBuilder &Desc(const std::string &d) {
        if (!spec_.inputs.empty()) spec_.inputs.back().desc = d;
        return *this;
    }
    template <typename Attrs>
    PluginOpBuilder &AttrType() {
        Attrs::Declare(spec_.attrs);
        return *this;
    }
    PluginOpBuilder &NumOfOut(int n) {
        spec_.num_outputs = n;
        return *this;
    }
    PluginSpecRegistrar Register() { return PluginSpecRegistrar(spec_); }

 private:
    PluginOpSpec spec_;
};

}  // namespace TECO_INFER

#define TECO_PLUGIN_CAT2(a, b) a##b
#define TECO_PLUGIN_CAT(a, b) TECO_PLUGIN_CAT2(a, b)

/* Binds op name `name` (an identifier) to implementation class `Impl`. */
#define REGISTER_PLUGIN_OP_IMPL(name, Impl)                                         \
    static const ::TECO_INFER::PluginImplRegistrar TECO_PLUGIN_CAT(                \
        teco_plugin_impl_, __COUNTER__)(#name, [] {                                 \
        return std::unique_ptr<::TECO_INFER::AbstractPluginOp>(new Impl());         \
    });

/* Starts the interface declaration of op `name` (a string); ends in .Register(). */
#define PLUGIN_REGISTER_OP(name)                                                    \
    static const ::TECO_INFER::PluginSpecRegistrar TECO_PLUGIN_CAT(                \
        teco_plugin_spec_, __COUNTER__) = ::TECO_INFER::PluginOpBuilder(name)

extern "C" {
#endif /* __cplusplus */

/* ------------------------------------------------------------------------
 * C entry points of libtecoops_plugin.so: an engine-side driver of the
 * registered plugins.  Shapes are passed flattened: tensor i has ndims[i]
 * dimensions, stored consecutively in dims.  Attributes are a string
 * "name=value;name=value" (integers, reals, or [a,b,c] integer lists);
 * attributes not given take the registered defaults.
 * ---------------------------------------------------------------------- */
typedef struct tecoopsPluginInstance *tecoopsPluginInstance_t;

/* Number of registered plugins and the name of the i-th (sorted). */
int tecoopsPluginCount(void);
const char *tecoopsPluginName(int index);

/* Declared inputs and outputs of a plugin; -1 when the name is unknown. */
int tecoopsPluginNumInputs(const char *op);
const char *tecoopsPluginInputName(const char *op, int index);
int tecoopsPluginNumOutputs(const char *op);

/* One plugin instance (the engine keeps one per graph node). */
tecoopsStatus_t tecoopsPluginCreate(const char *op, tecoopsPluginInstance_t *inst);
tecoopsStatus_t tecoopsPluginDestroy(tecoopsPluginInstance_t inst);

/* InferOutputShape: out_ndims[n_output] and out_dims[n_output * 8] are filled. */
tecoopsStatus_t tecoopsPluginInferOutputShape(tecoopsPluginInstance_t inst, int n_input,
                                              const int *in_ndims, const int *in_dims,
                                              const char *attrs, int n_output,
                                              int *out_ndims, int *out_dims);

/* Enqueue on `stream` with caller-allocated device inputs and outputs. */
tecoopsStatus_t tecoopsPluginEnqueue(tecoopsPluginInstance_t inst, int n_input,
                                     void *const *in_data, const int *in_dtypes,
                                     const int *in_ndims, const int *in_dims, int n_output,
                                     void *const *out_data, const int *out_dtypes,
                                     const int *out_ndims, const int *out_dims,
                                     const char *attrs, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TECOOPS_PLUGIN_H_ */
