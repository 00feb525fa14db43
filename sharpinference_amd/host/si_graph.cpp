// Logical graphs, the RWKV-7 forward-token graph and their lowering to HIP
// VM programs (si_graph.hpp).
#include "si_graph.hpp"

#include <algorithm>
#include <charconv>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <deque>
#include <functional>
#include <set>
#include <sstream>

namespace sharpinference {

namespace {

constexpr GraphElementType F32 = GraphElementType::Float32;
constexpr GraphElementType F16 = GraphElementType::Float16;
constexpr GraphElementType I32 = GraphElementType::Int32;
constexpr GraphElementType BYTE = GraphElementType::Byte;
constexpr GraphResourceAccess R = GraphResourceAccess::Read;
constexpr GraphResourceAccess W = GraphResourceAccess::Write;

using Dims = std::vector<int64_t>;

const char* const kElementTypeNames[] = {"Byte", "Int32", "UInt32", "Float16", "Float32"};

std::string Join(const Dims& d, const char* sep)
{
    std::string s;
    for (size_t i = 0; i < d.size(); i++)
        s += (i ? sep : "") + std::to_string(d[i]);
    return s;
}

int64_t Count(const Dims& d)
{
    int64_t n = 1;
    for (int64_t v : d) {
        if (v < 0 || (v != 0 && n > INT64_MAX / v))
            throw InvalidDataException("Tensor element count exceeds Int64.");
        n *= v;
    }
    return n;
}

// Shortest text that reads back as the same float (the invariant-culture
// round-trip value of TensorFillValue.ToAttributes).
std::string FloatText(float v)
{
    char buf[64];
    const auto r = std::to_chars(buf, buf + sizeof buf, v);
    return std::string(buf, r.ptr);
}

bool IsQuant(int type) { return type == SI_HIP_Q8_0 || type == SI_HIP_Q4_0 || type == SI_HIP_Q4_K; }

std::string FormatName(int type)
{
    switch (type) {
    case SI_HIP_Q8_0: return "q8_0";
    case SI_HIP_Q4_0: return "q4_0";
    case SI_HIP_Q4_K: return "q4_k";
    default: return "";
    }
}

uint64_t QuantRowBytes(int type, int64_t columns)
{
    uint64_t b = 0;
    if (si_hip_tensor_bytes(type, 1, columns, &b) != SI_HIP_OK)
        throw InvalidDataException("A " + FormatName(type) + " row of " + std::to_string(columns) +
                                   " columns is not a whole number of blocks.");
    return b;
}

}  // namespace

// ---- graph model --------------------------------------------------------------------------------

GraphResourceScope GraphResource::Scope() const
{
    switch (lifetime) {
    case GraphResourceLifetime::External:
        return kind == GraphResourceKind::Input || kind == GraphResourceKind::Output ? GraphResourceScope::Local
                                                                                     : GraphResourceScope::Global;
    case GraphResourceLifetime::Model: return GraphResourceScope::Global;
    case GraphResourceLifetime::Session: return GraphResourceScope::Session;
    case GraphResourceLifetime::Token:
    case GraphResourceLifetime::Invocation: return GraphResourceScope::Local;
    }
    throw InvalidDataException("Invalid lifetime for resource '" + id + "'.");
}

const NodeResourceBinding* LogicalNode::Binding(const std::string& port) const
{
    for (const auto& b : resources)
        if (b.port == port)
            return &b;
    return nullptr;
}

const GraphResource* LogicalGraph::FindResource(const std::string& id) const
{
    if (index_.size() > resources.size())
        index_.clear();
    for (size_t i = index_.size(); i < resources.size(); i++)
        index_.emplace(resources[i].id, i);
    const auto it = index_.find(id);
    return it != index_.end() && it->second < resources.size() && resources[it->second].id == id
               ? &resources[it->second]
               : nullptr;
}

const GraphResource& LogicalGraph::Resource(const std::string& id) const
{
    if (const auto* r = FindResource(id))
        return *r;
    throw InvalidDataException("Unknown graph resource '" + id + "'.");
}

// ---- T0 contract validation ----------------------------------------------------------------------

namespace {

struct PortableContract {
    std::vector<std::string> inputs;
    std::vector<std::string> attributes;
};

// PortableTensorOperationContracts.Contracts (:72-84).
const std::map<std::string, PortableContract>& PortableContracts()
{
    static const std::map<std::string, PortableContract> c = {
        {"core.tensor.fill", {{}, {"value"}}},
        {"core.tensor.cast-f16-f32", {{"input"}, {}}},
        {"core.tensor.reshape", {{"input"}, {}}},
        {"core.tensor.slice", {{"input"}, {"axis", "start", "length"}}},
        {"core.tensor.broadcast", {{"input"}, {}}},
        {"core.tensor.batched-mat-vec", {{"matrix", "vector"}, {}}},
        {"core.tensor.reduce-last-sum", {{"input"}, {}}},
        {"core.tensor.reduce-last-mean", {{"input"}, {}}},
        {"core.tensor.head-outer", {{"left", "right"}, {}}},
    };
    return c;
}

// The T0 primitive contracts (TierZeroOperationContracts.cs:147-175): the
// FP32 standard operators with their input ports.
const std::map<std::string, std::vector<std::string>>& PrimitiveContracts()
{
    static const std::map<std::string, std::vector<std::string>> c = {
        {"core.copy", {"input"}},          {"core.add", {"left", "right"}},
        {"core.subtract", {"left", "right"}}, {"core.multiply", {"left", "right"}},
        {"core.divide", {"left", "right"}},   {"core.maximum", {"left", "right"}},
        {"core.exp", {"input"}},           {"core.tanh", {"input"}},
        {"core.sigmoid", {"input"}},       {"core.rsqrt", {"input"}},
        {"core.square", {"input"}},        {"core.relu", {"input"}},
        {"core.reduce-sum", {"input"}},    {"core.reduce-mean", {"input"}},
        {"core.mat-vec", {"matrix", "input"}}, {"core.gather-row", {"table", "index"}},
    };
    return c;
}

bool IsRequiredFp32(const PrecisionRequirement& r)
{
    return Satisfies(F32, r.minimum_arithmetic_type) && Satisfies(F32, r.minimum_accumulator_type);
}

int ParseNonNegative(const LogicalNode& n, const std::string& key, const std::string& kind)
{
    const std::string& t = n.attributes.at(key);
    long long v = 0;
    bool ok = !t.empty() && t.size() <= 10;
    for (char c : t) {
        ok &= c >= '0' && c <= '9';
        v = v * 10 + (c - '0');
    }
    if (!ok || v > INT32_MAX)
        throw InvalidDataException(kind + " '" + n.id + "' requires a non-negative integer '" + key + "'.");
    return static_cast<int>(v);
}

void ValidatePortable(const LogicalNode& n, const LogicalGraph& g)
{
    const auto& contract = PortableContracts().at(n.operation);
    const auto err = [&](const std::string& why) { return InvalidDataException("Tensor operation '" + n.id + "' " + why); };
    if (n.version != 1)
        throw InvalidDataException("Unsupported tensor operation or version '" + n.operation + "@" +
                                   std::to_string(n.version) + "'.");
    if (!IsRequiredFp32(n.requirements))
        throw err("requires FP32 arithmetic and accumulation.");
    std::set<std::string> expected(contract.inputs.begin(), contract.inputs.end());
    expected.insert("output");
    std::set<std::string> ports;
    for (const auto& b : n.resources) {
        ports.insert(b.port);
        if (b.access != (b.port == "output" ? W : R))
            throw err("has invalid ports or access.");
    }
    if (n.resources.size() != expected.size() || ports != expected)
        throw err("has invalid ports or access.");
    const auto get = [&](const std::string& port) -> const GraphResource& {
        const auto* res = g.FindResource(n.Binding(port)->resource);
        if (!res)
            throw err("references unknown resource '" + n.Binding(port)->resource + "'.");
        if (res->tensor.dimensions.empty())
            throw err("requires dense, non-scalar tensors.");
        return *res;
    };
    const std::string out_id = n.Binding("output")->resource;
    for (const auto& b : n.resources)
        if (b.port != "output" && b.resource == out_id)
            throw err("cannot overwrite an input.");
    const GraphResource& out = get("output");
    if (out.kind == GraphResourceKind::Input || out.kind == GraphResourceKind::Weight ||
        out.kind == GraphResourceKind::Constant)
        throw err("cannot write a read-only resource.");
    std::vector<const GraphResource*> in;
    for (const auto& p : contract.inputs)
        in.push_back(&get(p));
    // element types: FP32 everywhere, FP16 in for the cast, an FP16 matrix allowed for batched-mat-vec
    bool types_ok = out.tensor.element_type == F32;
    for (size_t i = 0; i < in.size(); i++) {
        const GraphElementType t = in[i]->tensor.element_type;
        if (n.operation == "core.tensor.cast-f16-f32")
            types_ok &= t == F16;
        else if (n.operation == "core.tensor.batched-mat-vec" && i == 0)
            types_ok &= t == F32 || t == F16;
        else
            types_ok &= t == F32;
    }
    if (!types_ok)
        throw err("has unsupported element types.");
    std::set<std::string> attrs;
    for (const auto& [k, v] : n.attributes)
        attrs.insert(k);
    if (attrs != std::set<std::string>(contract.attributes.begin(), contract.attributes.end()))
        throw err("has invalid attributes.");
    const Dims& d = out.tensor.dimensions;
    const auto shape_error = [&]() { return err("has incompatible dimensions."); };
    if (n.operation == "core.tensor.fill") {
        const std::string& t = n.attributes.at("value");
        char* end = nullptr;
        const float v = std::strtof(t.c_str(), &end);
        if (t.empty() || std::isspace(static_cast<unsigned char>(t.front())) ||
            std::isspace(static_cast<unsigned char>(t.back())) || end != t.c_str() + t.size() || !std::isfinite(v))
            throw InvalidDataException("Tensor fill '" + n.id +
                                       "' requires a finite invariant-culture FP32 value.");
    } else if (n.operation == "core.tensor.slice") {
        const int axis = ParseNonNegative(n, "axis", "Tensor operation");
        const int start = ParseNonNegative(n, "start", "Tensor operation");
        const int length = ParseNonNegative(n, "length", "Tensor operation");
        const Dims& s = in[0]->tensor.dimensions;
        bool ok = axis < static_cast<int>(s.size()) && length > 0 && start <= s[axis] &&
                  static_cast<int64_t>(start) + length <= s[axis] && d.size() == s.size();
        for (size_t a = 0; ok && a < d.size(); a++)
            ok = d[a] == (static_cast<int>(a) == axis ? length : s[a]);
        if (!ok)
            throw InvalidDataException("Tensor slice '" + n.id + "' has incompatible dimensions.");
    } else if (n.operation == "core.tensor.cast-f16-f32") {
        if (d != in[0]->tensor.dimensions)
            throw shape_error();
    } else if (n.operation == "core.tensor.reshape") {
        if (Count(d) != Count(in[0]->tensor.dimensions))
            throw shape_error();
    } else if (n.operation == "core.tensor.broadcast") {
        const Dims& s = in[0]->tensor.dimensions;
        if (s.size() > d.size())
            throw shape_error();
        for (size_t a = 0; a < s.size(); a++)
            if (s[a] != 1 && s[a] != d[d.size() - s.size() + a])
                throw shape_error();
    } else if (n.operation == "core.tensor.batched-mat-vec") {
        const Dims& m = in[0]->tensor.dimensions;
        const Dims& v = in[1]->tensor.dimensions;
        if (m.size() != 3 || v.size() != 2 || d.size() != 2 || m[0] != v[0] || m[2] != v[1] || d[0] != m[0] ||
            d[1] != m[1])
            throw shape_error();
    } else if (n.operation == "core.tensor.reduce-last-sum" || n.operation == "core.tensor.reduce-last-mean") {
        const Dims& s = in[0]->tensor.dimensions;
        if ((s.size() != 2 && s.size() != 3) || d.size() != s.size() - 1 || !std::equal(d.begin(), d.end(), s.begin()))
            throw shape_error();
    } else if (n.operation == "core.tensor.head-outer") {
        const Dims& l = in[0]->tensor.dimensions;
        const Dims& r = in[1]->tensor.dimensions;
        if (l.size() != 2 || r.size() != 2 || d.size() != 3 || l[0] != r[0] || d[0] != l[0] || d[1] != l[1] ||
            d[2] != r[1])
            throw shape_error();
    }
}

void ValidatePrimitive(const LogicalNode& n, const LogicalGraph& g)
{
    const auto it = PrimitiveContracts().find(n.operation);
    if (it == PrimitiveContracts().end() || n.version != 1)
        throw NotSupportedException("Unsupported T0 operation or version '" + n.operation + "@" +
                                    std::to_string(n.version) + "'.");
    const auto err = [&](const std::string& why) {
        return InvalidDataException("T0 operation '" + n.id + "' (" + n.operation + "): " + why);
    };
    if (!IsRequiredFp32(n.requirements))
        throw err("requires FP32 arithmetic and accumulation.");
    std::vector<std::string> ports = it->second;
    // existing logical graphs use "weight"; "matrix" is the canonical T0 port (:24-29)
    if (n.operation == "core.mat-vec" && n.Binding("weight"))
        ports = {"weight", "input"};
    std::set<std::string> expected(ports.begin(), ports.end()), got;
    expected.insert("output");
    bool ok = n.attributes.empty() && n.resources.size() == ports.size() + 1;
    for (const auto& b : n.resources) {
        got.insert(b.port);
        ok &= b.access == (b.port == "output" ? W : R);
    }
    if (!ok || got != expected)
        throw err("invalid ports, attributes or access.");
    const auto get = [&](const std::string& port) -> const GraphResource& {
        const auto* res = g.FindResource(n.Binding(port)->resource);
        if (!res)
            throw err("unknown resource '" + n.Binding(port)->resource + "'.");
        if (res->tensor.dimensions.empty())
            throw err("requires dense, non-scalar tensors.");
        return *res;
    };
    const GraphResource& out = get("output");
    std::vector<const GraphResource*> in;
    for (const auto& p : ports)
        in.push_back(&get(p));
    if (out.kind == GraphResourceKind::Input || out.kind == GraphResourceKind::Weight ||
        out.kind == GraphResourceKind::Constant)
        throw err("cannot write a read-only resource.");
    for (const auto* r : in)
        if (r->id == out.id)
            throw err("cannot overwrite an input.");
    bool types = out.tensor.element_type == F32;
    for (size_t i = 0; i < in.size(); i++) {
        const GraphElementType t = in[i]->tensor.element_type;
        if ((n.operation == "core.mat-vec" || n.operation == "core.gather-row") && i == 0)
            types &= t == F32 || t == F16;
        else if (n.operation == "core.gather-row" && i == 1)
            types &= t == I32;
        else
            types &= t == F32;
    }
    if (!types)
        throw NotSupportedException("T0 operation '" + n.operation + "' has unsupported element types.");
    const Dims& s = in[0]->tensor.dimensions;
    const Dims& d = out.tensor.dimensions;
    bool shape;
    if (n.operation == "core.mat-vec")
        shape = s.size() == 2 && in[1]->tensor.dimensions == Dims{s[1]} && d == Dims{s[0]};
    else if (n.operation == "core.gather-row")
        shape = s.size() == 2 && in[1]->tensor.dimensions == Dims{1} && d == Dims{s[1]};
    else if (n.operation == "core.reduce-sum" || n.operation == "core.reduce-mean")
        shape = d == Dims{1};
    else {
        shape = true;
        for (const auto* r : in)
            shape &= r->tensor.dimensions == d;
    }
    if (!shape)
        throw err("incompatible dimensions.");
}

// quant.mat-vec / quant.gather-row: adapted by the HIP quantized collection
// itself (ports, attributes and the Byte [rows, row_bytes] operand).
void ValidateQuant(const LogicalNode& n, const LogicalGraph& g, const InstructionRegistry& registry)
{
    const auto instruction = registry.Resolve(HipInstructionCollectionIds::QuantizedFloat32, n.operation,
                                              InstructionTarget::Hip());
    std::vector<InstructionParameter> params;
    for (const auto& b : n.resources)
        params.push_back(InstructionParameter::Tensor(b.port, g.Resource(b.resource).tensor, b.access, b.resource));
    for (const auto& [k, v] : n.attributes)
        params.push_back(InstructionParameter::Attribute(k, v));
    try {
        instruction->Adapt(params, n.requirements);
    } catch (const InstructionAdaptationException& e) {
        throw InvalidDataException("Quantized operation '" + n.id + "': " + e.what());
    }
    const auto& out = g.Resource(n.Binding("output")->resource);
    if (out.kind == GraphResourceKind::Input || out.kind == GraphResourceKind::Weight ||
        out.kind == GraphResourceKind::Constant)
        throw InvalidDataException("Quantized operation '" + n.id + "' cannot write a read-only resource.");
}

}  // namespace

void ValidateGraph(const LogicalGraph& g)
{
    std::set<std::string> ids, nodes;
    for (const auto& r : g.resources)
        if (r.id.empty() || !ids.insert(r.id).second)
            throw InvalidDataException("Duplicate or blank resource id '" + r.id + "'.");
    for (const auto& id : g.inputs)
        g.Resource(id);
    for (const auto& id : g.outputs)
        g.Resource(id);
    for (const auto& s : g.state)
        g.Resource(s.resource);
    const auto registry = DefaultHipRegistry();
    for (const auto& n : g.nodes) {
        if (n.id.empty() || !nodes.insert(n.id).second)
            throw InvalidDataException("Duplicate or blank node id '" + n.id + "'.");
        for (const auto& dep : n.dependencies)
            if (!nodes.count(dep))
                throw InvalidDataException("Node '" + n.id + "' depends on '" + dep + "', which does not precede it.");
        for (const auto& b : n.resources)
            if (!ids.count(b.resource))
                throw InvalidDataException("Node '" + n.id + "' binds unknown resource '" + b.resource + "'.");
        if (n.operation.rfind("core.tensor.", 0) == 0) {
            if (!PortableContracts().count(n.operation))
                throw InvalidDataException("Unsupported tensor operation or version '" + n.operation + "'.");
            ValidatePortable(n, g);
        } else if (n.operation.rfind("quant.", 0) == 0) {
            ValidateQuant(n, g, *registry);
        } else {
            ValidatePrimitive(n, g);
        }
    }
}

// ---- RWKV-7 graph builder ------------------------------------------------------------------------

namespace {

class Rwkv7Builder {
public:
    explicit Rwkv7Builder(const ModelTensorCatalog& t) : t_(t) {}

    LogicalGraph Build()
    {
        const auto rk = t_.tensors.find("blocks.0.att.r_k");
        if (rk == t_.tensors.end() || !t_.tensors.count("blocks.0.att.x_rwkvag"))
            throw InvalidDataException("The tensor catalog does not satisfy the RWKV-7 x070 contract.");
        width_ = t_.embedding;
        const Dims& rkd = rk->second.dims;
        if (rkd.size() != 2 || width_ <= 0 || rkd[1] <= 0 || width_ % rkd[1] != 0)
            throw InvalidDataException("RWKV-7 head dimensions do not match the embedding size.");
        heads_ = rkd[1];
        head_ = width_ / heads_;
        if (rkd[0] != head_)
            throw InvalidDataException("RWKV-7 receptance-key dimensions do not match the head shape.");

        g_.name = "rwkv7.forward-token.portable";
        g_.architecture = "rwkv-7";
        g_.state_abi = "rwkv-7.state.fp32@1";
        g_.state_schema = "RWKV7_State";
        AddResource("token", "Token", GraphResourceKind::Input, GraphResourceLifetime::External, {I32, {1}});
        AddResource("logits", "Logits", GraphResourceKind::Output, GraphResourceLifetime::External,
                    {F32, {t_.vocabulary}});
        g_.inputs.push_back("token");
        g_.outputs.push_back("logits");
        for (const auto& [name, tensor] : t_.tensors) {   // ordinal name order
            const std::string id = "weight." + name;
            TensorDescriptor d;
            if (IsQuant(tensor.type)) {
                if (tensor.dims.size() != 2 || tensor.dims[0] < 1 || tensor.dims[1] < 1)
                    throw InvalidDataException("Tensor '" + name + "' must be a [input, output] matrix.");
                d = {BYTE, {tensor.dims[1], static_cast<int64_t>(QuantRowBytes(tensor.type, tensor.dims[0]))}};
            } else if (tensor.type == SI_HIP_F16 || tensor.type == SI_HIP_F32) {
                d = {tensor.type == SI_HIP_F16 ? F16 : F32, tensor.dims};
            } else {
                throw InvalidDataException("Tensor '" + name + "' must have FP16, FP32 or Q8_0 / Q4_0 / Q4_K values.");
            }
            AddResource(id, name, GraphResourceKind::Weight, GraphResourceLifetime::Model, d, name);
            types_[id] = tensor.type;
            catalog_dims_[id] = tensor.dims;
        }
        for (int64_t layer = 0; layer < t_.layers; layer++)
            for (const auto& [suffix, dims] : std::vector<std::pair<std::string, Dims>>{
                     {"ffn-previous", {width_}}, {"att-previous", {width_}}, {"wkv", {heads_, head_, head_}}}) {
                const std::string id = "state." + std::to_string(layer) + "." + suffix;
                AddResource(id, id, GraphResourceKind::SessionState, GraphResourceLifetime::Session, {F32, dims});
                g_.state.push_back({id, id});
            }
        Body();
        ValidateGraph(g_);
        return std::move(g_);
    }

private:
    // -- resources and nodes --
    void AddResource(const std::string& id, const std::string& name, GraphResourceKind kind,
                     GraphResourceLifetime lifetime, TensorDescriptor tensor, const std::string& key = "")
    {
        GraphResource r;
        r.id = id;
        r.name = name;
        r.kind = kind;
        r.lifetime = lifetime;
        r.tensor = std::move(tensor);
        r.binding_key = key;
        shapes_[id] = r.tensor.dimensions;
        g_.resources.push_back(std::move(r));
    }

    std::string Node(const std::string& op, const std::vector<std::pair<std::string, std::string>>& inputs,
                     const Dims& shape, std::string result = "", std::map<std::string, std::string> attributes = {})
    {
        char id[32];
        std::snprintf(id, sizeof id, "portable.%05d", serial_++);
        if (result.empty())
            result = id;
        const auto it = shapes_.find(result);
        if (it != shapes_.end()) {
            if (it->second != shape)
                throw InvalidDataException("Resource '" + result + "' has incompatible dimensions.");
        } else {
            AddResource(result, result, GraphResourceKind::Temporary, GraphResourceLifetime::Invocation, {F32, shape});
        }
        LogicalNode n;
        n.id = id;
        n.operation = op;
        for (const auto& [port, res] : inputs)
            n.resources.push_back({port, res, R});
        n.resources.push_back({"output", result, W});
        if (!previous_.empty())
            n.dependencies.push_back(previous_);
        n.attributes = std::move(attributes);
        g_.nodes.push_back(std::move(n));
        previous_ = id;
        return result;
    }

    const Dims& Shape(const std::string& r) const { return shapes_.at(r); }

    std::string Reshape(const std::string& input, const Dims& dims)
    {
        if (Count(Shape(input)) != Count(dims))
            throw InvalidDataException("Cannot reshape '" + input + "'.");
        return Shape(input) == dims ? input : Node("core.tensor.reshape", {{"input", input}}, dims);
    }
    std::string Broadcast(const std::string& input, const Dims& dims)
    {
        return Node("core.tensor.broadcast", {{"input", input}}, dims);
    }
    std::string Fill(float value, const Dims& dims)
    {
        return Node("core.tensor.fill", {}, dims, "", {{"value", FloatText(value)}});
    }
    std::string Weight(const std::string& name)
    {
        const std::string id = "weight." + name;
        const auto it = types_.find(id);
        if (it == types_.end())
            throw InvalidDataException("The tensor catalog has no tensor '" + name + "'.");
        if (it->second == SI_HIP_F16)
            return Node("core.tensor.cast-f16-f32", {{"input", id}}, Shape(id));
        return id;   // FP32, or quantized blocks read by the quantized operators
    }
    std::string VectorWeight(const std::string& name, int64_t length)
    {
        if (IsQuant(types_.at("weight." + name)))
            throw InvalidDataException("Tensor '" + name + "' must have FP16 or FP32 values.");
        const std::string t = Weight(name);
        if (Count(Shape(t)) != length)
            throw InvalidDataException("Tensor '" + name + "' does not have " + std::to_string(length) + " elements.");
        return Reshape(t, {length});
    }
    std::string Unary(const std::string& op, const std::string& input) { return Node(op, {{"input", input}}, Shape(input)); }
    std::string Binary(const std::string& op, const std::string& l, const std::string& r)
    {
        if (Shape(l) != Shape(r))
            throw InvalidDataException("Incompatible elementwise dimensions: '" + l + "', '" + r + "'.");
        return Node(op, {{"left", l}, {"right", r}}, Shape(l));
    }
    std::string Add(const std::string& l, const std::string& r) { return Binary("core.add", l, r); }
    std::string Sub(const std::string& l, const std::string& r) { return Binary("core.subtract", l, r); }
    std::string Mul(const std::string& l, const std::string& r) { return Binary("core.multiply", l, r); }
    std::string Mean(const std::string& input) { return Node("core.reduce-mean", {{"input", input}}, {1}); }
    std::string ReduceHead(const std::string& input, bool mean)
    {
        Dims d = Shape(input);
        d.pop_back();
        return Node(mean ? "core.tensor.reduce-last-mean" : "core.tensor.reduce-last-sum", {{"input", input}}, d);
    }
    std::string ExpandHead(const std::string& input) { return Broadcast(Reshape(input, {heads_, 1}), {heads_, head_}); }

    // A projection's matrix: GGML [input, output] read as row-major
    // [output, input]; a quantized matrix is its Byte [output, row_bytes]
    // weight itself.
    std::string Matrix(const std::string& name, int64_t input_length, int* type)
    {
        const std::string id = "weight." + name;
        if (!types_.count(id))
            throw InvalidDataException("The tensor catalog has no tensor '" + name + "'.");
        const Dims& cd = catalog_dims_.at(id);
        *type = types_.at(id);
        if (cd.size() != 2 || cd[0] != input_length)
            throw InvalidDataException("Tensor '" + name + "' has invalid projection dimensions.");
        if (IsQuant(*type))
            return id;
        return Reshape(Weight(name), {cd[1], cd[0]});
    }
    std::string Project(const std::string& name, const std::string& input)
    {
        const Dims& d = Shape(input);
        if (d.size() != 1)
            throw InvalidDataException("Projection input '" + input + "' must be a vector.");
        int type = 0;
        const std::string m = Matrix(name, d[0], &type);
        if (IsQuant(type))
            return Node("quant.mat-vec", {{"matrix", m}, {"input", input}}, {Shape(m)[0]}, "",
                        {{"format", FormatName(type)}, {"columns", std::to_string(d[0])}});
        return Node("core.mat-vec", {{"matrix", m}, {"input", input}}, {Shape(m)[0]});
    }
    std::string Normalize(const std::string& input, float eps)
    {
        const Dims d = Shape(input);
        const std::string centered = Sub(input, Broadcast(Mean(input), d));
        const std::string variance = Mean(Unary("core.square", centered));
        const std::string inv = Unary("core.rsqrt", Add(variance, Fill(eps, {1})));
        return Mul(centered, Broadcast(inv, d));
    }
    std::string GroupNormalize(const std::string& input)
    {
        const std::string grouped = Reshape(input, {heads_, head_});
        const std::string centered = Sub(grouped, ExpandHead(ReduceHead(grouped, true)));
        const std::string variance = ReduceHead(Unary("core.square", centered), true);
        const std::string inv = Unary("core.rsqrt", Add(variance, Fill(64e-5f, {heads_})));
        return Reshape(Mul(centered, ExpandHead(inv)), {width_});
    }
    std::string Affine(const std::string& input, const std::string& weight, const std::string& bias)
    {
        const int64_t n = Shape(input)[0];
        return Add(Mul(input, VectorWeight(weight, n)), VectorWeight(bias, n));
    }
    std::string Mix(const std::string& input, const std::string& prev, const std::string& mix)
    {
        return Add(input, Mul(Sub(prev, input), mix));
    }
    std::string SliceMix(const std::string& mixes, int row)
    {
        return Reshape(Node("core.tensor.slice", {{"input", mixes}}, {1, width_}, "",
                            {{"axis", "0"}, {"start", std::to_string(row)}, {"length", "1"}}),
                       {width_});
    }
    std::string Outer(const std::string& l, const std::string& r)
    {
        return Node("core.tensor.head-outer", {{"left", l}, {"right", r}}, {heads_, head_, head_});
    }
    std::string BatchedMatVec(const std::string& m, const std::string& v)
    {
        return Node("core.tensor.batched-mat-vec", {{"matrix", m}, {"vector", v}}, {heads_, head_});
    }
    void Store(const std::string& source, const std::string& state)
    {
        Node("core.copy", {{"input", source}}, Shape(state), state);
    }

    // PortableRwkv7GraphProvider.Build's node sequence (:186-292).
    void Body()
    {
        int type = 0;
        const std::string embedding = Matrix("emb.weight", width_, &type);
        if ((IsQuant(type) ? Shape(embedding)[0] : Shape(embedding)[0]) != t_.vocabulary)
            throw InvalidDataException("The embedding does not match the vocabulary size.");
        std::string x = IsQuant(type)
                            ? Node("quant.gather-row", {{"table", embedding}, {"index", "token"}}, {width_}, "",
                                   {{"format", FormatName(type)}, {"columns", std::to_string(width_)}})
                            : Node("core.gather-row", {{"table", embedding}, {"index", "token"}}, {width_});
        x = Affine(Normalize(x, 1e-5f), "blocks.0.ln0.weight", "blocks.0.ln0.bias");
        std::string first_value;
        for (int64_t layer = 0; layer < t_.layers; layer++) {
            const std::string prefix = "blocks." + std::to_string(layer) + ".";
            const auto att = [&](const std::string& s) { return prefix + "att." + s; };
            const std::string att_prev = "state." + std::to_string(layer) + ".att-previous";
            const std::string ffn_prev = "state." + std::to_string(layer) + ".ffn-previous";
            const std::string wkv = "state." + std::to_string(layer) + ".wkv";
            const std::string normalized = Affine(Normalize(x, 1e-5f), prefix + "ln1.weight", prefix + "ln1.bias");
            const std::string mixes = Reshape(Weight(att("x_rwkvag")), {6, width_});
            const std::string xr = Mix(normalized, att_prev, SliceMix(mixes, 0));
            const std::string xw = Mix(normalized, att_prev, SliceMix(mixes, 1));
            const std::string xk = Mix(normalized, att_prev, SliceMix(mixes, 2));
            const std::string xv = Mix(normalized, att_prev, SliceMix(mixes, 3));
            const std::string xa = Mix(normalized, att_prev, SliceMix(mixes, 4));
            const std::string xg = Mix(normalized, att_prev, SliceMix(mixes, 5));
            const std::string r = Project(att("receptance.weight"), xr);
            std::string key = Project(att("key.weight"), xk);
            std::string value = Project(att("value.weight"), xv);
            const std::string decay_offset =
                Add(Project(att("w2"), Unary("core.tanh", Project(att("w1"), xw))), VectorWeight(att("w0"), width_));
            const std::string decay =
                Unary("core.exp", Mul(Fill(-0.606531f, {width_}), Unary("core.sigmoid", decay_offset)));
            const std::string adaptation = Unary(
                "core.sigmoid", Add(Project(att("a2"), Project(att("a1"), xa)), VectorWeight(att("a0"), width_)));
            const std::string gate = Project(att("g2"), Unary("core.sigmoid", Project(att("g1"), xg)));

            const std::string scaled_key = Mul(key, VectorWeight(att("k_k"), width_));
            const std::string key_heads = Reshape(scaled_key, {heads_, head_});
            const std::string squares = ReduceHead(Unary("core.square", key_heads), false);
            const std::string inverse_magnitude =
                Unary("core.rsqrt", Binary("core.maximum", squares, Fill(1e-24f, {heads_})));
            const std::string normalized_key = Mul(key_heads, ExpandHead(inverse_magnitude));
            const std::string ka = Mul(key, VectorWeight(att("k_a"), width_));
            key = Sub(Add(key, Mul(adaptation, ka)), ka);
            if (first_value.empty()) {
                first_value = value;
            } else {
                const std::string value_gate = Unary(
                    "core.sigmoid", Add(Project(att("v2"), Project(att("v1"), xv)), VectorWeight(att("v0"), width_)));
                value = Add(value, Mul(Sub(first_value, value), value_gate));
            }

            const std::string keyed = Reshape(key, {heads_, head_});
            const std::string valued = Reshape(value, {heads_, head_});
            const std::string received = Reshape(r, {heads_, head_});
            const std::string adapted_key = Mul(normalized_key, Reshape(adaptation, {heads_, head_}));
            const std::string negative_projection =
                Sub(Fill(0.0f, {heads_, head_}), BatchedMatVec(wkv, normalized_key));
            const std::string decay_matrix = Broadcast(Reshape(decay, {heads_, 1, head_}), {heads_, head_, head_});
            // S'[h,i,j] = S[h,i,j] w[h,j] + v[h,i] k[h,j] - (sum_l S[h,i,l] kn[h,l]) kn[h,j] a[h,j]
            const std::string updated =
                Add(Add(Mul(wkv, decay_matrix), Outer(valued, keyed)), Outer(negative_projection, adapted_key));
            std::string attention = Reshape(BatchedMatVec(updated, received), {width_});
            Store(updated, wkv);
            attention = Affine(GroupNormalize(attention), att("ln_x.weight"), att("ln_x.bias"));
            const std::string bonus_factors = Mul(Mul(key, r), VectorWeight(att("r_k"), width_));
            const std::string bonus = ExpandHead(ReduceHead(Reshape(bonus_factors, {heads_, head_}), false));
            attention = Mul(Add(attention, Mul(value, Reshape(bonus, {width_}))), gate);
            x = Add(x, Project(att("output.weight"), attention));
            Store(normalized, att_prev);

            const std::string ffn_normalized = Affine(Normalize(x, 1e-5f), prefix + "ln2.weight", prefix + "ln2.bias");
            const std::string key_input = Mix(ffn_normalized, ffn_prev, VectorWeight(prefix + "ffn.x_k", width_));
            const std::string hidden = Unary("core.relu", Project(prefix + "ffn.key.weight", key_input));
            x = Add(x, Project(prefix + "ffn.value.weight", Unary("core.square", hidden)));
            Store(ffn_normalized, ffn_prev);
        }
        const std::string output = Affine(Normalize(x, 1e-5f), "ln_out.weight", "ln_out.bias");
        const std::string logits = Project("head.weight", output);
        Node("core.copy", {{"input", logits}}, {t_.vocabulary}, "logits");
    }

    const ModelTensorCatalog& t_;
    LogicalGraph g_;
    std::map<std::string, Dims> shapes_;
    std::map<std::string, int> types_;
    std::map<std::string, Dims> catalog_dims_;
    int serial_ = 0;
    std::string previous_;
    int64_t width_ = 0, heads_ = 0, head_ = 0;
};

}  // namespace

LogicalGraph BuildRwkv7Graph(const ModelTensorCatalog& tensors) { return Rwkv7Builder(tensors).Build(); }

// ---- GPU mat-vec selection -------------------------------------------------------------------------

GpuMatVecOptimizationSettings::GpuMatVecOptimizationSettings(GpuMatVecMode mode,
                                                             std::optional<MatVecCostProfile> profile,
                                                             std::optional<std::string> fingerprint)
    : mode_(mode), profile_(std::move(profile)), fingerprint_(std::move(fingerprint))
{
    if (static_cast<int>(mode) < 0 || static_cast<int>(mode) > 3)
        throw ArgumentOutOfRangeException("mode");
    const bool blank = !fingerprint_ || fingerprint_->find_first_not_of(" \t\r\n") == std::string::npos;
    if (mode == GpuMatVecMode::Profile && (!profile_ || blank))
        throw ArgumentException("Profile selection requires explicit costs and a current environment fingerprint.");
    if (mode != GpuMatVecMode::Profile && (profile_ || fingerprint_))
        throw ArgumentException("Costs are only accepted in profile mode.");
}

std::string GpuMatVecOptimizationSettings::Shape(const std::vector<InstructionParameter>& parameters)
{
    const InstructionParameter *m = nullptr, *x = nullptr, *y = nullptr;
    for (const auto& p : parameters) {
        if (p.kind != InstructionParameter::Kind::Tensor)
            continue;
        if (p.name == "matrix" || p.name == "weight")
            m = &p;
        else if (p.name == "input")
            x = &p;
        else if (p.name == "output")
            y = &p;
    }
    if (!m || !x || !y)
        throw InvalidOperationException("A mat-vec needs matrix (or weight), input and output parameters.");
    const auto type = [](const InstructionParameter* p) {
        return std::string(kElementTypeNames[static_cast<int>(p->tensor.element_type)]);
    };
    return Join(m->tensor.dimensions, "x") + "|" + type(m) + "," + type(x) + "," + type(y);
}

std::pair<bool, std::string> GpuMatVecOptimizationSettings::Select(const std::vector<InstructionParameter>& parameters,
                                                                   const HipVmOptimizationOptions& options,
                                                                   int64_t now) const
{
    switch (mode_) {
    case GpuMatVecMode::Serial: return {false, "Explicit serial MatVec."};
    case GpuMatVecMode::Default: return {true, "Default GPU MatVec implementation: cooperative."};
    case GpuMatVecMode::Cooperative: return {true, "Explicit cooperative MatVec; not a measured selection."};
    case GpuMatVecMode::Profile: break;
    }
    const MatVecCostProfile& profile = *profile_;
    if (profile.environment_fingerprint != *fingerprint_)
        return {false, "MatVec profile environment fingerprint mismatch."};
    if (profile.measured_at_unix_seconds > now + 5 * 60 || now - profile.measured_at_unix_seconds > 30 * 24 * 3600)
        return {false, "MatVec profile timestamp is stale or in the future."};
    const std::string shape = Shape(parameters);
    const MatVecCostMeasurement* found = nullptr;
    int matches = 0;
    for (const auto& m : profile.measurements)
        if (m.operation == "core.mat-vec" && m.implementation_fingerprint == HipMatVecExecution::ImplementationFingerprint &&
            m.shape == shape && m.input_aliases == "0,1" && m.threads_per_group == options.threads_per_group &&
            m.threads_per_group == HipMatVecExecution::Threads && m.reuse_local_storage == options.reuse_local_storage) {
            found = &m;
            matches++;
        }
    if (matches > 1)
        throw InvalidOperationException("Sequence contains more than one matching element");
    if (!found)
        return {false, "No trusted MatVec costs for this shape/storage/launch domain."};
    return found->conservative_saving_microseconds > 0
               ? std::make_pair(true, std::string("Cooperative MatVec selected from positive conservative offline savings."))
               : std::make_pair(false, std::string("MatVec costs do not establish a conservative benefit; serial retained."));
}

// ---- lowering ----------------------------------------------------------------------------------------

namespace {

struct Lowered {
    std::vector<LogicalNode> nodes;
    std::map<std::string, GraphResource> descriptors;
    std::map<std::string, std::string> aliases;   // view -> source resource
    int removed = 0;
};

// VmGraphOptimizer.LowerWeightViews (:198-299): an FP16 weight cast whose
// output (through reshapes) only feeds the matrix of a mat-vec, the table of
// a gather-row or the matrix of a batched-mat-vec becomes an FP16 view of the
// weight; a reshape of an immutable tensor (a weight, a view of one, or the
// output of a cast of one) whose output is only read becomes a view of it.
void LowerWeightViews(const LogicalGraph& g, bool native_half, Lowered& L)
{
    std::map<std::string, std::vector<std::pair<size_t, const NodeResourceBinding*>>> consumers;
    for (size_t i = 0; i < L.nodes.size(); i++)
        for (const auto& b : L.nodes[i].resources)
            consumers[b.resource].push_back({i, &b});
    std::set<std::string> visible(g.inputs.begin(), g.inputs.end());
    visible.insert(g.outputs.begin(), g.outputs.end());
    for (const auto& s : g.state)
        visible.insert(s.resource);
    const auto out_of = [&](size_t i) { return L.nodes[i].Binding("output")->resource; };
    const auto read_only_uses = [&](const std::string& id, size_t producer) {
        for (const auto& [node, b] : consumers[id])
            if (node != producer && b->access != R)
                return false;
        return true;
    };
    std::set<size_t> removed;
    if (native_half)
        for (size_t i = 0; i < L.nodes.size(); i++) {
            const LogicalNode& n = L.nodes[i];
            if (n.operation != "core.tensor.cast-f16-f32")
                continue;
            const std::string input = n.Binding("input")->resource, output = out_of(i);
            const GraphResource& in = L.descriptors.at(input);
            if (in.kind != GraphResourceKind::Weight || in.tensor.element_type != F16 || visible.count(output))
                continue;
            std::map<size_t, bool> path{{i, true}};
            std::deque<std::string> pending{output};
            std::set<std::string> seen;
            bool safe = true;
            while (!pending.empty() && safe) {
                const std::string v = pending.front();
                pending.pop_front();
                if (!seen.insert(v).second)
                    continue;
                if (visible.count(v)) {
                    safe = false;
                    break;
                }
                for (const auto& [node, b] : consumers[v]) {
                    if (path.count(node))
                        continue;
                    const std::string& op = L.nodes[node].operation;
                    if (b->access != R) {
                        safe = false;
                        break;
                    }
                    if (op == "core.tensor.reshape" && b->port == "input") {
                        path[node] = true;
                        pending.push_back(out_of(node));
                    } else if (!((op == "core.mat-vec" && (b->port == "matrix" || b->port == "weight")) ||
                                 (op == "core.gather-row" && b->port == "table") ||
                                 (op == "core.tensor.batched-mat-vec" && b->port == "matrix"))) {
                        safe = false;
                        break;
                    }
                }
            }
            if (!safe)
                continue;
            for (const auto& [node, unused] : path) {
                (void)unused;
                const std::string id = out_of(node);
                L.aliases[id] = input;
                L.descriptors[id].tensor.element_type = F16;
                removed.insert(node);
            }
        }
    std::set<std::string> immutable;
    for (const auto& [id, r] : L.descriptors)
        if (r.kind == GraphResourceKind::Weight)
            immutable.insert(id);
    for (const auto& [alias, source] : L.aliases)
        immutable.insert(alias);
    for (size_t i = 0; i < L.nodes.size(); i++)
        if (L.nodes[i].operation == "core.tensor.cast-f16-f32" && !removed.count(i) &&
            immutable.count(L.nodes[i].Binding("input")->resource) && read_only_uses(out_of(i), i))
            immutable.insert(out_of(i));
    std::deque<std::string> views(immutable.begin(), immutable.end());
    while (!views.empty()) {
        const std::string input = views.front();
        views.pop_front();
        for (const auto& [node, b] : consumers[input]) {
            if (L.nodes[node].operation != "core.tensor.reshape" || b->port != "input" || removed.count(node))
                continue;
            const std::string output = out_of(node);
            if (visible.count(output) || !read_only_uses(output, node))
                continue;
            const auto a = L.aliases.find(input);
            L.aliases[output] = a != L.aliases.end() ? a->second : input;
            L.descriptors[output].tensor.element_type = L.descriptors.at(input).tensor.element_type;
            removed.insert(node);
            views.push_back(output);
        }
    }
    if (removed.empty())
        return;
    std::vector<LogicalNode> kept;
    std::string last_kept;
    std::map<std::string, std::string> replaced;   // removed node -> the kept node it depended on
    for (size_t i = 0; i < L.nodes.size(); i++) {
        LogicalNode n = L.nodes[i];
        std::vector<std::string> deps;
        for (const auto& d : n.dependencies) {
            const auto it = replaced.find(d);
            const std::string dep = it != replaced.end() ? it->second : d;
            if (!dep.empty() && std::find(deps.begin(), deps.end(), dep) == deps.end())
                deps.push_back(dep);
        }
        if (removed.count(i)) {
            replaced[n.id] = deps.empty() ? "" : deps.front();
            continue;
        }
        n.dependencies = deps;
        kept.push_back(std::move(n));
    }
    L.removed = static_cast<int>(removed.size());
    L.nodes = std::move(kept);
}

// GraphResourceAllocator.PlanLocal (GraphResourceAllocator.cs:38-200) over a
// chain of nodes (each depends on the one before it): every local
// intermediate, in resource order, takes the first slot whose occupants
// have its lifetime, element type and dimensions and whose uses all come
// before its own (or after them).
std::map<std::string, int> PlanLocal(const LogicalGraph& g, const Lowered& L, std::vector<TensorDescriptor>& slots)
{
    const auto source = [&](const std::string& id) {
        const auto a = L.aliases.find(id);
        return a != L.aliases.end() ? a->second : id;
    };
    std::map<std::string, std::pair<size_t, size_t>> span;   // first and last use
    std::map<std::string, GraphResourceAccess> first_access;
    for (size_t i = 0; i < L.nodes.size(); i++)
        for (const auto& b : L.nodes[i].resources) {
            const std::string id = source(b.resource);
            const auto it = span.find(id);
            if (it == span.end()) {
                span[id] = {i, i};
                first_access[id] = b.access;
            } else {
                it->second.second = i;
            }
        }
    std::set<std::string> endpoints(g.inputs.begin(), g.inputs.end());
    endpoints.insert(g.outputs.begin(), g.outputs.end());
    std::map<std::string, int> assignment;
    std::vector<std::vector<std::string>> occupants;
    for (const auto& r : g.resources) {
        if (L.aliases.count(r.id) || r.Scope() != GraphResourceScope::Local || endpoints.count(r.id) ||
            !span.count(r.id))
            continue;
        if (first_access.at(r.id) == R)
            throw InvalidDataException("Local resource '" + r.id + "' must be written before its first read.");
        const GraphResource& d = L.descriptors.at(r.id);
        const auto [first, last] = span.at(r.id);
        int slot = -1;
        for (size_t s = 0; s < occupants.size() && slot < 0; s++) {
            bool fits = true;
            for (const auto& other : occupants[s]) {
                const GraphResource& o = L.descriptors.at(other);
                const auto [of, ol] = span.at(other);
                fits &= o.lifetime == d.lifetime && o.tensor.element_type == d.tensor.element_type &&
                        o.tensor.dimensions == d.tensor.dimensions && (ol < first || last < of);
            }
            if (fits)
                slot = static_cast<int>(s);
        }
        if (slot < 0) {
            slot = static_cast<int>(occupants.size());
            occupants.emplace_back();
            slots.push_back(d.tensor);
        }
        occupants[slot].push_back(r.id);
        assignment[r.id] = slot;
    }
    return assignment;
}

std::string CollectionOf(const std::string& operation)
{
    return operation.rfind("quant.", 0) == 0 ? HipInstructionCollectionIds::QuantizedFloat32
                                             : InstructionCollectionIds::TierZeroFloat32;
}

}  // namespace

HipVmOptimizationResult OptimizeWithReport(const LogicalGraph& graph, const HipVmOptimizationOptions& options,
                                           const std::shared_ptr<const InstructionRegistry>& registry_in)
{
    if (options.threads_per_group == 0 || options.threads_per_group > 1024)
        throw ArgumentOutOfRangeException("Thread group size must be between 1 and 1024.");
    const auto registry = registry_in ? registry_in : DefaultHipRegistry();
    ValidateGraph(graph);
    Lowered L;
    L.nodes = graph.nodes;
    for (const auto& r : graph.resources)
        L.descriptors[r.id] = r;
    if (options.weight_views)
        LowerWeightViews(graph, options.native_half_weights, L);

    HipVmOptimizationResult result;
    HipVmProgram& p = result.program;
    p.name = graph.name;
    p.abi = "vm:" + graph.state_abi;
    p.state_schema = graph.state_schema;
    p.state_version = 1;
    std::map<std::string, std::string> physical;
    std::set<std::string> used;   // resources a kept node binds, views counted as their sources
    for (const auto& n : L.nodes)
        for (const auto& b : n.resources) {
            const auto a = L.aliases.find(b.resource);
            used.insert(a != L.aliases.end() ? a->second : b.resource);
        }
    if (options.reuse_local_storage) {
        std::vector<TensorDescriptor> locals;
        for (const auto& [id, slot] : PlanLocal(graph, L, locals))
            physical[id] = "local." + std::to_string(slot);
        for (size_t s = 0; s < locals.size(); s++)
            p.AddSlot({"local." + std::to_string(s), locals[s], VmAccess::ReadWrite, VmSlotScope::Local, ""});
        result.local_slots = static_cast<int>(locals.size());
    }
    std::set<std::string> endpoints(graph.inputs.begin(), graph.inputs.end());
    endpoints.insert(graph.outputs.begin(), graph.outputs.end());
    for (const auto& s : graph.state)
        endpoints.insert(s.resource);
    for (const auto& r : graph.resources) {
        if (L.aliases.count(r.id) || physical.count(r.id))
            continue;
        if (!used.count(r.id) && !endpoints.count(r.id))
            continue;   // not retained: nothing binds it
        physical[r.id] = r.id;
        const VmSlotScope scope = r.Scope() == GraphResourceScope::Global    ? VmSlotScope::Global
                                  : r.Scope() == GraphResourceScope::Session ? VmSlotScope::Session
                                                                             : VmSlotScope::Local;
        const bool ro = r.kind == GraphResourceKind::Weight || r.kind == GraphResourceKind::Constant ||
                        r.kind == GraphResourceKind::Input;
        p.AddSlot({r.id, r.tensor, ro ? VmAccess::ReadOnly : VmAccess::ReadWrite, scope, r.binding_key});
    }
    for (const auto& [alias, source] : L.aliases)
        physical[alias] = physical.at(source);
    for (const auto& s : graph.state)
        p.state.push_back({s.name, physical.at(s.resource)});
    result.removed_nodes = L.removed;

    std::map<std::string, std::string> definitions;   // operator key -> definition id
    std::set<std::string> diagnostics;
    const int64_t now = options.now_unix_seconds
                            ? options.now_unix_seconds
                            : std::chrono::duration_cast<std::chrono::seconds>(
                                  std::chrono::system_clock::now().time_since_epoch())
                                  .count();
    for (const auto& n : L.nodes) {
        std::vector<InstructionParameter> params;
        for (const auto& b : n.resources)
            params.push_back(InstructionParameter::Tensor(b.port, L.descriptors.at(b.resource).tensor,
                                                          b.access == R ? R : W, physical.at(b.resource)));
        for (const auto& [k, v] : n.attributes)
            params.push_back(InstructionParameter::Attribute(k, v));
        const auto instruction = registry->Resolve(CollectionOf(n.operation), n.operation, InstructionTarget::Hip());
        HipVmNodeReport rep;
        rep.node = n.id;
        rep.operation = n.operation;
        rep.threads = options.threads_per_group;
        std::string implementation;   // empty: the instruction's own
        uint64_t outputs = 0;
        for (const auto& prm : params)
            if (prm.kind == InstructionParameter::Kind::Tensor && prm.access != R)
                outputs = prm.tensor.ElementCount();
        if (n.operation == "core.mat-vec" || n.operation == "quant.mat-vec") {
            result.matvec.calls++;
            const auto choice = options.gpu_matvec
                                    ? options.gpu_matvec->Select(params, options, now)
                                    : std::make_pair(true, std::string("Default GPU MatVec implementation: cooperative."));
            rep.matvec = true;
            rep.cooperative = choice.first;
            rep.diagnostic = choice.second;
            diagnostics.insert(choice.second);
            if (choice.first) {
                result.matvec.cooperative_calls++;
                rep.threads = HipMatVecExecution::Threads;
                // the cooperative grid of GpuMatVecExecution.Groups: one row per group, y splits past 65535
                const uint32_t y = static_cast<uint32_t>((outputs + 65534) / 65535);
                rep.groups[0] = static_cast<uint32_t>((outputs + y - 1) / y);
                rep.groups[1] = y;
            } else {
                implementation = "any_shape";
            }
        }
        if (!rep.cooperative) {
            const uint64_t groups = (outputs + rep.threads - 1) / rep.threads;
            if (groups > 65535)
                throw NotSupportedException("Node '" + n.id + "' exceeds the configured one-dimensional GPU dispatch grid.");
            rep.groups[0] = static_cast<uint32_t>(groups < 1 ? 1 : groups);
        }
        // the operator key: one definition per distinct operator
        std::ostringstream key;
        key << n.operation << '@' << n.version << '|' << InstructionTarget::Hip().architecture << '|' << rep.threads
            << '|' << implementation << '|' << static_cast<int>(n.requirements.minimum_arithmetic_type) << ','
            << static_cast<int>(n.requirements.minimum_accumulator_type);
        for (const auto& prm : params)
            if (prm.kind == InstructionParameter::Kind::Tensor)
                key << '|' << prm.name << ':' << static_cast<int>(prm.access) << ':'
                    << kElementTypeNames[static_cast<int>(prm.tensor.element_type)] << '['
                    << Join(prm.tensor.dimensions, ",") << ']';
        for (const auto& [k, v] : n.attributes)
            key << '|' << k << '=' << v;
        auto dit = definitions.find(key.str());
        if (dit == definitions.end()) {
            char id[32];
            std::snprintf(id, sizeof id, "op.%04d", static_cast<int>(definitions.size()));
            dit = definitions.emplace(key.str(), id).first;
        }
        rep.definition = dit->second;
        HipVmKernelLaunch launch;
        launch.definition = rep.definition;
        launch.threads = rep.threads;
        std::copy(rep.groups, rep.groups + 3, launch.groups);
        launch.implementation_variant = implementation;
        p.AddKernelDispatch("forward", instruction, params, n.requirements, launch);
        rep.implementation = p.Entries().at("forward").back().recording.operation;
        result.nodes.push_back(std::move(rep));
    }
    result.definitions = static_cast<int>(definitions.size());
    result.matvec.diagnostics.assign(diagnostics.begin(), diagnostics.end());
    return result;
}

std::string JsonString(const std::string& s)
{
    std::string o = "\"";
    for (char c : s) {
        const unsigned char u = static_cast<unsigned char>(c);
        if (c == '"' || c == '\\') {
            o += '\\';
            o += c;
        } else if (u < 0x20) {
            static const char hex[] = "0123456789abcdef";
            o += "\\u00";
            o += hex[u >> 4];
            o += hex[u & 15];
        } else {
            o += c;
        }
    }
    return o + "\"";
}

std::string OptimizationReportJson(const HipVmOptimizationResult& r)
{
    const auto str = [](const std::string& s) { return JsonString(s); };
    std::ostringstream j;
    j << "{\"matvec\":{\"calls\":" << r.matvec.calls << ",\"cooperativeCalls\":" << r.matvec.cooperative_calls
      << ",\"diagnostics\":[";
    for (size_t i = 0; i < r.matvec.diagnostics.size(); i++)
        j << (i ? "," : "") << str(r.matvec.diagnostics[i]);
    j << "]},\"removedNodes\":" << r.removed_nodes << ",\"localSlots\":" << r.local_slots
      << ",\"definitions\":" << r.definitions << ",\"nodes\":[";
    for (size_t i = 0; i < r.nodes.size(); i++) {
        const auto& n = r.nodes[i];
        j << (i ? "," : "") << "{\"node\":" << str(n.node) << ",\"operation\":" << str(n.operation)
          << ",\"definition\":" << str(n.definition) << ",\"implementation\":" << str(n.implementation)
          << ",\"threads\":" << n.threads << ",\"groups\":[" << n.groups[0] << "," << n.groups[1] << ","
          << n.groups[2] << "],\"cooperative\":" << (n.cooperative ? "true" : "false")
          << ",\"diagnostic\":" << str(n.diagnostic) << "}";
    }
    j << "]}";
    return j.str();
}

}  // namespace sharpinference
