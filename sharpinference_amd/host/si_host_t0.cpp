// The T0 primitive and portable tensor instructions of the reference's
// TierZeroFloat32 collection on the HIP target (TierZeroInstruction.cs,
// TierZeroOperationContracts.cs, PortableTensorOperationContracts.cs), and
// their launches through the C ABI (si_hip_t0_*).  core.mat-vec,
// core.gather-row and core.tensor.batched-mat-vec are in si_host_ops.cpp.
#include "si_host.hpp"

#include <cmath>
#include <cstdlib>
#include <set>

namespace sharpinference {

namespace {

constexpr GraphElementType F32 = GraphElementType::Float32;
constexpr GraphElementType F16 = GraphElementType::Float16;
constexpr GraphResourceAccess R = GraphResourceAccess::Read;
constexpr GraphResourceAccess W = GraphResourceAccess::Write;

using Dims = std::vector<int64_t>;

// Elementwise operators: name -> si_hip_t0_op.
const std::map<std::string, int>& ElementwiseOps()
{
    static const std::map<std::string, int> ops = {
        {"core.copy", SI_HIP_T0_COPY},         {"core.add", SI_HIP_T0_ADD},
        {"core.subtract", SI_HIP_T0_SUBTRACT}, {"core.multiply", SI_HIP_T0_MULTIPLY},
        {"core.divide", SI_HIP_T0_DIVIDE},     {"core.maximum", SI_HIP_T0_MAXIMUM},
        {"core.exp", SI_HIP_T0_EXP},           {"core.tanh", SI_HIP_T0_TANH},
        {"core.sigmoid", SI_HIP_T0_SIGMOID},   {"core.rsqrt", SI_HIP_T0_RSQRT},
        {"core.square", SI_HIP_T0_SQUARE},     {"core.relu", SI_HIP_T0_RELU},
    };
    return ops;
}

bool Binary(int op) { return op >= SI_HIP_T0_ADD && op <= SI_HIP_T0_MAXIMUM; }

const InstructionParameter* Find(const std::vector<InstructionParameter>& ps, const std::string& n)
{
    for (const auto& p : ps)
        if (p.name == n)
            return &p;
    return nullptr;
}

int64_t Count(const Dims& d)
{
    int64_t n = 1;
    for (int64_t v : d)
        n *= v;
    return n;
}

int NonNegative(const std::string& t)
{
    long long v = 0;
    bool ok = !t.empty() && t.size() <= 10;
    for (char c : t) {
        ok &= c >= '0' && c <= '9';
        v = v * 10 + (c - '0');
    }
    return ok && v <= INT32_MAX ? static_cast<int>(v) : -1;
}

// One T0 operator other than the three matrix operators, with the
// contract's ports, element types and attributes (TierZeroInstruction.cs:
// 81-107) and its shape rules.
class TierZeroOpInstruction : public HipFixedInstruction {
public:
    TierZeroOpInstruction(const std::string& name, std::vector<std::vector<InstructionPort>> ports,
                          std::vector<std::string> attributes)
        : HipFixedInstruction(InstructionCollectionIds::TierZeroFloat32, name, std::move(ports), std::move(attributes))
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& ps) const override
    {
        for (const auto& p : ps)
            if (p.kind == InstructionParameter::Kind::Tensor && p.tensor.dimensions.empty())
                Fail("requires dense, non-scalar tensors.");
        const std::string& n = Name();
        const Dims& out = TensorOf(ps, "output").tensor.dimensions;
        const auto in = [&](const char* port) -> const Dims& { return TensorOf(ps, port).tensor.dimensions; };
        bool ok = true;
        if (ElementwiseOps().count(n)) {
            const int op = ElementwiseOps().at(n);
            ok = Binary(op) ? in("left") == out && in("right") == out : in("input") == out;
        } else if (n == "core.reduce-sum" || n == "core.reduce-mean") {
            ok = out == Dims{1};
        } else if (n == "core.tensor.fill") {
            const std::string& t = Find(ps, "value")->value;
            char* end = nullptr;
            const float v = std::strtof(t.c_str(), &end);
            ok = !t.empty() && !std::isspace(static_cast<unsigned char>(t.front())) &&
                 end == t.c_str() + t.size() && std::isfinite(v);
        } else if (n == "core.tensor.cast-f16-f32") {
            ok = in("input") == out;
        } else if (n == "core.tensor.reshape") {
            ok = Count(in("input")) == Count(out);
        } else if (n == "core.tensor.broadcast") {
            const Dims& s = in("input");
            ok = s.size() <= out.size() && out.size() <= 4;
            for (size_t a = 0; ok && a < s.size(); a++)
                ok = s[a] == 1 || s[a] == out[out.size() - s.size() + a];
        } else if (n == "core.tensor.slice") {
            const Dims& s = in("input");
            const int axis = NonNegative(Find(ps, "axis")->value);
            const int start = NonNegative(Find(ps, "start")->value);
            const int length = NonNegative(Find(ps, "length")->value);
            ok = axis >= 0 && start >= 0 && length > 0 && s.size() <= 4 && axis < static_cast<int>(s.size()) &&
                 static_cast<int64_t>(start) + length <= s[axis] && out.size() == s.size();
            for (size_t a = 0; ok && a < s.size(); a++)
                ok = out[a] == (static_cast<int>(a) == axis ? length : s[a]);
        } else if (n == "core.tensor.reduce-last-sum" || n == "core.tensor.reduce-last-mean") {
            const Dims& s = in("input");
            ok = (s.size() == 2 || s.size() == 3) && out.size() == s.size() - 1 &&
                 std::equal(out.begin(), out.end(), s.begin());
        } else if (n == "core.tensor.head-outer") {
            const Dims& l = in("left");
            const Dims& r = in("right");
            ok = l.size() == 2 && r.size() == 2 && out.size() == 3 && l[0] == r[0] && out[0] == l[0] &&
                 out[1] == l[1] && out[2] == r[1];
        }
        if (!ok)
            Fail("incompatible dimensions or attributes.");
    }

    InstructionRecording Generate(const std::vector<InstructionParameter>& ps) const override
    {
        const std::string& n = Name();
        if (ElementwiseOps().count(n))
            return {"si_hip_t0_elementwise." + n.substr(5), ps};
        if (n == "core.tensor.reshape")
            return {"si_hip_t0_elementwise.copy", ps};
        if (n == "core.reduce-sum" || n == "core.reduce-mean")
            return {std::string("si_hip_t0_reduce.") + (n == "core.reduce-sum" ? "sum" : "mean"), ps};
        if (n == "core.tensor.reduce-last-sum" || n == "core.tensor.reduce-last-mean")
            return {std::string("si_hip_t0_reduce_last.") + (n == "core.tensor.reduce-last-sum" ? "sum" : "mean"), ps};
        if (n == "core.tensor.fill")
            return {"si_hip_t0_fill", ps};
        if (n == "core.tensor.cast-f16-f32")
            return {"si_hip_t0_cast_f16_f32", ps};
        if (n == "core.tensor.broadcast")
            return {"si_hip_t0_broadcast", ps};
        if (n == "core.tensor.slice")
            return {"si_hip_t0_slice", ps};
        return {"si_hip_t0_head_outer", ps};
    }
};

}  // namespace

std::shared_ptr<const Instruction> MakeTierZeroOpInstruction(const std::string& name)
{
    using P = std::vector<std::vector<InstructionPort>>;
    const P unary{{{"input", F32, R}, {"output", F32, W}}};
    const P binary{{{"left", F32, R}, {"right", F32, R}, {"output", F32, W}}};
    if (ElementwiseOps().count(name))
        return std::make_shared<TierZeroOpInstruction>(name, Binary(ElementwiseOps().at(name)) ? binary : unary,
                                                       std::vector<std::string>{});
    if (name == "core.reduce-sum" || name == "core.reduce-mean" || name == "core.tensor.reshape" ||
        name == "core.tensor.broadcast" || name == "core.tensor.reduce-last-sum" ||
        name == "core.tensor.reduce-last-mean")
        return std::make_shared<TierZeroOpInstruction>(name, unary, std::vector<std::string>{});
    if (name == "core.tensor.fill")
        return std::make_shared<TierZeroOpInstruction>(name, P{{{"output", F32, W}}}, std::vector<std::string>{"value"});
    if (name == "core.tensor.cast-f16-f32")
        return std::make_shared<TierZeroOpInstruction>(name, P{{{"input", F16, R}, {"output", F32, W}}},
                                                       std::vector<std::string>{});
    if (name == "core.tensor.slice")
        return std::make_shared<TierZeroOpInstruction>(name, unary,
                                                       std::vector<std::string>{"axis", "start", "length"});
    if (name == "core.tensor.head-outer")
        return std::make_shared<TierZeroOpInstruction>(name, binary, std::vector<std::string>{});
    return nullptr;
}

bool LaunchTierZeroOp(si_hip_context* ctx, const InstructionRecording& r,
                      const std::function<void*(const InstructionParameter&)>& address)
{
    const std::string& op = r.operation;
    if (op.rfind("si_hip_t0_", 0) != 0)
        return false;
    const auto ptr = [&](const char* n) { return address(*Find(r.parameters, n)); };
    const auto dims = [&](const char* n) -> const Dims& { return Find(r.parameters, n)->tensor.dimensions; };
    const int64_t count = static_cast<int64_t>(Find(r.parameters, "output")->tensor.ElementCount());
    float* out = static_cast<float*>(ptr("output"));
    if (op.rfind("si_hip_t0_elementwise.", 0) == 0) {
        const auto it = ElementwiseOps().find("core." + op.substr(22));
        if (it == ElementwiseOps().end())
            throw NotSupportedException("Unknown T0 launch '" + op + "'.");
        const bool binary = Binary(it->second);
        Check(si_hip_t0_elementwise(ctx, it->second, static_cast<const float*>(ptr(binary ? "left" : "input")),
                                    binary ? static_cast<const float*>(ptr("right")) : nullptr, out, count),
              ctx);
    } else if (op == "si_hip_t0_reduce.sum" || op == "si_hip_t0_reduce.mean") {
        Check(si_hip_t0_reduce_last(ctx, op == "si_hip_t0_reduce.mean", static_cast<const float*>(ptr("input")), out, 1,
                                    Count(dims("input"))),
              ctx);
    } else if (op == "si_hip_t0_reduce_last.sum" || op == "si_hip_t0_reduce_last.mean") {
        const Dims& s = dims("input");
        Check(si_hip_t0_reduce_last(ctx, op == "si_hip_t0_reduce_last.mean", static_cast<const float*>(ptr("input")),
                                    out, Count(s) / s.back(), s.back()),
              ctx);
    } else if (op == "si_hip_t0_fill") {
        Check(si_hip_t0_fill(ctx, std::strtof(Find(r.parameters, "value")->value.c_str(), nullptr), out, count), ctx);
    } else if (op == "si_hip_t0_cast_f16_f32") {
        Check(si_hip_t0_cast_f16_f32(ctx, ptr("input"), out, count), ctx);
    } else if (op == "si_hip_t0_broadcast") {
        const Dims& s = dims("input");
        const Dims& d = dims("output");
        Check(si_hip_t0_broadcast(ctx, static_cast<const float*>(ptr("input")), static_cast<int>(s.size()), s.data(),
                                  out, static_cast<int>(d.size()), d.data()),
              ctx);
    } else if (op == "si_hip_t0_slice") {
        const Dims& s = dims("input");
        Check(si_hip_t0_slice(ctx, static_cast<const float*>(ptr("input")), static_cast<int>(s.size()), s.data(),
                              NonNegative(Find(r.parameters, "axis")->value),
                              NonNegative(Find(r.parameters, "start")->value),
                              NonNegative(Find(r.parameters, "length")->value), out),
              ctx);
    } else if (op == "si_hip_t0_head_outer") {
        const Dims& l = dims("left");
        Check(si_hip_t0_head_outer(ctx, static_cast<const float*>(ptr("left")), static_cast<const float*>(ptr("right")),
                                   out, l[0], l[1], dims("right")[1]),
              ctx);
    } else {
        throw NotSupportedException("Unknown T0 launch '" + op + "'.");
    }
    return true;
}

}  // namespace sharpinference
