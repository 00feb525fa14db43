// The reference's T0 and transformer instruction collections on the HIP
// target, and the Phi-4 decode program built from them dispatch by
// dispatch (si_host.hpp).
#include "si_host.hpp"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <set>

namespace sharpinference {

namespace {

const InstructionParameter* FindParameter(const std::vector<InstructionParameter>& parameters, const std::string& name)
{
    for (const auto& p : parameters)
        if (p.name == name)
            return &p;
    return nullptr;
}

constexpr KernelPrecisionProfile kFp32{GraphElementType::Float32, GraphElementType::Float32};
constexpr GraphElementType F32 = GraphElementType::Float32;
constexpr GraphElementType F16 = GraphElementType::Float16;
constexpr GraphElementType I32 = GraphElementType::Int32;
constexpr GraphResourceAccess R = GraphResourceAccess::Read;
constexpr GraphResourceAccess W = GraphResourceAccess::Write;

uint64_t Count(const InstructionParameter& p) { return p.tensor.ElementCount(); }

}  // namespace

// ---- HipFixedInstruction -------------------------------------------------------------------

HipFixedInstruction::HipFixedInstruction(std::string collection, std::string name,
                                         std::vector<std::vector<InstructionPort>> signatures,
                                         std::vector<std::string> attributes)
    : collection_(std::move(collection)), name_(std::move(name)), signatures_(std::move(signatures)),
      attributes_(std::move(attributes))
{
}

std::vector<InstructionSignature> HipFixedInstruction::Signatures() const
{
    std::vector<InstructionSignature> out;
    for (const auto& ports : signatures_)
        out.push_back({ports, attributes_, kFp32});
    return out;
}

const InstructionParameter& HipFixedInstruction::TensorOf(const std::vector<InstructionParameter>& parameters,
                                                          const std::string& name) const
{
    const auto* p = FindParameter(parameters, name);
    if (!p || p->kind != InstructionParameter::Kind::Tensor)
        Fail("missing tensor parameter '" + name + "'.");
    return *p;
}

int HipFixedInstruction::PositiveInteger(const std::vector<InstructionParameter>& parameters,
                                         const std::string& name) const
{
    const std::string& text = FindParameter(parameters, name)->value;
    long long v = 0;
    bool ok = !text.empty() && text.size() <= 9;
    for (char c : text) {
        ok &= c >= '0' && c <= '9';
        v = v * 10 + (c - '0');
    }
    if (!ok || v <= 0)
        throw InstructionAdaptationException(InstructionCollectionIds::TransformerFloat32, name,
                                             "Attribute '" + name + "' must be a positive integer.");
    return static_cast<int>(v);
}

float HipFixedInstruction::PositiveFloat(const std::vector<InstructionParameter>& parameters,
                                         const std::string& name) const
{
    const std::string& text = FindParameter(parameters, name)->value;
    char* end = nullptr;
    const float v = std::strtof(text.c_str(), &end);
    if (text.empty() || end != text.c_str() + text.size() || !std::isfinite(v) || v <= 0.0f)
        throw InstructionAdaptationException(InstructionCollectionIds::TransformerFloat32, name,
                                             "Attribute '" + name + "' must be finite and positive.");
    return v;
}

// ---- T0 ----------------------------------------------------------------------------------------

TierZeroMatVecInstruction::TierZeroMatVecInstruction()
    : HipFixedInstruction(InstructionCollectionIds::TierZeroFloat32, "core.mat-vec",
                          {{{"matrix", F32, R}, {"input", F32, R}, {"output", F32, W}},
                           {{"matrix", F16, R}, {"input", F32, R}, {"output", F32, W}},
                           {{"weight", F32, R}, {"input", F32, R}, {"output", F32, W}},
                           {{"weight", F16, R}, {"input", F32, R}, {"output", F32, W}}},
                          {})
{
}

void TierZeroMatVecInstruction::Validate(const std::vector<InstructionParameter>& parameters) const
{
    const auto* m = FindParameter(parameters, "matrix");
    if (!m)
        m = FindParameter(parameters, "weight");
    const auto& x = TensorOf(parameters, "input");
    const auto& y = TensorOf(parameters, "output");
    const auto& d = m->tensor.dimensions;
    if (d.size() != 2 || x.tensor.dimensions != std::vector<int64_t>{d[1]} ||
        y.tensor.dimensions != std::vector<int64_t>{d[0]})
        Fail("incompatible dimensions.");
}

InstructionRecording TierZeroMatVecInstruction::Generate(const std::vector<InstructionParameter>& parameters) const
{
    return {"si_hip_gemv.dense", parameters};
}

TierZeroGatherRowInstruction::TierZeroGatherRowInstruction()
    : HipFixedInstruction(InstructionCollectionIds::TierZeroFloat32, "core.gather-row",
                          {{{"table", F32, R}, {"index", I32, R}, {"output", F32, W}},
                           {{"table", F16, R}, {"index", I32, R}, {"output", F32, W}}},
                          {})
{
}

void TierZeroGatherRowInstruction::Validate(const std::vector<InstructionParameter>& parameters) const
{
    const auto& t = TensorOf(parameters, "table");
    const auto& i = TensorOf(parameters, "index");
    const auto& y = TensorOf(parameters, "output");
    const auto& d = t.tensor.dimensions;
    if (d.size() != 2 || i.tensor.dimensions != std::vector<int64_t>{1} ||
        y.tensor.dimensions != std::vector<int64_t>{d[1]})
        Fail("incompatible dimensions.");
}

InstructionRecording TierZeroGatherRowInstruction::Generate(const std::vector<InstructionParameter>& parameters) const
{
    return {"si_hip_gather_row.dense", parameters};
}

TierZeroBatchedMatVecInstruction::TierZeroBatchedMatVecInstruction()
    : HipFixedInstruction(InstructionCollectionIds::TierZeroFloat32, "core.tensor.batched-mat-vec",
                          {{{"matrix", F32, R}, {"vector", F32, R}, {"output", F32, W}}}, {})
{
}

void TierZeroBatchedMatVecInstruction::Validate(const std::vector<InstructionParameter>& parameters) const
{
    const auto& m = TensorOf(parameters, "matrix").tensor.dimensions;
    const auto& v = TensorOf(parameters, "vector").tensor.dimensions;
    const auto& y = TensorOf(parameters, "output").tensor.dimensions;
    if (m.size() != 3 || v != std::vector<int64_t>{m[0], m[2]} || y != std::vector<int64_t>{m[0], m[1]})
        Fail("incompatible dimensions.");
}

InstructionRecording TierZeroBatchedMatVecInstruction::Generate(const std::vector<InstructionParameter>& parameters) const
{
    return {"si_hip_batched_matvec", parameters};
}

std::vector<InstructionCollectionDescription> HipTierZeroInstructions::QueryInstructionCollection() const
{
    return {{InstructionCollectionIds::TierZeroFloat32, "T0 FP32 primitives", 0, InstructionTarget::Hip()}};
}

std::vector<std::shared_ptr<const Instruction>> HipTierZeroInstructions::QueryInstruction(
    const std::string& collection_id, const std::string& name) const
{
    if (collection_id != InstructionCollectionIds::TierZeroFloat32)
        return {};
    if (name == "core.mat-vec")
        return {std::make_shared<TierZeroMatVecInstruction>()};
    if (name == "core.gather-row")
        return {std::make_shared<TierZeroGatherRowInstruction>()};
    if (name == "core.tensor.batched-mat-vec")
        return {std::make_shared<TierZeroBatchedMatVecInstruction>()};
    if (auto op = MakeTierZeroOpInstruction(name))
        return {op};
    return {};
}

// ---- transformer collection ----------------------------------------------------------------

namespace {

class RmsNormInstruction : public HipFixedInstruction {
public:
    RmsNormInstruction()
        : HipFixedInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.rms-norm",
                              {{{"input", F32, R}, {"weight", F32, R}, {"output", F32, W}}}, {"epsilon"})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        PositiveFloat(p, "epsilon");
        const uint64_t n = Count(TensorOf(p, "output"));
        if (Count(TensorOf(p, "input")) != n || Count(TensorOf(p, "weight")) != n)
            Fail("input, weight and output must hold the same number of values.");
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_rms_norm", p};
    }
};

class ResidualRmsNormInstruction : public HipFixedInstruction {
public:
    ResidualRmsNormInstruction()
        : HipFixedInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.residual-rms-norm",
                              {{{"hidden", F32, R},
                                {"residual", F32, R},
                                {"weight", F32, R},
                                {"updated", F32, W},
                                {"output", F32, W}}},
                              {"epsilon"})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        PositiveFloat(p, "epsilon");
        const uint64_t n = Count(TensorOf(p, "output"));
        for (const char* port : {"hidden", "residual", "weight", "updated"})
            if (Count(TensorOf(p, port)) != n)
                Fail("every port must hold the same number of values.");
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_residual_rms_norm", p};
    }
};

class SwiGluInstruction : public HipFixedInstruction {
public:
    SwiGluInstruction()
        : HipFixedInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.swiglu",
                              {{{"gate_up", F32, R}, {"output", F32, W}}}, {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        if (Count(TensorOf(p, "gate_up")) != 2 * Count(TensorOf(p, "output")))
            Fail("gate_up must hold twice the output's values.");
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_swiglu", p};
    }
};

std::vector<std::vector<InstructionPort>> CacheSignatures(
    const std::function<std::vector<InstructionPort>(GraphElementType)>& ports)
{
    return {ports(F32), ports(F16)};
}

class RopeKvWriteInstruction : public HipFixedInstruction {
public:
    RopeKvWriteInstruction()
        : HipFixedInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.rope-kv-write",
                              CacheSignatures([](GraphElementType c) {
                                  return std::vector<InstructionPort>{{"qkv", F32, R},         {"position", I32, R},
                                                                      {"frequencies", F32, R}, {"query", F32, W},
                                                                      {"key_cache", c, W},     {"value_cache", c, W}};
                              }),
                              {"head_size", "rotary_size", "rope_scale"})
    {
    }

protected:
    // GpuTransformerInstructionCollection.cs:474-494.
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const int head = PositiveInteger(p, "head_size"), rotary = PositiveInteger(p, "rotary_size");
        PositiveFloat(p, "rope_scale");
        const auto& k = TensorOf(p, "key_cache").tensor.dimensions;
        const auto& v = TensorOf(p, "value_cache").tensor.dimensions;
        const uint64_t q = Count(TensorOf(p, "query"));
        if (k.size() != 3 || v != k || k[2] != head || rotary > head || rotary % 2 != 0 || q % head != 0)
            Fail("Invalid query, cache, head, or rotary dimensions.");
        if (Count(TensorOf(p, "frequencies")) != static_cast<uint64_t>(rotary / 2))
            Fail("RoPE frequency shape is invalid.");
        if (Count(TensorOf(p, "qkv")) != q + 2 * static_cast<uint64_t>(k[1] * k[2]))
            Fail("QKV shape does not match query and cache shapes.");
        if (Count(TensorOf(p, "position")) != 1)
            Fail("position must hold one value.");
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_rope_kv_write", p};
    }
};

class GroupedQueryAttentionInstruction : public HipFixedInstruction {
public:
    GroupedQueryAttentionInstruction()
        : HipFixedInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.grouped-query-attention",
                              CacheSignatures([](GraphElementType c) {
                                  return std::vector<InstructionPort>{{"query", F32, R},
                                                                      {"key_cache", c, R},
                                                                      {"value_cache", c, R},
                                                                      {"position", I32, R},
                                                                      {"output", F32, W}};
                              }),
                              {})
    {
    }

protected:
    // GpuTransformerInstructionCollection.cs:64-83.
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto& k = TensorOf(p, "key_cache").tensor.dimensions;
        if (k.size() != 3 || TensorOf(p, "value_cache").tensor.dimensions != k)
            Fail("Expected matching rank-three key and value caches.");
        const uint64_t q = Count(TensorOf(p, "query")), o = Count(TensorOf(p, "output"));
        if (q != o || q % static_cast<uint64_t>(k[2]) != 0)
            Fail("Query and output must contain complete matching heads.");
        if ((q / static_cast<uint64_t>(k[2])) % static_cast<uint64_t>(k[1]) != 0)
            Fail("Query heads must be divisible by key/value heads.");
        if (Count(TensorOf(p, "position")) != 1)
            Fail("position must hold one value.");
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_grouped_query_attention", p};
    }
};

class ArgMaxInstruction : public HipFixedInstruction {
public:
    ArgMaxInstruction()
        : HipFixedInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.argmax",
                              {{{"input", F32, R}, {"output", I32, W}}}, {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        if (Count(TensorOf(p, "output")) != 1)
            Fail("Argmax output must be scalar.");
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_argmax", p};
    }
};

// ---- batched (prefill) operators: GpuBatchTransformerInstructions.cs ------------------------

// Shape helpers with the reference's rules and messages
// (GpuBatchTransformerInstructions.cs:12-96).
class BatchInstruction : public HipFixedInstruction {
public:
    using HipFixedInstruction::HipFixedInstruction;

protected:
    std::pair<int64_t, int64_t> BatchMatrix(const std::vector<InstructionParameter>& p, const std::string& name) const
    {
        const auto& d = Rank(p, name, 2);
        if (d[0] <= 0 || d[1] <= 0)
            Fail("'" + name + "' dimensions must be positive.");
        return {d[0], d[1]};
    }
    int64_t Vector(const std::vector<InstructionParameter>& p, const std::string& name) const
    {
        const auto& d = Rank(p, name, 1);
        if (d[0] <= 0)
            Fail("'" + name + "' dimensions must be positive.");
        return d[0];
    }
    std::vector<int64_t> Cache(const std::vector<InstructionParameter>& p, const std::string& name) const
    {
        const auto& d = Rank(p, name, 3);
        for (const int64_t v : d)
            if (v <= 0)
                Fail("'" + name + "' dimensions must be positive.");
        return d;
    }
    void RequireControl(const std::vector<InstructionParameter>& p) const
    {
        const auto& d = TensorOf(p, "control").tensor.dimensions;
        if (d.size() != 1 || d[0] != 2)
            Fail("'control' must have shape [2].");
    }
    void RequireSameShape(const std::vector<InstructionParameter>& p, const std::string& a, const std::string& b) const
    {
        if (TensorOf(p, a).tensor.dimensions != TensorOf(p, b).tensor.dimensions)
            Fail("'" + a + "' and '" + b + "' must have matching shapes.");
    }
    // The HIP launches hold at most 16 batch rows (the reference's prefill batch).
    void RequireBatch(int64_t batch) const
    {
        if (batch > 16)
            Fail("the HIP batched operators take at most 16 rows.");
    }

private:
    const std::vector<int64_t>& Rank(const std::vector<InstructionParameter>& p, const std::string& name,
                                     size_t rank) const
    {
        const auto& d = TensorOf(p, name).tensor.dimensions;
        if (d.size() != rank)
            Fail("'" + name + "' must have rank " + std::to_string(rank) + ".");
        return d;
    }
};

class BatchRmsNormInstruction : public BatchInstruction {
public:
    BatchRmsNormInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-rms-norm",
                           {{{"input", F32, R}, {"weight", F32, R}, {"control", I32, R}, {"output", F32, W}}},
                           {"epsilon"})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto [batch, width] = BatchMatrix(p, "input");
        RequireSameShape(p, "input", "output");
        if (Vector(p, "weight") != width)
            Fail("'weight' must have shape [H].");
        RequireControl(p);
        PositiveFloat(p, "epsilon");
        RequireBatch(batch);
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_rms_norm", p};
    }
};

class BatchResidualRmsNormInstruction : public BatchInstruction {
public:
    BatchResidualRmsNormInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-residual-rms-norm",
                           {{{"hidden", F32, R},
                             {"residual", F32, R},
                             {"weight", F32, R},
                             {"control", I32, R},
                             {"updated", F32, W},
                             {"output", F32, W}}},
                           {"epsilon"})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto [batch, width] = BatchMatrix(p, "hidden");
        RequireSameShape(p, "hidden", "residual");
        RequireSameShape(p, "hidden", "updated");
        RequireSameShape(p, "hidden", "output");
        if (Vector(p, "weight") != width)
            Fail("'weight' must have shape [H].");
        RequireControl(p);
        PositiveFloat(p, "epsilon");
        RequireBatch(batch);
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_residual_rms_norm", p};
    }
};

// The reference's weight is F16; F32 weights are a second signature here.
class BatchSharedMatVecInstruction : public BatchInstruction {
public:
    BatchSharedMatVecInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-shared-matvec",
                           {{{"weight", F16, R}, {"input", F32, R}, {"control", I32, R}, {"output", F32, W}},
                            {{"weight", F32, R}, {"input", F32, R}, {"control", I32, R}, {"output", F32, W}}},
                           {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto [out_size, in_size] = BatchMatrix(p, "weight");
        const auto [batch, in_width] = BatchMatrix(p, "input");
        const auto [out_batch, out_width] = BatchMatrix(p, "output");
        if (in_width != in_size || out_batch != batch || out_width != out_size)
            Fail("Expected weight [O,I], input [B,I], and output [B,O].");
        RequireControl(p);
        RequireBatch(batch);
        if (in_size % 32 != 0)
            Fail("the HIP batched mat-vec takes a multiple of 32 input columns.");
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_matvec.dense", p};
    }
};

class BatchSwiGluInstruction : public BatchInstruction {
public:
    BatchSwiGluInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-swiglu",
                           {{{"gate_up", F32, R}, {"control", I32, R}, {"output", F32, W}}}, {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto [batch, combined] = BatchMatrix(p, "gate_up");
        const auto [out_batch, width] = BatchMatrix(p, "output");
        if (combined != 2 * width || out_batch != batch)
            Fail("Expected gate_up [B,2I] and output [B,I].");
        RequireControl(p);
        RequireBatch(batch);
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_swiglu", p};
    }
};

class BatchRopeKvWriteInstruction : public BatchInstruction {
public:
    BatchRopeKvWriteInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-rope-kv-write",
                           CacheSignatures([](GraphElementType c) {
                               return std::vector<InstructionPort>{{"qkv", F32, R},         {"control", I32, R},
                                                                   {"frequencies", F32, R}, {"query", F32, W},
                                                                   {"key_cache", c, W},     {"value_cache", c, W}};
                           }),
                           {"head_size", "rotary_size", "rope_scale"})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto [batch, qkv_width] = BatchMatrix(p, "qkv");
        const auto [query_batch, query_size] = BatchMatrix(p, "query");
        const auto k = Cache(p, "key_cache");
        const auto v = Cache(p, "value_cache");
        const int head = PositiveInteger(p, "head_size"), rotary = PositiveInteger(p, "rotary_size");
        PositiveFloat(p, "rope_scale");
        const int64_t kv = k[1] * head;
        if (query_batch != batch || v != k || k[2] != head || query_size % head != 0 || rotary > head ||
            rotary % 2 != 0 || qkv_width != query_size + 2 * kv)
            Fail("Invalid qkv, query, cache, head, or rotary dimensions.");
        if (Vector(p, "frequencies") != rotary / 2)
            Fail("'frequencies' must have shape [rotary_size/2].");
        RequireControl(p);
        RequireBatch(batch);
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_rope_kv_write", p};
    }
};

class BatchGqaScoresInstruction : public BatchInstruction {
public:
    BatchGqaScoresInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-gqa-scores",
                           CacheSignatures([](GraphElementType c) {
                               return std::vector<InstructionPort>{
                                   {"query", F32, R}, {"key_cache", c, R}, {"control", I32, R}, {"scores", F32, W}};
                           }),
                           {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto [batch, query_size] = BatchMatrix(p, "query");
        const auto k = Cache(p, "key_cache");
        const auto& s = TensorOf(p, "scores").tensor.dimensions;
        if (s.size() != 3 || s[0] != batch || s[2] != k[0])
            Fail("'scores' must have shape [B,qheads,context].");
        if (s[1] <= 0 || s[1] % k[1] != 0 || query_size != s[1] * k[2])
            Fail("Incompatible query, cache, and GQA score shapes.");
        RequireControl(p);
        RequireBatch(batch);
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_gqa_scores", p};
    }
};

class BatchCausalSoftmaxInstruction : public BatchInstruction {
public:
    BatchCausalSoftmaxInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-causal-softmax",
                           {{{"scores", F32, R}, {"control", I32, R}, {"probabilities", F32, W}}}, {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto& s = TensorOf(p, "scores").tensor.dimensions;
        if (s.size() != 3)
            Fail("'scores' must have shape [B,heads,context].");
        RequireSameShape(p, "scores", "probabilities");
        if (s[0] <= 0 || s[1] <= 0 || s[2] <= 0)
            Fail("'scores' dimensions must be positive.");
        RequireControl(p);
        RequireBatch(s[0]);
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_causal_softmax", p};
    }
};

class BatchGqaValuesInstruction : public BatchInstruction {
public:
    BatchGqaValuesInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-gqa-values",
                           CacheSignatures([](GraphElementType c) {
                               return std::vector<InstructionPort>{{"probabilities", F32, R},
                                                                   {"value_cache", c, R},
                                                                   {"control", I32, R},
                                                                   {"output", F32, W}};
                           }),
                           {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto& pr = TensorOf(p, "probabilities").tensor.dimensions;
        if (pr.size() != 3)
            Fail("'probabilities' must have shape [B,qheads,context].");
        const auto v = Cache(p, "value_cache");
        const auto [out_batch, out_width] = BatchMatrix(p, "output");
        if (pr[0] <= 0 || pr[1] <= 0 || pr[2] != v[0] || pr[1] % v[1] != 0 || out_batch != pr[0] ||
            out_width != pr[1] * v[2])
            Fail("Incompatible probability, value cache, and output shapes.");
        RequireControl(p);
        RequireBatch(pr[0]);
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_gqa_values", p};
    }
};

class BatchSelectLastInstruction : public BatchInstruction {
public:
    BatchSelectLastInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-select-last",
                           {{{"input", F32, R}, {"control", I32, R}, {"output", F32, W}}}, {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto [batch, width] = BatchMatrix(p, "input");
        if (Vector(p, "output") != width)
            Fail("Expected input [B,H] and output [H].");
        RequireControl(p);
        RequireBatch(batch);
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_select_last", p};
    }
};

class BatchGatherRowsInstruction : public BatchInstruction {
public:
    BatchGatherRowsInstruction()
        : BatchInstruction(InstructionCollectionIds::TransformerFloat32, "transformer.batch-gather-rows",
                           {{{"table", F32, R}, {"control", I32, R}, {"output", F32, W}}}, {})
    {
    }

protected:
    void Validate(const std::vector<InstructionParameter>& p) const override
    {
        const auto [rows, width] = BatchMatrix(p, "table");
        const auto [batch, out_width] = BatchMatrix(p, "output");
        if (out_width != width)
            Fail("Expected table [N,H] and output [B,H].");
        RequireControl(p);
        RequireBatch(batch);
        (void)rows;
    }
    InstructionRecording Generate(const std::vector<InstructionParameter>& p) const override
    {
        return {"si_hip_batch_gather_rows", p};
    }
};

}  // namespace

std::vector<InstructionCollectionDescription> HipTransformerInstructions::QueryInstructionCollection() const
{
    return {{InstructionCollectionIds::TransformerFloat32, "FP32 transformer operations", 1, InstructionTarget::Hip()}};
}

std::vector<std::shared_ptr<const Instruction>> HipTransformerInstructions::QueryInstruction(
    const std::string& collection_id, const std::string& name) const
{
    if (collection_id != InstructionCollectionIds::TransformerFloat32)
        return {};
    if (name == "transformer.rms-norm") return {std::make_shared<RmsNormInstruction>()};
    if (name == "transformer.residual-rms-norm") return {std::make_shared<ResidualRmsNormInstruction>()};
    if (name == "transformer.swiglu") return {std::make_shared<SwiGluInstruction>()};
    if (name == "transformer.rope-kv-write") return {std::make_shared<RopeKvWriteInstruction>()};
    if (name == "transformer.grouped-query-attention") return {std::make_shared<GroupedQueryAttentionInstruction>()};
    if (name == "transformer.argmax") return {std::make_shared<ArgMaxInstruction>()};
    if (name == "transformer.batch-rms-norm") return {std::make_shared<BatchRmsNormInstruction>()};
    if (name == "transformer.batch-residual-rms-norm") return {std::make_shared<BatchResidualRmsNormInstruction>()};
    if (name == "transformer.batch-shared-matvec") return {std::make_shared<BatchSharedMatVecInstruction>()};
    if (name == "transformer.batch-swiglu") return {std::make_shared<BatchSwiGluInstruction>()};
    if (name == "transformer.batch-rope-kv-write") return {std::make_shared<BatchRopeKvWriteInstruction>()};
    if (name == "transformer.batch-gqa-scores") return {std::make_shared<BatchGqaScoresInstruction>()};
    if (name == "transformer.batch-causal-softmax") return {std::make_shared<BatchCausalSoftmaxInstruction>()};
    if (name == "transformer.batch-gqa-values") return {std::make_shared<BatchGqaValuesInstruction>()};
    if (name == "transformer.batch-select-last") return {std::make_shared<BatchSelectLastInstruction>()};
    if (name == "transformer.batch-gather-rows") return {std::make_shared<BatchGatherRowsInstruction>()};
    return {};
}

std::shared_ptr<const InstructionRegistry> DefaultHipRegistry()
{
    return std::make_shared<InstructionRegistry>(std::vector<std::shared_ptr<const IInstructionCollectionProvider>>{
        std::make_shared<HipQuantizedInstructions>(), std::make_shared<HipTierZeroInstructions>(),
        std::make_shared<HipTransformerInstructions>()});
}

// ---- the Phi-4 decode program -------------------------------------------------------------------

std::vector<float> Phi4RopeFrequencies(const Phi4ProgramShape& s)
{
    std::vector<float> f(s.rotary_dim / 2);
    for (int i = 0; i < s.rotary_dim / 2; i++)
        f[i] = 1.0f / std::pow(s.rope_base, 2.0f * static_cast<float>(i) / static_cast<float>(s.rotary_dim));
    return f;
}

namespace {

bool Dense(int fmt) { return fmt == SI_HIP_F16 || fmt == SI_HIP_F32; }

std::string FormatName(int fmt)
{
    switch (fmt) {
    case SI_HIP_Q8_0: return "q8_0";
    case SI_HIP_Q4_0: return "q4_0";
    case SI_HIP_Q4_K: return "q4_k";
    case SI_HIP_F16: return "f16";
    case SI_HIP_F32: return "f32";
    default: throw ArgumentException("format " + std::to_string(fmt) + " is not a weight format of the matrix kernels.");
    }
}

// A weight slot's tensor: typed [rows, columns] for F16 / F32 (core.mat-vec),
// Byte [rows, row_bytes] for the block formats (quant.mat-vec).
TensorDescriptor WeightTensor(int fmt, int64_t rows, int64_t columns)
{
    if (fmt == SI_HIP_F16)
        return {F16, {rows, columns}};
    if (fmt == SI_HIP_F32)
        return {F32, {rows, columns}};
    uint64_t rb = 0;
    Check(si_hip_tensor_bytes(fmt, 1, columns, &rb));
    return {GraphElementType::Byte, {rows, static_cast<int64_t>(rb)}};
}

TensorDescriptor Vec(int64_t n, GraphElementType t = F32) { return {t, {n}}; }

}  // namespace

namespace {

// The reference's prefill entry (Phi4D3D12TextSession.cs:952-1168) on the
// program's slots: 16-row batches of the fused prompt embeddings.
template <typename TensorFn, typename MatVecFn>
void AddPhi4Prefill(HipVmProgram& p, const Phi4ProgramShape& s, const std::shared_ptr<const InstructionRegistry>& registry,
                    const TensorFn& tensor, const MatVecFn& matvec)
{
    constexpr int64_t B = 16;
    const std::string E = "prefill_fused_16";
    const auto resolve = [&](const std::string& collection, const std::string& name) {
        return registry->Resolve(collection, name, InstructionTarget::Hip());
    };
    const auto& T = InstructionCollectionIds::TransformerFloat32;
    const auto quant_bmv = resolve(HipInstructionCollectionIds::QuantizedFloat32, "quant.batch-mat-vec");
    const auto dense_bmv = resolve(T, "transformer.batch-shared-matvec");
    const auto gather = resolve(T, "transformer.batch-gather-rows"), rms = resolve(T, "transformer.batch-rms-norm");
    const auto residual_rms = resolve(T, "transformer.batch-residual-rms-norm");
    const auto swiglu = resolve(T, "transformer.batch-swiglu"), rope = resolve(T, "transformer.batch-rope-kv-write");
    const auto scores = resolve(T, "transformer.batch-gqa-scores");
    const auto softmax = resolve(T, "transformer.batch-causal-softmax");
    const auto values = resolve(T, "transformer.batch-gqa-values");
    const auto last = resolve(T, "transformer.batch-select-last");
    const auto argmax = resolve(T, "transformer.argmax");
    const int64_t H = s.hidden, F = s.ffn, Q = s.hidden, KV = static_cast<int64_t>(s.kv_heads) * s.head_dim;
    const auto rw = VmAccess::ReadWrite;
    p.AddSlot({"fused_embeddings", {F32, {s.prompt_rows, H}}, VmAccess::ReadOnly, VmSlotScope::Local});
    for (const auto& [name, dims] : std::vector<std::pair<const char*, std::vector<int64_t>>>{
             {"batch_hidden", {B, H}}, {"batch_normalized", {B, H}}, {"batch_qkv", {B, Q + 2 * KV}},
             {"batch_query", {B, Q}}, {"batch_scores", {B, s.heads, s.context}},
             {"batch_probabilities", {B, s.heads, s.context}}, {"batch_attention", {B, H}},
             {"batch_projected", {B, H}}, {"batch_hidden_after_attention", {B, H}}, {"batch_gate_up", {B, 2 * F}},
             {"batch_activated", {B, F}}, {"batch_down", {B, H}}, {"batch_last", {H}}})
        p.AddSlot({name, {F32, dims}, rw, VmSlotScope::Local});

    using P = InstructionParameter;
    const PrecisionRequirement fp32{F32, F32};
    const auto control = tensor("control", "control", R, 0, nullptr);
    char eps[64], scale[64];
    std::snprintf(eps, sizeof eps, "%.9g", static_cast<double>(s.rms_eps));
    std::snprintf(scale, sizeof scale, "%.9g", static_cast<double>(s.rope_scale));
    const auto batch_matvec = [&](const std::string& weight, const std::string& input, const std::string& output,
                                  int64_t columns) {
        std::vector<P> args{tensor("weight", weight, R, 0, nullptr), tensor("input", input, R, 0, nullptr), control,
                            tensor("output", output, W, 0, nullptr)};
        if (Dense(s.weight_format)) {
            p.AddDispatch(E, dense_bmv, args, fp32);
        } else {
            args.push_back(P::Attribute("format", FormatName(s.weight_format)));
            args.push_back(P::Attribute("columns", std::to_string(columns)));
            p.AddDispatch(E, quant_bmv, args, fp32);
        }
    };
    const auto t = [&](const char* port, const std::string& slot, GraphResourceAccess access) {
        return tensor(port, slot, access, 0, nullptr);
    };
    p.AddDispatch(E, gather, {t("table", "fused_embeddings", R), control, t("output", "batch_hidden", W)}, fp32);
    p.AddDispatch(E, rms,
                  {t("input", "batch_hidden", R), t("weight", "attn_norm_0", R), control,
                   t("output", "batch_normalized", W), P::Attribute("epsilon", eps)},
                  fp32);
    for (int l = 0; l < s.layers; l++) {
        const std::string L = std::to_string(l);
        batch_matvec("qkv_weight_" + L, "batch_normalized", "batch_qkv", H);
        p.AddDispatch(E, rope,
                      {t("qkv", "batch_qkv", R), control, t("frequencies", "rope_frequencies", R),
                       t("query", "batch_query", W), t("key_cache", "key_cache_" + L, W),
                       t("value_cache", "value_cache_" + L, W), P::Attribute("head_size", std::to_string(s.head_dim)),
                       P::Attribute("rotary_size", std::to_string(s.rotary_dim)), P::Attribute("rope_scale", scale)},
                      fp32);
        p.AddDispatch(E, scores,
                      {t("query", "batch_query", R), t("key_cache", "key_cache_" + L, R), control,
                       t("scores", "batch_scores", W)},
                      fp32);
        p.AddDispatch(E, softmax, {t("scores", "batch_scores", R), control, t("probabilities", "batch_probabilities", W)},
                      fp32);
        p.AddDispatch(E, values,
                      {t("probabilities", "batch_probabilities", R), t("value_cache", "value_cache_" + L, R), control,
                       t("output", "batch_attention", W)},
                      fp32);
        batch_matvec("attn_output_weight_" + L, "batch_attention", "batch_projected", H);
        p.AddDispatch(E, residual_rms,
                      {t("hidden", "batch_hidden", R), t("residual", "batch_projected", R),
                       t("weight", "ffn_norm_" + L, R), control, t("updated", "batch_hidden_after_attention", W),
                       t("output", "batch_normalized", W), P::Attribute("epsilon", eps)},
                      fp32);
        batch_matvec("ffn_up_weight_" + L, "batch_normalized", "batch_gate_up", H);
        p.AddDispatch(E, swiglu, {t("gate_up", "batch_gate_up", R), control, t("output", "batch_activated", W)}, fp32);
        batch_matvec("ffn_down_weight_" + L, "batch_activated", "batch_down", F);
        const std::string next_norm = l + 1 < s.layers ? "attn_norm_" + std::to_string(l + 1) : "output_norm";
        p.AddDispatch(E, residual_rms,
                      {t("hidden", "batch_hidden_after_attention", R), t("residual", "batch_down", R),
                       t("weight", next_norm, R), control, t("updated", "batch_hidden", W),
                       t("output", "batch_normalized", W), P::Attribute("epsilon", eps)},
                      fp32);
    }
    p.AddDispatch(E, last, {t("input", "batch_normalized", R), control, t("output", "batch_last", W)}, fp32);
    matvec(s.head_format, s.tied ? "token_embedding" : "output_weight", "batch_last", "logits", H, E);
    p.AddDispatch(E, argmax, {t("input", "logits", R), t("output", "next_token", W)}, fp32);
}

}  // namespace

HipVmProgram BuildPhi4DecodeProgram(const Phi4ProgramShape& s)
{
    if (s.layers < 1 || s.hidden < 1 || s.heads < 1 || s.kv_heads < 1 || s.heads % s.kv_heads != 0 ||
        s.hidden != s.heads * s.head_dim || s.ffn < 1 || s.vocab < 1 || s.context < 1 || s.rotary_dim < 2 ||
        s.rotary_dim > s.head_dim || s.rotary_dim % 2 != 0 || s.prompt_rows < 0 || s.prompt_rows > s.context)
        throw ArgumentException("Invalid Phi-4 program shape.");
    if (s.cache_type != F32 && s.cache_type != F16)
        throw ArgumentException("The KV cache is Float32 or Float16.");
    if (s.tied && s.head_format != s.embed_format)
        throw ArgumentException("A tied vocabulary projection uses the embedding's format.");
    const auto registry = DefaultHipRegistry();
    const auto resolve = [&](const std::string& collection, const std::string& name) {
        return registry->Resolve(collection, name, InstructionTarget::Hip());
    };
    const auto quant_mv = resolve(HipInstructionCollectionIds::QuantizedFloat32, "quant.mat-vec");
    const auto t0_mv = resolve(InstructionCollectionIds::TierZeroFloat32, "core.mat-vec");
    const auto quant_gather = resolve(HipInstructionCollectionIds::QuantizedFloat32, "quant.gather-row");
    const auto t0_gather = resolve(InstructionCollectionIds::TierZeroFloat32, "core.gather-row");
    const auto& T = InstructionCollectionIds::TransformerFloat32;
    const auto rms = resolve(T, "transformer.rms-norm"), residual_rms = resolve(T, "transformer.residual-rms-norm");
    const auto swiglu = resolve(T, "transformer.swiglu"), rope = resolve(T, "transformer.rope-kv-write");
    const auto gqa = resolve(T, "transformer.grouped-query-attention"), argmax = resolve(T, "transformer.argmax");

    const int64_t H = s.hidden, F = s.ffn, Q = s.hidden, KV = static_cast<int64_t>(s.kv_heads) * s.head_dim;
    const int64_t QKV = Q + 2 * KV;
    HipVmProgram p;
    p.name = "phi4-hip-decode";
    p.abi = s.cache_type == F16 ? "phi4.decode.fp16" : "phi4.decode.fp32";
    p.state_schema = "phi4-kv-cache";
    const auto ro = VmAccess::ReadOnly, rw = VmAccess::ReadWrite;
    const auto session = VmSlotScope::Session, local = VmSlotScope::Local;
    p.AddSlot({"token_embedding", WeightTensor(s.embed_format, s.vocab, H), ro});
    if (!s.tied)
        p.AddSlot({"output_weight", WeightTensor(s.head_format, s.vocab, H), ro});
    p.AddSlot({"output_norm", Vec(H), ro});
    p.AddSlot({"rope_frequencies", Vec(s.rotary_dim / 2), ro});
    const TensorDescriptor cache{s.cache_type, {s.context, s.kv_heads, s.head_dim}};
    for (int l = 0; l < s.layers; l++) {
        const std::string L = std::to_string(l);
        p.AddSlot({"attn_norm_" + L, Vec(H), ro});
        p.AddSlot({"ffn_norm_" + L, Vec(H), ro});
        p.AddSlot({"qkv_weight_" + L, WeightTensor(s.weight_format, QKV, H), ro});
        p.AddSlot({"attn_output_weight_" + L, WeightTensor(s.weight_format, H, H), ro});
        p.AddSlot({"ffn_up_weight_" + L, WeightTensor(s.weight_format, 2 * F, H), ro});
        p.AddSlot({"ffn_down_weight_" + L, WeightTensor(s.weight_format, H, F), ro});
        p.AddSlot({"key_cache_" + L, cache, rw, session});
        p.AddSlot({"value_cache_" + L, cache, rw, session});
        p.state.push_back({"key_cache_" + L, "key_cache_" + L});
        p.state.push_back({"value_cache_" + L, "value_cache_" + L});
    }
    p.AddSlot({"control", Vec(2, I32), ro, local});
    for (const auto& [name, n] : std::vector<std::pair<const char*, int64_t>>{
             {"hidden", H}, {"hidden_after_attention", H}, {"normalized", H}, {"qkv", QKV}, {"query", Q},
             {"attention", H}, {"projected", H}, {"gate_up", 2 * F}, {"activated", F}, {"down", H},
             {"logits", s.vocab}})
        p.AddSlot({name, Vec(n), rw, local});
    p.AddSlot({"next_token", Vec(1, I32), rw, local});

    using P = InstructionParameter;
    const PrecisionRequirement fp32{F32, F32};
    const auto tensor = [&](const std::string& port, const std::string& slot, GraphResourceAccess access,
                            uint64_t offset = 0, const TensorDescriptor* view = nullptr) {
        const int i = p.SlotIndex(slot);
        return P::Tensor(port, view ? *view : p.Slots()[i].tensor, access, slot, offset);
    };
    const TensorDescriptor one_int = Vec(1, I32);
    const auto token = tensor("index", "control", R, 0, &one_int);
    const auto position = tensor("position", "control", R, 4, &one_int);
    const std::string eps = [&] {
        char b[64];
        std::snprintf(b, sizeof b, "%.9g", static_cast<double>(s.rms_eps));
        return std::string(b);
    }();
    const auto matvec = [&](int fmt, const std::string& weight, const std::string& input, const std::string& output,
                            int64_t columns, const std::string& entry = "decode") {
        std::vector<P> args{tensor("weight", weight, R), tensor("input", input, R), tensor("output", output, W)};
        if (Dense(fmt)) {
            p.AddDispatch(entry, t0_mv, args, fp32);
        } else {
            args.push_back(P::Attribute("format", FormatName(fmt)));
            args.push_back(P::Attribute("columns", std::to_string(columns)));
            p.AddDispatch(entry, quant_mv, args, fp32);
        }
    };
    // embedding
    {
        std::vector<P> args{tensor("table", "token_embedding", R), token, tensor("output", "hidden", W)};
        if (Dense(s.embed_format)) {
            p.AddDispatch("decode", t0_gather, args, fp32);
        } else {
            args.push_back(P::Attribute("format", FormatName(s.embed_format)));
            args.push_back(P::Attribute("columns", std::to_string(H)));
            p.AddDispatch("decode", quant_gather, args, fp32);
        }
    }
    p.AddDispatch("decode", rms,
                  {tensor("input", "hidden", R), tensor("weight", "attn_norm_0", R), tensor("output", "normalized", W),
                   P::Attribute("epsilon", eps)},
                  fp32);
    char scale[64];
    std::snprintf(scale, sizeof scale, "%.9g", static_cast<double>(s.rope_scale));
    for (int l = 0; l < s.layers; l++) {
        const std::string L = std::to_string(l);
        matvec(s.weight_format, "qkv_weight_" + L, "normalized", "qkv", H);
        p.AddDispatch("decode", rope,
                      {tensor("qkv", "qkv", R), position, tensor("frequencies", "rope_frequencies", R),
                       tensor("query", "query", W), tensor("key_cache", "key_cache_" + L, W),
                       tensor("value_cache", "value_cache_" + L, W),
                       P::Attribute("head_size", std::to_string(s.head_dim)),
                       P::Attribute("rotary_size", std::to_string(s.rotary_dim)), P::Attribute("rope_scale", scale)},
                      fp32);
        p.AddDispatch("decode", gqa,
                      {tensor("query", "query", R), tensor("key_cache", "key_cache_" + L, R),
                       tensor("value_cache", "value_cache_" + L, R), position, tensor("output", "attention", W)},
                      fp32);
        matvec(s.weight_format, "attn_output_weight_" + L, "attention", "projected", H);
        p.AddDispatch("decode", residual_rms,
                      {tensor("hidden", "hidden", R), tensor("residual", "projected", R),
                       tensor("weight", "ffn_norm_" + L, R), tensor("updated", "hidden_after_attention", W),
                       tensor("output", "normalized", W), P::Attribute("epsilon", eps)},
                      fp32);
        matvec(s.weight_format, "ffn_up_weight_" + L, "normalized", "gate_up", H);
        p.AddDispatch("decode", swiglu, {tensor("gate_up", "gate_up", R), tensor("output", "activated", W)}, fp32);
        matvec(s.weight_format, "ffn_down_weight_" + L, "activated", "down", F);
        const std::string next_norm = l + 1 < s.layers ? "attn_norm_" + std::to_string(l + 1) : "output_norm";
        p.AddDispatch("decode", residual_rms,
                      {tensor("hidden", "hidden_after_attention", R), tensor("residual", "down", R),
                       tensor("weight", next_norm, R), tensor("updated", "hidden", W), tensor("output", "normalized", W),
                       P::Attribute("epsilon", eps)},
                      fp32);
    }
    matvec(s.head_format, s.tied ? "token_embedding" : "output_weight", "normalized", "logits", H);
    p.AddDispatch("decode", argmax, {tensor("input", "logits", R), tensor("output", "next_token", W)}, fp32);
    if (s.prompt_rows > 0)
        AddPhi4Prefill(p, s, registry, tensor, matvec);
    return p;
}

}  // namespace sharpinference
