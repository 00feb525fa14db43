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

HipVmProgram BuildPhi4DecodeProgram(const Phi4ProgramShape& s)
{
    if (s.layers < 1 || s.hidden < 1 || s.heads < 1 || s.kv_heads < 1 || s.heads % s.kv_heads != 0 ||
        s.hidden != s.heads * s.head_dim || s.ffn < 1 || s.vocab < 1 || s.context < 1 || s.rotary_dim < 2 ||
        s.rotary_dim > s.head_dim || s.rotary_dim % 2 != 0)
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
    const auto ro = VmAccess::ReadOnly, rw = VmAccess::ReadWrite;
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
        p.AddSlot({"key_cache_" + L, cache, rw});
        p.AddSlot({"value_cache_" + L, cache, rw});
    }
    p.AddSlot({"control", Vec(2, I32), ro});
    for (const auto& [name, n] : std::vector<std::pair<const char*, int64_t>>{
             {"hidden", H}, {"hidden_after_attention", H}, {"normalized", H}, {"qkv", QKV}, {"query", Q},
             {"attention", H}, {"projected", H}, {"gate_up", 2 * F}, {"activated", F}, {"down", H},
             {"logits", s.vocab}})
        p.AddSlot({name, Vec(n), rw});
    p.AddSlot({"next_token", Vec(1, I32), rw});

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
                            int64_t columns) {
        std::vector<P> args{tensor("weight", weight, R), tensor("input", input, R), tensor("output", output, W)};
        if (Dense(fmt)) {
            p.AddDispatch("decode", t0_mv, args, fp32);
        } else {
            args.push_back(P::Attribute("format", FormatName(fmt)));
            args.push_back(P::Attribute("columns", std::to_string(columns)));
            p.AddDispatch("decode", quant_mv, args, fp32);
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
    return p;
}

}  // namespace sharpinference
