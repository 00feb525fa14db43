// Host side of the HIP backend: instruction contract, registry, the HIP
// quantized instruction collection, and the VM program executor, over the
// C ABI of libsharpinference_hip.  See si_host.hpp for the mapping to the
// reference's managed types.
#include "si_host.hpp"

#include <algorithm>
#include <set>
#include <sstream>

namespace sharpinference {

namespace {

std::string TypeName(GraphElementType t)
{
    switch (t) {
    case GraphElementType::Byte: return "Byte";
    case GraphElementType::Int32: return "Int32";
    case GraphElementType::UInt32: return "UInt32";
    case GraphElementType::Float16: return "Float16";
    case GraphElementType::Float32: return "Float32";
    }
    return "?";
}

bool Blank(const std::string& s)
{
    return std::all_of(s.begin(), s.end(), [](char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r'; });
}

const InstructionParameter* Find(const std::vector<InstructionParameter>& parameters, const std::string& name)
{
    for (const auto& p : parameters)
        if (p.name == name)
            return &p;
    return nullptr;
}

}  // namespace

InstructionAdaptationException::InstructionAdaptationException(const std::string& collection, const std::string& name,
                                                               const std::string& reason)
    : InvalidOperationException("Instruction '" + collection + "/" + name + "' cannot adapt parameters: " + reason)
{
}

void Check(int status, const si_hip_context* context)
{
    if (status == SI_HIP_OK)
        return;
    const char* m = si_hip_last_error(context);
    const std::string message = m ? m : "";
    switch (status) {
    case SI_HIP_ERR_ARGUMENT: throw ArgumentException(message);
    case SI_HIP_ERR_UNSUPPORTED: throw NotSupportedException(message);
    case SI_HIP_ERR_ADAPTATION: throw InvalidOperationException(message);
    case SI_HIP_ERR_OUT_OF_MEMORY: throw OutOfMemoryException(message);
    case SI_HIP_ERR_STATE: throw InvalidOperationException(message);
    case SI_HIP_ERR_FORMAT: throw InvalidDataException(message);
    case SI_HIP_ERR_IO: throw IOException(message);
    default: throw DeviceException(message);
    }
}

int ElementSize(GraphElementType type)
{
    switch (type) {
    case GraphElementType::Byte: return 1;
    case GraphElementType::Int32: return 4;
    case GraphElementType::UInt32: return 4;
    case GraphElementType::Float16: return 2;
    case GraphElementType::Float32: return 4;
    }
    return 0;
}

bool Satisfies(GraphElementType provided, GraphElementType required)
{
    for (GraphElementType t : {provided, required})
        if (t != GraphElementType::Float16 && t != GraphElementType::Float32)
            throw ArgumentException("'" + TypeName(t) + "' is not a supported floating-point precision.");
    return provided == required || (provided == GraphElementType::Float32 && required == GraphElementType::Float16);
}

uint64_t TensorDescriptor::ElementCount() const
{
    uint64_t n = 1;
    for (int64_t d : dimensions)
        n *= static_cast<uint64_t>(d);
    return n;
}

uint64_t TensorDescriptor::ByteLength() const { return ElementCount() * static_cast<uint64_t>(ElementSize(element_type)); }

InstructionParameter InstructionParameter::Tensor(std::string name, TensorDescriptor tensor, GraphResourceAccess access,
                                                  std::string source, uint64_t byte_offset)
{
    InstructionParameter p;
    p.kind = Kind::Tensor;
    p.name = std::move(name);
    p.tensor = std::move(tensor);
    p.access = access;
    p.source = std::move(source);
    p.byte_offset = byte_offset;
    return p;
}

InstructionParameter InstructionParameter::Attribute(std::string name, std::string value)
{
    InstructionParameter p;
    p.kind = Kind::Attribute;
    p.name = std::move(name);
    p.value = std::move(value);
    return p;
}

// ---- Instruction ---------------------------------------------------------------------------

void Instruction::Fail(const std::string& reason) const { throw InstructionAdaptationException(CollectionId(), Name(), reason); }

void Instruction::Invoke(IInstructionRecorder& recorder, const std::vector<InstructionParameter>& parameters,
                         const PrecisionRequirement& precision) const
{
    if (recorder.Target() != Target())
        Fail("requires " + Target().architecture + ", recorder is " + recorder.Target().architecture + ".");
    Adapt(parameters, precision);
    recorder.Record(Generate(parameters));
}

InstructionSignature Instruction::Adapt(const std::vector<InstructionParameter>& parameters,
                                        const PrecisionRequirement& precision) const
{
    InstructionSignature signature = GetSignature(parameters, precision);
    Validate(parameters);
    return signature;
}

InstructionSignature Instruction::GetSignature(const std::vector<InstructionParameter>& parameters,
                                               const PrecisionRequirement& precision) const
{
    std::set<std::string> names;
    for (const auto& p : parameters)
        names.insert(p.name);
    if (names.size() != parameters.size())
        Fail("Invalid or duplicate parameters.");
    std::vector<const InstructionParameter*> tensors;
    std::set<std::string> attributes;
    for (const auto& p : parameters) {
        if (p.kind == InstructionParameter::Kind::Tensor)
            tensors.push_back(&p);
        else
            attributes.insert(p.name);
    }
    std::vector<InstructionSignature> matches;
    for (const auto& sig : Signatures()) {
        if (sig.ports.size() != tensors.size())
            continue;
        if (std::set<std::string>(sig.attributes.begin(), sig.attributes.end()) != attributes)
            continue;
        bool all = true;
        for (const auto& port : sig.ports) {
            bool found = false;
            for (const auto* t : tensors)
                if (t->name == port.name && t->tensor.element_type == port.element_type &&
                    (port.access == GraphResourceAccess::Read || t->access != GraphResourceAccess::Read))
                    found = true;
            all &= found;
        }
        if (all)
            matches.push_back(sig);
    }
    if (matches.empty())
        Fail("No supported parameter signature.");
    std::vector<InstructionSignature> compatible;
    for (const auto& sig : matches)
        if (Satisfies(sig.precision.arithmetic_type, precision.minimum_arithmetic_type) &&
            Satisfies(sig.precision.accumulator_type, precision.minimum_accumulator_type))
            compatible.push_back(sig);
    if (compatible.empty()) {
        std::ostringstream os;
        os << "On " << Target().architecture << ", required arithmetic=" << TypeName(precision.minimum_arithmetic_type)
           << ", accumulator=" << TypeName(precision.minimum_accumulator_type) << "; provided ";
        for (size_t i = 0; i < matches.size(); i++)
            os << (i ? "; " : "") << "arithmetic=" << TypeName(matches[i].precision.arithmetic_type)
               << ", accumulator=" << TypeName(matches[i].precision.accumulator_type);
        os << ".";
        Fail(os.str());
    }
    if (compatible.size() != 1)
        Fail("Ambiguous supported parameter/precision signatures.");
    return compatible[0];
}

// ---- InstructionRegistry -------------------------------------------------------------------

InstructionRegistry::InstructionRegistry(std::vector<std::shared_ptr<const IInstructionCollectionProvider>> providers)
    : providers_(std::move(providers))
{
    for (const auto& p : providers_)
        if (!p)
            throw ArgumentException("IC providers cannot contain null.");
    std::vector<InstructionCollectionDescription> all;
    for (const auto& p : providers_)
        for (const auto& d : p->QueryInstructionCollection())
            all.push_back(d);
    for (size_t i = 0; i < all.size(); i++)
        for (size_t j = i + 1; j < all.size(); j++)
            if (all[i].id == all[j].id && all[i].architecture == all[j].architecture && !(all[i] == all[j]))
                throw InvalidDataException("Conflicting IC descriptions for '" + all[i].id + "'.");
    for (const auto& d : all)
        if (Blank(d.name) || d.tier < 0 || Blank(d.architecture.architecture))
            throw InvalidDataException("IC descriptions require a name and non-negative Tier.");
    for (const auto& d : all)
        if (std::find(collections_.begin(), collections_.end(), d) == collections_.end())
            collections_.push_back(d);
    std::sort(collections_.begin(), collections_.end(), [](const auto& a, const auto& b) {
        return a.id != b.id ? a.id < b.id : a.architecture.architecture < b.architecture.architecture;
    });
}

std::vector<std::shared_ptr<const Instruction>> InstructionRegistry::QueryInstruction(const std::string& collection_id,
                                                                                     const std::string& name) const
{
    if (Blank(name))
        throw ArgumentException("instructionName cannot be empty.");
    const bool installed = std::any_of(collections_.begin(), collections_.end(),
                                       [&](const auto& c) { return c.id == collection_id; });
    if (!installed)
        throw NotSupportedException("Instruction collection '" + collection_id + "' is not installed.");
    std::vector<std::shared_ptr<const Instruction>> values;
    for (const auto& p : providers_) {
        const auto cs = p->QueryInstructionCollection();
        if (std::none_of(cs.begin(), cs.end(), [&](const auto& c) { return c.id == collection_id; }))
            continue;
        for (const auto& v : p->QueryInstruction(collection_id, name))
            values.push_back(v);
    }
    for (const auto& v : values) {
        const bool known = std::any_of(collections_.begin(), collections_.end(), [&](const auto& c) {
            return c.id == collection_id && c.architecture == v->Target();
        });
        if (!v || v->CollectionId() != collection_id || v->Name() != name || !known)
            throw InvalidDataException("Provider returned an instruction with a different identity.");
    }
    for (size_t i = 0; i < values.size(); i++)
        for (size_t j = i + 1; j < values.size(); j++)
            if (values[i]->Target() == values[j]->Target())
                throw InvalidDataException("Ambiguous implementations for '" + collection_id + "/" + name + "'.");
    for (const auto& v : values)
        for (const auto& sig : v->Signatures()) {
            std::set<std::string> ports, attrs(sig.attributes.begin(), sig.attributes.end());
            for (const auto& port : sig.ports) {
                if (Blank(port.name))
                    throw InvalidDataException("Invalid signatures for '" + collection_id + "/" + name + "'.");
                ports.insert(port.name);
            }
            if (ports.size() != sig.ports.size() || attrs.size() != sig.attributes.size())
                throw InvalidDataException("Invalid signatures for '" + collection_id + "/" + name + "'.");
        }
    return values;
}

std::shared_ptr<const Instruction> InstructionRegistry::Resolve(const std::string& collection_id,
                                                                const std::string& name,
                                                                const InstructionTarget& target) const
{
    for (const auto& v : QueryInstruction(collection_id, name))
        if (v->Target() == target)
            return v;
    throw NotSupportedException("No " + target.architecture + " implementation for '" + collection_id + "/" + name +
                                "'.");
}

// ---- the HIP quantized collection ----------------------------------------------------------

int FormatId(const std::string& name)
{
    if (name == "q8_0") return SI_HIP_Q8_0;
    if (name == "q4_0") return SI_HIP_Q4_0;
    if (name == "q4_k") return SI_HIP_Q4_K;
    if (name == "f16") return SI_HIP_F16;
    if (name == "f32") return SI_HIP_F32;
    return -1;
}

namespace {

constexpr KernelPrecisionProfile FP32{GraphElementType::Float32, GraphElementType::Float32};

// format and columns attributes, and the weight row length they imply
struct QuantShape {
    int format;
    int64_t columns;
    uint64_t row_bytes;
};

QuantShape ReadQuantShape(const Instruction& self, const std::vector<InstructionParameter>& parameters)
{
    auto fail = [&](const std::string& why) -> QuantShape {
        throw InstructionAdaptationException(self.CollectionId(), self.Name(), why);
    };
    const auto* f = Find(parameters, "format");
    const auto* c = Find(parameters, "columns");
    const int format = FormatId(f->value);
    if (format < 0)
        return fail("format '" + f->value + "' is not q8_0, q4_0, q4_k, f16 or f32.");
    int64_t columns = 0;
    try {
        size_t used = 0;
        columns = std::stoll(c->value, &used);
        if (used != c->value.size())
            columns = -1;
    } catch (const std::exception&) {
        columns = -1;
    }
    uint64_t row_bytes = 0;
    if (columns < 1 || si_hip_tensor_bytes(format, 1, columns, &row_bytes) != SI_HIP_OK)
        return fail("columns '" + c->value + "' is not a positive whole number of " + f->value + " blocks.");
    return {format, columns, row_bytes};
}

}  // namespace

std::vector<InstructionSignature> QuantizedMatVecInstruction::Signatures() const
{
    std::vector<InstructionSignature> s;
    for (const char* weight : {"weight", "matrix"})
        s.push_back({{{weight, GraphElementType::Byte, GraphResourceAccess::Read},
                      {"input", GraphElementType::Float32, GraphResourceAccess::Read},
                      {"output", GraphElementType::Float32, GraphResourceAccess::Write}},
                     {"format", "columns"},
                     FP32});
    return s;
}

void QuantizedMatVecInstruction::Validate(const std::vector<InstructionParameter>& parameters) const
{
    const QuantShape q = ReadQuantShape(*this, parameters);
    const auto* w = Find(parameters, "weight");
    if (!w)
        w = Find(parameters, "matrix");
    const auto* x = Find(parameters, "input");
    const auto* y = Find(parameters, "output");
    if (w->tensor.dimensions.size() != 2 || w->tensor.dimensions[1] != static_cast<int64_t>(q.row_bytes) ||
        w->tensor.dimensions[0] < 1)
        Fail("the weight must be [rows, " + std::to_string(q.row_bytes) + "] bytes for " +
             std::to_string(q.columns) + " columns.");
    if (x->tensor.ElementCount() != static_cast<uint64_t>(q.columns))
        Fail("input has " + std::to_string(x->tensor.ElementCount()) + " elements, columns is " +
             std::to_string(q.columns) + ".");
    if (y->tensor.ElementCount() != static_cast<uint64_t>(w->tensor.dimensions[0]))
        Fail("output has " + std::to_string(y->tensor.ElementCount()) + " elements for " +
             std::to_string(w->tensor.dimensions[0]) + " weight rows.");
}

InstructionRecording QuantizedMatVecInstruction::Generate(const std::vector<InstructionParameter>& parameters) const
{
    return {"si_hip_gemv", parameters};
}

std::vector<InstructionSignature> QuantizedGatherRowInstruction::Signatures() const
{
    return {{{{"table", GraphElementType::Byte, GraphResourceAccess::Read},
              {"index", GraphElementType::Int32, GraphResourceAccess::Read},
              {"output", GraphElementType::Float32, GraphResourceAccess::Write}},
             {"format", "columns"},
             FP32}};
}

void QuantizedGatherRowInstruction::Validate(const std::vector<InstructionParameter>& parameters) const
{
    const QuantShape q = ReadQuantShape(*this, parameters);
    const auto* t = Find(parameters, "table");
    const auto* i = Find(parameters, "index");
    const auto* y = Find(parameters, "output");
    if (t->tensor.dimensions.size() != 2 || t->tensor.dimensions[1] != static_cast<int64_t>(q.row_bytes) ||
        t->tensor.dimensions[0] < 1)
        Fail("the table must be [rows, " + std::to_string(q.row_bytes) + "] bytes.");
    if (i->tensor.ElementCount() != 1)
        Fail("index must hold one element.");
    if (y->tensor.ElementCount() != static_cast<uint64_t>(q.columns))
        Fail("output must hold the " + std::to_string(q.columns) + " columns of a row.");
}

InstructionRecording QuantizedGatherRowInstruction::Generate(const std::vector<InstructionParameter>& parameters) const
{
    return {"si_hip_gather_row", parameters};
}

std::vector<InstructionSignature> QuantizedBatchMatVecInstruction::Signatures() const
{
    return {{{{"weight", GraphElementType::Byte, GraphResourceAccess::Read},
              {"input", GraphElementType::Float32, GraphResourceAccess::Read},
              {"control", GraphElementType::Int32, GraphResourceAccess::Read},
              {"output", GraphElementType::Float32, GraphResourceAccess::Write}},
             {"format", "columns"},
             FP32}};
}

void QuantizedBatchMatVecInstruction::Validate(const std::vector<InstructionParameter>& parameters) const
{
    const QuantShape q = ReadQuantShape(*this, parameters);
    const auto& w = Find(parameters, "weight")->tensor.dimensions;
    const auto& x = Find(parameters, "input")->tensor.dimensions;
    const auto& y = Find(parameters, "output")->tensor.dimensions;
    if (w.size() != 2 || w[1] != static_cast<int64_t>(q.row_bytes) || w[0] < 1)
        Fail("the weight must be [rows, " + std::to_string(q.row_bytes) + "] bytes for " + std::to_string(q.columns) +
             " columns.");
    if (x.size() != 2 || y.size() != 2 || x[1] != q.columns || y[0] != x[0] || y[1] != w[0] || x[0] < 1)
        Fail("Expected weight [O,I], input [B,I], and output [B,O].");
    if (Find(parameters, "control")->tensor.ElementCount() != 2)
        Fail("'control' must have shape [2].");
}

InstructionRecording QuantizedBatchMatVecInstruction::Generate(const std::vector<InstructionParameter>& parameters) const
{
    return {"si_hip_batch_matvec", parameters};
}

std::vector<InstructionCollectionDescription> HipQuantizedInstructions::QueryInstructionCollection() const
{
    return {{HipInstructionCollectionIds::QuantizedFloat32, "HIP quantized products", 0, InstructionTarget::Hip()}};
}

std::vector<std::shared_ptr<const Instruction>> HipQuantizedInstructions::QueryInstruction(
    const std::string& collection_id, const std::string& name) const
{
    if (collection_id != HipInstructionCollectionIds::QuantizedFloat32)
        return {};
    if (name == "quant.mat-vec")
        return {std::make_shared<QuantizedMatVecInstruction>()};
    if (name == "quant.gather-row")
        return {std::make_shared<QuantizedGatherRowInstruction>()};
    if (name == "quant.batch-mat-vec")
        return {std::make_shared<QuantizedBatchMatVecInstruction>()};
    return {};
}

// ---- HipVmProgram --------------------------------------------------------------------------

namespace {

class EntryRecorder : public IInstructionRecorder {
public:
    InstructionTarget Target() const override { return InstructionTarget::Hip(); }
    void Record(InstructionRecording recording) override { recordings.push_back(std::move(recording)); }
    std::vector<InstructionRecording> recordings;
};

}  // namespace

int HipVmProgram::SlotIndex(const std::string& id) const
{
    for (size_t i = 0; i < slots_.size(); i++)
        if (slots_[i].id == id)
            return static_cast<int>(i);
    return -1;
}

void HipVmProgram::AddSlot(HipVmSlot slot)
{
    if (Blank(slot.id) || SlotIndex(slot.id) >= 0)
        throw InvalidDataException("Empty or duplicate slot '" + slot.id + "'.");
    if (slot.tensor.ByteLength() == 0)
        throw InvalidDataException("Slot '" + slot.id + "' is empty.");
    slots_.push_back(std::move(slot));
}

void HipVmProgram::AddDispatch(const std::string& entry, std::shared_ptr<const Instruction> instruction,
                               const std::vector<InstructionParameter>& parameters,
                               const PrecisionRequirement& precision)
{
    if (!instruction)
        throw ArgumentException("instruction cannot be null.");
    if (Blank(entry))
        throw ArgumentException("entry cannot be empty.");
    std::vector<const InstructionParameter*> tensors;
    for (const auto& p : parameters) {
        if (p.kind != InstructionParameter::Kind::Tensor)
            continue;
        const int s = SlotIndex(p.source);
        if (s < 0)
            throw ArgumentException("Parameter '" + p.name + "' names unknown slot '" + p.source + "'.");
        const uint64_t end = p.byte_offset + p.tensor.ByteLength();
        if (end < p.byte_offset || end > slots_[s].tensor.ByteLength())
            throw InvalidDataException("Parameter '" + p.name + "' does not fit in slot '" + p.source + "'.");
        if (p.access != GraphResourceAccess::Read && slots_[s].access != VmAccess::ReadWrite)
            throw InvalidDataException("Parameter '" + p.name + "' writes read-only slot '" + p.source + "'.");
        tensors.push_back(&p);
    }
    for (size_t i = 0; i < tensors.size(); i++)
        for (size_t j = i + 1; j < tensors.size(); j++) {
            const auto* a = tensors[i];
            const auto* b = tensors[j];
            if (a->source == b->source &&
                (a->access != GraphResourceAccess::Read || b->access != GraphResourceAccess::Read) &&
                a->byte_offset < b->byte_offset + b->tensor.ByteLength() &&
                b->byte_offset < a->byte_offset + a->tensor.ByteLength())
                throw NotSupportedException("Dispatch '" + entry + "' aliases writable kernel parameters.");
        }
    EntryRecorder recorder;
    instruction->Invoke(recorder, parameters, precision);
    const KernelPrecisionProfile resolved = instruction->Adapt(parameters, precision).precision;
    for (auto& r : recorder.recordings)
        entries_[entry].push_back({instruction, std::move(r), precision, resolved, {}});
}

void HipVmProgram::AddKernelDispatch(const std::string& entry, std::shared_ptr<const Instruction> instruction,
                                     const std::vector<InstructionParameter>& parameters,
                                     const PrecisionRequirement& precision, const HipVmKernelLaunch& launch)
{
    auto& ds = entries_[entry];
    const size_t before = ds.size();
    AddDispatch(entry, std::move(instruction), parameters, precision);
    for (size_t i = before; i < ds.size(); i++) {
        HipVmDispatch& d = ds[i];
        if (!launch.implementation_variant.empty()) {
            if (launch.implementation_variant != "any_shape" ||
                (d.recording.operation != "si_hip_gemv" && d.recording.operation != "si_hip_gemv.dense")) {
                ds.resize(before);
                throw NotSupportedException("Instruction '" + d.instruction->Name() + "' has no '" +
                                            launch.implementation_variant + "' implementation.");
            }
            d.recording.operation += ".any_shape";
        }
        d.launch = launch;
    }
}

// ---- HipVmExecutor -------------------------------------------------------------------------

HipVmExecutor::HipVmExecutor(HipVmProgram program, int device) : program_(std::move(program))
{
    Check(si_hip_init(device, &context_));
    try {
        for (const auto& slot : program_.Slots()) {
            void* p = nullptr;
            const uint64_t bytes = slot.tensor.ByteLength();
            Check(si_hip_alloc(context_, bytes < 4 ? 4 : bytes, &p), context_);
            buffers_.push_back(p);
            Check(si_hip_fill_u32(context_, p, 0, (bytes + 3) / 4), context_);
        }
        // the executor's own scratch: argmax partials, attention chunk partials
        uint64_t scratch = 0;
        Check(si_hip_argmax_workspace_bytes(&scratch));
        for (const auto& entry : program_.Entries())
            for (const auto& d : entry.second)
                if (d.recording.operation == "si_hip_grouped_query_attention") {
                    const auto& k = Find(d.recording.parameters, "key_cache")->tensor.dimensions;
                    const int heads = static_cast<int>(Find(d.recording.parameters, "query")->tensor.ElementCount() / k[2]);
                    uint64_t b = 0;
                    Check(si_hip_gqa_workspace_bytes(heads, static_cast<int>(k[2]), static_cast<int>(k[0]), &b));
                    scratch = std::max(scratch, b);
                } else if (d.recording.operation == "si_hip_batch_gqa_values") {
                    const auto& pr = Find(d.recording.parameters, "probabilities")->tensor.dimensions;
                    uint64_t b = 0;
                    Check(si_hip_batch_values_workspace_bytes(static_cast<int>(pr[0]), static_cast<int>(pr[1]),
                                                              static_cast<int>(pr[2]), &b));
                    scratch = std::max(scratch, b);
                }
        Check(si_hip_alloc(context_, scratch, &scratch_), context_);
        Check(si_hip_sync(context_), context_);
    } catch (...) {
        for (void* p : buffers_)
            si_hip_free(context_, p);
        if (scratch_)
            si_hip_free(context_, scratch_);
        si_hip_destroy(context_);
        throw;
    }
}

HipVmExecutor::~HipVmExecutor()
{
    for (auto& kv : plans_)
        si_hip_plan_destroy(kv.second);
    for (void* p : buffers_)
        si_hip_free(context_, p);
    if (scratch_)
        si_hip_free(context_, scratch_);
    si_hip_destroy(context_);
}

void HipVmExecutor::Upload(const std::string& slot, const void* bytes, uint64_t length)
{
    const int s = program_.SlotIndex(slot);
    if (s < 0)
        throw ArgumentException("Unknown slot '" + slot + "'.");
    const uint64_t expected = program_.Slots()[s].tensor.ByteLength();
    if (length != expected)
        throw ArgumentException("Expected " + std::to_string(expected) + " bytes for slot '" + slot + "', received " +
                                std::to_string(length) + ".");
    if (!bytes)
        throw ArgumentException("bytes cannot be null.");
    Check(si_hip_upload(context_, buffers_[s], bytes, length), context_);
}

std::vector<uint8_t> HipVmExecutor::Readback(const std::string& slot)
{
    const int s = program_.SlotIndex(slot);
    if (s < 0)
        throw ArgumentException("Unknown slot '" + slot + "'.");
    std::vector<uint8_t> out(program_.Slots()[s].tensor.ByteLength());
    Check(si_hip_readback(context_, out.data(), buffers_[s], out.size()), context_);
    return out;
}

void* HipVmExecutor::Address(const InstructionParameter& p) const
{
    return static_cast<uint8_t*>(buffers_[program_.SlotIndex(p.source)]) + p.byte_offset;
}

void HipVmExecutor::Launch(const InstructionRecording& r)
{
    const auto attr = [&](const char* n) { return Find(r.parameters, n)->value; };
    const auto F = [&](const InstructionRecording& rec, const char* n) {
        return static_cast<const float*>(Address(*Find(rec.parameters, n)));
    };
    const auto Fw = [&](const InstructionRecording& rec, const char* n) {
        return static_cast<float*>(Address(*Find(rec.parameters, n)));
    };
    const auto I = [&](const InstructionRecording& rec, const char* n) {
        return static_cast<const int32_t*>(Address(*Find(rec.parameters, n)));
    };
    if (LaunchTierZeroOp(context_, r, [&](const InstructionParameter& p) { return Address(p); }))
        return;
    if (r.operation == "si_hip_gemv.any_shape" || r.operation == "si_hip_gemv.dense.any_shape") {
        const auto* w = Find(r.parameters, "weight");
        if (!w)
            w = Find(r.parameters, "matrix");
        const bool quant = r.operation == "si_hip_gemv.any_shape";
        const int fmt = quant ? FormatId(attr("format"))
                        : w->tensor.element_type == GraphElementType::Float16 ? SI_HIP_F16
                                                                              : SI_HIP_F32;
        Check(si_hip_gemv_any_shape(context_, fmt, Address(*w), F(r, "input"), Fw(r, "output"), w->tensor.dimensions[0],
                                    quant ? std::stoll(attr("columns")) : w->tensor.dimensions[1]),
              context_);
    } else if (r.operation == "si_hip_gemv") {
        const auto* w = Find(r.parameters, "weight");
        if (!w)
            w = Find(r.parameters, "matrix");
        const auto* x = Find(r.parameters, "input");
        const auto* y = Find(r.parameters, "output");
        Check(si_hip_gemv(context_, FormatId(attr("format")), Address(*w), static_cast<const float*>(Address(*x)),
                          static_cast<float*>(Address(*y)), w->tensor.dimensions[0], std::stoll(attr("columns")),
                          nullptr, nullptr),
              context_);
    } else if (r.operation == "si_hip_gather_row") {
        const auto* t = Find(r.parameters, "table");
        const auto* i = Find(r.parameters, "index");
        const auto* y = Find(r.parameters, "output");
        Check(si_hip_gather_row(context_, FormatId(attr("format")), Address(*t), t->tensor.dimensions[0],
                                std::stoll(attr("columns")), static_cast<const int32_t*>(Address(*i)),
                                static_cast<float*>(Address(*y))),
              context_);
    } else if (r.operation == "si_hip_gemv.dense") {
        const auto* w = Find(r.parameters, "weight");
        if (!w)
            w = Find(r.parameters, "matrix");
        const int fmt = w->tensor.element_type == GraphElementType::Float16 ? SI_HIP_F16 : SI_HIP_F32;
        Check(si_hip_gemv(context_, fmt, Address(*w), F(r, "input"), Fw(r, "output"), w->tensor.dimensions[0],
                          w->tensor.dimensions[1], nullptr, nullptr),
              context_);
    } else if (r.operation == "si_hip_gather_row.dense") {
        const auto* t = Find(r.parameters, "table");
        const int fmt = t->tensor.element_type == GraphElementType::Float16 ? SI_HIP_F16 : SI_HIP_F32;
        Check(si_hip_gather_row(context_, fmt, Address(*t), t->tensor.dimensions[0], t->tensor.dimensions[1],
                                static_cast<const int32_t*>(Address(*Find(r.parameters, "index"))), Fw(r, "output")),
              context_);
    } else if (r.operation == "si_hip_batched_matvec") {
        const auto& d = Find(r.parameters, "matrix")->tensor.dimensions;
        Check(si_hip_batched_matvec(context_, F(r, "matrix"), F(r, "vector"), Fw(r, "output"), static_cast<int>(d[0]),
                                    static_cast<int>(d[1]), static_cast<int>(d[2])),
              context_);
    } else if (r.operation == "si_hip_rms_norm") {
        Check(si_hip_rms_norm(context_, F(r, "input"), F(r, "weight"), Fw(r, "output"),
                              static_cast<int64_t>(Find(r.parameters, "output")->tensor.ElementCount()),
                              std::stof(attr("epsilon"))),
              context_);
    } else if (r.operation == "si_hip_residual_rms_norm") {
        Check(si_hip_residual_rms_norm(context_, F(r, "hidden"), F(r, "residual"), F(r, "weight"), Fw(r, "updated"),
                                       Fw(r, "output"),
                                       static_cast<int64_t>(Find(r.parameters, "output")->tensor.ElementCount()),
                                       std::stof(attr("epsilon"))),
              context_);
    } else if (r.operation == "si_hip_swiglu") {
        Check(si_hip_swiglu(context_, F(r, "gate_up"), Fw(r, "output"),
                            static_cast<int64_t>(Find(r.parameters, "output")->tensor.ElementCount())),
              context_);
    } else if (r.operation == "si_hip_rope_kv_write") {
        const auto& k = Find(r.parameters, "key_cache")->tensor;
        si_hip_rope_kv_write_args a{};
        a.qkv = F(r, "qkv");
        a.position = static_cast<const int32_t*>(Address(*Find(r.parameters, "position")));
        a.frequencies = F(r, "frequencies");
        a.query = Fw(r, "query");
        a.key_cache = Address(*Find(r.parameters, "key_cache"));
        a.value_cache = Address(*Find(r.parameters, "value_cache"));
        a.cache_format = k.element_type == GraphElementType::Float16 ? SI_HIP_F16 : SI_HIP_F32;
        a.query_size = static_cast<int32_t>(Find(r.parameters, "query")->tensor.ElementCount());
        a.kv_size = static_cast<int32_t>(k.dimensions[1] * k.dimensions[2]);
        a.head_size = std::stoi(attr("head_size"));
        a.rotary_size = std::stoi(attr("rotary_size"));
        a.context = static_cast<int32_t>(k.dimensions[0]);
        a.rope_scale = std::stof(attr("rope_scale"));
        Check(si_hip_rope_kv_write(context_, &a), context_);
    } else if (r.operation == "si_hip_grouped_query_attention") {
        const auto& k = Find(r.parameters, "key_cache")->tensor;
        si_hip_gqa_args a{};
        a.query = F(r, "query");
        a.key_cache = Address(*Find(r.parameters, "key_cache"));
        a.value_cache = Address(*Find(r.parameters, "value_cache"));
        a.position = static_cast<const int32_t*>(Address(*Find(r.parameters, "position")));
        a.output = Fw(r, "output");
        a.cache_format = k.element_type == GraphElementType::Float16 ? SI_HIP_F16 : SI_HIP_F32;
        a.kv_heads = static_cast<int32_t>(k.dimensions[1]);
        a.head_size = static_cast<int32_t>(k.dimensions[2]);
        a.query_heads = static_cast<int32_t>(Find(r.parameters, "query")->tensor.ElementCount() / k.dimensions[2]);
        a.context = static_cast<int32_t>(k.dimensions[0]);
        a.workspace = static_cast<float*>(scratch_);
        Check(si_hip_grouped_query_attention(context_, &a), context_);
    } else if (r.operation == "si_hip_argmax") {
        Check(si_hip_argmax(context_, F(r, "input"),
                            static_cast<int64_t>(Find(r.parameters, "input")->tensor.ElementCount()), scratch_,
                            static_cast<int32_t*>(Address(*Find(r.parameters, "output")))),
              context_);
    } else if (r.operation == "si_hip_batch_gather_rows") {
        const auto& t = Find(r.parameters, "table")->tensor.dimensions;
        Check(si_hip_batch_gather_rows(context_, F(r, "table"), t[0], t[1], I(r, "control"), Fw(r, "output"),
                                       static_cast<int>(Find(r.parameters, "output")->tensor.dimensions[0])),
              context_);
    } else if (r.operation == "si_hip_batch_rms_norm") {
        const auto& d = Find(r.parameters, "input")->tensor.dimensions;
        Check(si_hip_batch_rms_norm(context_, F(r, "input"), F(r, "weight"), I(r, "control"), Fw(r, "output"),
                                    static_cast<int>(d[0]), d[1], std::stof(attr("epsilon"))),
              context_);
    } else if (r.operation == "si_hip_batch_residual_rms_norm") {
        const auto& d = Find(r.parameters, "hidden")->tensor.dimensions;
        Check(si_hip_batch_residual_rms_norm(context_, F(r, "hidden"), F(r, "residual"), F(r, "weight"),
                                             I(r, "control"), Fw(r, "updated"), Fw(r, "output"),
                                             static_cast<int>(d[0]), d[1], std::stof(attr("epsilon"))),
              context_);
    } else if (r.operation == "si_hip_batch_matvec" || r.operation == "si_hip_batch_matvec.dense") {
        const auto* w = Find(r.parameters, "weight");
        const auto& x = Find(r.parameters, "input")->tensor.dimensions;
        const int fmt = r.operation == "si_hip_batch_matvec"
                            ? FormatId(attr("format"))
                            : (w->tensor.element_type == GraphElementType::Float16 ? SI_HIP_F16 : SI_HIP_F32);
        Check(si_hip_batch_matvec(context_, fmt, Address(*w), F(r, "input"), I(r, "control"), Fw(r, "output"),
                                  static_cast<int>(x[0]), w->tensor.dimensions[0], x[1]),
              context_);
    } else if (r.operation == "si_hip_batch_swiglu") {
        const auto& d = Find(r.parameters, "output")->tensor.dimensions;
        Check(si_hip_batch_swiglu(context_, F(r, "gate_up"), I(r, "control"), Fw(r, "output"), static_cast<int>(d[0]),
                                  d[1]),
              context_);
    } else if (r.operation == "si_hip_batch_rope_kv_write") {
        const auto& k = Find(r.parameters, "key_cache")->tensor;
        const auto& q = Find(r.parameters, "query")->tensor.dimensions;
        si_hip_batch_rope_args a{};
        a.qkv = F(r, "qkv");
        a.control = I(r, "control");
        a.frequencies = F(r, "frequencies");
        a.query = Fw(r, "query");
        a.key_cache = Address(*Find(r.parameters, "key_cache"));
        a.value_cache = Address(*Find(r.parameters, "value_cache"));
        a.cache_format = k.element_type == GraphElementType::Float16 ? SI_HIP_F16 : SI_HIP_F32;
        a.batch = static_cast<int32_t>(q[0]);
        a.query_size = static_cast<int32_t>(q[1]);
        a.kv_size = static_cast<int32_t>(k.dimensions[1] * k.dimensions[2]);
        a.head_size = std::stoi(attr("head_size"));
        a.rotary_size = std::stoi(attr("rotary_size"));
        a.context = static_cast<int32_t>(k.dimensions[0]);
        a.rope_scale = std::stof(attr("rope_scale"));
        Check(si_hip_batch_rope_kv_write(context_, &a), context_);
    } else if (r.operation == "si_hip_batch_gqa_scores" || r.operation == "si_hip_batch_gqa_values") {
        const bool values = r.operation == "si_hip_batch_gqa_values";
        const auto& c = Find(r.parameters, values ? "value_cache" : "key_cache")->tensor;
        const auto& sd = Find(r.parameters, values ? "probabilities" : "scores")->tensor.dimensions;
        si_hip_batch_attention_args a{};
        a.query = values ? nullptr : F(r, "query");
        a.probabilities = values ? F(r, "probabilities") : nullptr;
        a.cache = Address(*Find(r.parameters, values ? "value_cache" : "key_cache"));
        a.control = I(r, "control");
        a.output = Fw(r, values ? "output" : "scores");
        a.workspace = values ? static_cast<float*>(scratch_) : nullptr;
        a.cache_format = c.element_type == GraphElementType::Float16 ? SI_HIP_F16 : SI_HIP_F32;
        a.batch = static_cast<int32_t>(sd[0]);
        a.query_heads = static_cast<int32_t>(sd[1]);
        a.kv_heads = static_cast<int32_t>(c.dimensions[1]);
        a.head_size = static_cast<int32_t>(c.dimensions[2]);
        a.context = static_cast<int32_t>(c.dimensions[0]);
        Check(values ? si_hip_batch_gqa_values(context_, &a) : si_hip_batch_gqa_scores(context_, &a), context_);
    } else if (r.operation == "si_hip_batch_causal_softmax") {
        const auto& d = Find(r.parameters, "scores")->tensor.dimensions;
        Check(si_hip_batch_causal_softmax(context_, F(r, "scores"), I(r, "control"), Fw(r, "probabilities"),
                                          static_cast<int>(d[0]), static_cast<int>(d[1]), d[2]),
              context_);
    } else if (r.operation == "si_hip_batch_select_last") {
        const auto& d = Find(r.parameters, "input")->tensor.dimensions;
        Check(si_hip_batch_select_last(context_, F(r, "input"), I(r, "control"), Fw(r, "output"),
                                       static_cast<int>(d[0]), d[1]),
              context_);
    } else {
        throw NotSupportedException("No HIP launch for recording '" + r.operation + "'.");
    }
}

namespace {

bool IsGemv(const std::vector<HipVmDispatch>& ds, size_t k)
{
    return k < ds.size() && (ds[k].recording.operation == "si_hip_gemv" || ds[k].recording.operation == "si_hip_gemv.dense");
}

bool IsOp(const std::vector<HipVmDispatch>& ds, size_t k, const char* op)
{
    return k < ds.size() && ds[k].recording.operation == op;
}

// The same slot bytes (both tensor parameters).
bool SameView(const InstructionParameter* a, const InstructionParameter* b)
{
    return a && b && a->source == b->source && a->byte_offset == b->byte_offset &&
           a->tensor.ByteLength() == b->tensor.ByteLength();
}

// No dispatch after index i reads `slot` before one overwrites it whole:
// its contents after dispatch i are never observed inside the entry and are
// replaced before the entry ends.
bool DeadAfter(const std::vector<HipVmDispatch>& ds, size_t i, const std::string& slot, uint64_t slot_bytes)
{
    for (size_t j = i + 1; j < ds.size(); j++) {
        bool reads = false, overwrites = false;
        for (const auto& p : ds[j].recording.parameters) {
            if (p.kind != InstructionParameter::Kind::Tensor || p.source != slot)
                continue;
            if (p.access != GraphResourceAccess::Write)
                reads = true;
            else if (p.byte_offset == 0 && p.tensor.ByteLength() >= slot_bytes)
                overwrites = true;
        }
        if (reads)
            return false;
        if (overwrites)
            return true;
    }
    return false;
}

// Column count of a mat-vec recording, and whether the fused transforms
// cover it (the tiled kernel's column set, dword-aligned operands).
int64_t GemvColumns(const InstructionRecording& g)
{
    if (g.operation == "si_hip_gemv")
        return std::stoll(Find(g.parameters, "columns")->value);
    const auto* w = Find(g.parameters, "weight");
    if (!w)
        w = Find(g.parameters, "matrix");
    return static_cast<int64_t>(w->tensor.dimensions[1]);
}

bool FusableColumns(const InstructionRecording& g)
{
    const int64_t c = GemvColumns(g);
    return c == 1024 || c == 2048 || c == 3072 || c == 4096 || c == 6144 || c == 8192;
}

bool Aligned16(const InstructionParameter* p) { return p && p->byte_offset % 16 == 0; }

}  // namespace

void HipVmExecutor::LaunchGemvFused(const InstructionRecording& g, const void* x, void* y, const void* residual,
                                    int xform, const void* norm_weight, float eps)
{
    const auto* w = Find(g.parameters, "weight");
    if (!w)
        w = Find(g.parameters, "matrix");
    const int fmt = g.operation == "si_hip_gemv" ? FormatId(Find(g.parameters, "format")->value)
                    : w->tensor.element_type == GraphElementType::Float16 ? SI_HIP_F16
                                                                          : SI_HIP_F32;
    Check(si_hip_gemv_fused(context_, fmt, Address(*w), static_cast<const float*>(x), static_cast<float*>(y),
                            static_cast<int64_t>(w->tensor.dimensions[0]), GemvColumns(g),
                            static_cast<const float*>(residual), xform, static_cast<const float*>(norm_weight), eps,
                            nullptr),
          context_);
}

void HipVmExecutor::LaunchBatchAttentionFused(const InstructionRecording& sr, const InstructionRecording& vr)
{
    const auto& k = Find(sr.parameters, "key_cache")->tensor;
    const auto& sd = Find(sr.parameters, "scores")->tensor.dimensions;
    si_hip_batch_attention_args a{};
    a.query = static_cast<const float*>(Address(*Find(sr.parameters, "query")));
    a.cache = Address(*Find(sr.parameters, "key_cache"));
    a.control = static_cast<const int32_t*>(Address(*Find(sr.parameters, "control")));
    a.output = static_cast<float*>(Address(*Find(vr.parameters, "output")));
    a.workspace = static_cast<float*>(scratch_);
    a.cache_format = k.element_type == GraphElementType::Float16 ? SI_HIP_F16 : SI_HIP_F32;
    a.batch = static_cast<int32_t>(sd[0]);
    a.query_heads = static_cast<int32_t>(sd[1]);
    a.kv_heads = static_cast<int32_t>(k.dimensions[1]);
    a.head_size = static_cast<int32_t>(k.dimensions[2]);
    a.context = static_cast<int32_t>(k.dimensions[0]);
    Check(si_hip_batch_gqa_attention(context_, &a, Address(*Find(vr.parameters, "value_cache"))), context_);
}

size_t HipVmExecutor::FuseAt(const std::vector<HipVmDispatch>& ds, size_t i, bool launch, int* launches)
{
    const auto slot_bytes = [&](const InstructionParameter* p) {
        return program_.Slots()[program_.SlotIndex(p->source)].tensor.ByteLength();
    };
    const auto param = [&](size_t k, const char* n) { return Find(ds[k].recording.parameters, n); };
    *launches = 0;
    // batch gqa-scores -> causal-softmax -> gqa-values, when nothing reads the
    // scores or probabilities afterwards: si_hip_batch_gqa_attention
    if (IsOp(ds, i, "si_hip_batch_gqa_scores") && IsOp(ds, i + 1, "si_hip_batch_causal_softmax") &&
        IsOp(ds, i + 2, "si_hip_batch_gqa_values")) {
        const auto* sc = param(i, "scores");
        const auto* pr = param(i + 1, "probabilities");
        const auto* kc = param(i, "key_cache");
        const auto* vc = param(i + 2, "value_cache");
        if (SameView(sc, param(i + 1, "scores")) && SameView(pr, param(i + 2, "probabilities")) &&
            SameView(param(i, "control"), param(i + 1, "control")) &&
            SameView(param(i, "control"), param(i + 2, "control")) &&
            kc->tensor.element_type == vc->tensor.element_type && kc->tensor.dimensions == vc->tensor.dimensions &&
            sc->tensor.dimensions == pr->tensor.dimensions && DeadAfter(ds, i + 2, sc->source, slot_bytes(sc)) &&
            DeadAfter(ds, i + 2, pr->source, slot_bytes(pr))) {
            if (launch)
                LaunchBatchAttentionFused(ds[i].recording, ds[i + 2].recording);
            *launches = 1;
            return 3;
        }
    }
    // rms-norm -> mat-vec
    if (IsOp(ds, i, "si_hip_rms_norm") && IsGemv(ds, i + 1)) {
        const auto* out = param(i, "output");
        if (SameView(out, param(i + 1, "input")) && DeadAfter(ds, i + 1, out->source, slot_bytes(out)) &&
            FusableColumns(ds[i + 1].recording) && Aligned16(param(i, "input")) && Aligned16(param(i, "weight"))) {
            if (launch)
                LaunchGemvFused(ds[i + 1].recording, Address(*param(i, "input")), Address(*param(i + 1, "output")),
                                nullptr, SI_HIP_X_RMSNORM, Address(*param(i, "weight")),
                                std::stof(param(i, "epsilon")->value));
            *launches = 1;
            return 2;
        }
    }
    // [swiglu ->] mat-vec [-> residual-rms-norm -> mat-vec]
    size_t j = i;
    const InstructionParameter* swiglu_in = nullptr;
    if (IsOp(ds, i, "si_hip_swiglu") && IsGemv(ds, i + 1)) {
        const auto* out = param(i, "output");
        const auto* in = param(i, "gate_up");
        if (SameView(out, param(i + 1, "input")) && DeadAfter(ds, i + 1, out->source, slot_bytes(out)) &&
            FusableColumns(ds[i + 1].recording) && Aligned16(in) &&
            in->tensor.ElementCount() == 2 * static_cast<uint64_t>(GemvColumns(ds[i + 1].recording))) {
            swiglu_in = in;
            j = i + 1;
        }
    }
    if (!IsGemv(ds, j))
        return 0;
    const InstructionParameter* x1 = swiglu_in ? swiglu_in : param(j, "input");
    const int xf1 = swiglu_in ? SI_HIP_X_SWIGLU : SI_HIP_X_PLAIN;
    if (IsOp(ds, j + 1, "si_hip_residual_rms_norm") && IsGemv(ds, j + 2)) {
        const auto* product = param(j, "output");
        const auto* normed = param(j + 1, "output");
        if (SameView(product, param(j + 1, "residual")) && SameView(normed, param(j + 2, "input")) &&
            DeadAfter(ds, j + 1, product->source, slot_bytes(product)) &&
            DeadAfter(ds, j + 2, normed->source, slot_bytes(normed)) && FusableColumns(ds[j + 2].recording) &&
            Aligned16(param(j + 1, "updated")) && Aligned16(param(j + 1, "weight"))) {
            if (launch) {
                // updated = hidden + W1 . x1 (the residual add of the norm, in the product's output)
                LaunchGemvFused(ds[j].recording, Address(*x1), Address(*param(j + 1, "updated")),
                                Address(*param(j + 1, "hidden")), xf1, nullptr, 0.0f);
                LaunchGemvFused(ds[j + 2].recording, Address(*param(j + 1, "updated")),
                                Address(*param(j + 2, "output")), nullptr, SI_HIP_X_RMSNORM,
                                Address(*param(j + 1, "weight")), std::stof(param(j + 1, "epsilon")->value));
            }
            *launches = 2;
            return j + 3 - i;
        }
    }
    if (swiglu_in) {
        if (launch)
            LaunchGemvFused(ds[j].recording, Address(*x1), Address(*param(j, "output")), nullptr, SI_HIP_X_SWIGLU,
                            nullptr, 0.0f);
        *launches = 1;
        return j + 1 - i;
    }
    return 0;
}

void HipVmExecutor::SetDispatchFusion(bool on)
{
    if (on == fuse_)
        return;
    for (auto& kv : plans_)
        si_hip_plan_destroy(kv.second);
    plans_.clear();
    fuse_ = on;
}

int HipVmExecutor::LaunchCount(const std::string& entry)
{
    const auto it = program_.Entries().find(entry);
    if (it == program_.Entries().end())
        throw ArgumentException("Unknown entry '" + entry + "'.");
    const auto& ds = it->second;
    int count = 0;
    for (size_t i = 0; i < ds.size();) {
        int n = 0;
        const size_t used = fuse_ ? FuseAt(ds, i, false, &n) : 0;
        count += used ? n : 1;
        i += used ? used : 1;
    }
    return count;
}

si_hip_plan* HipVmExecutor::PrepareEntry(const std::string& entry)
{
    const auto it = program_.Entries().find(entry);
    if (it == program_.Entries().end())
        throw ArgumentException("Unknown entry '" + entry + "'.");
    const auto cached = plans_.find(entry);
    if (cached != plans_.end())
        return cached->second;
    Check(si_hip_plan_begin(context_), context_);
    try {
        const auto& ds = it->second;
        for (size_t i = 0; i < ds.size();) {
            int n = 0;
            const size_t used = fuse_ ? FuseAt(ds, i, true, &n) : 0;
            if (used == 0)
                Launch(ds[i].recording);
            i += used ? used : 1;
        }
    } catch (...) {
        si_hip_plan* broken = nullptr;
        if (si_hip_plan_end(context_, &broken) == SI_HIP_OK)
            si_hip_plan_destroy(broken);
        throw;
    }
    si_hip_plan* plan = nullptr;
    Check(si_hip_plan_end(context_, &plan), context_);
    plans_[entry] = plan;
    return plan;
}

void HipVmExecutor::Execute(const std::string& entry)
{
    si_hip_plan* plan = PrepareEntry(entry);
    Check(si_hip_plan_launch(plan), context_);
    Check(si_hip_sync(context_), context_);
}

void HipVmExecutor::ExecuteWithTransfers(const std::string& entry, const std::string& upload_slot,
                                         const std::vector<uint8_t>& upload_bytes, const std::string& readback_slot,
                                         std::vector<uint8_t>& readback_bytes)
{
    const int r = program_.SlotIndex(readback_slot);
    if (r < 0)
        throw ArgumentException("Unknown slot '" + readback_slot + "'.");
    if (readback_bytes.size() != program_.Slots()[r].tensor.ByteLength())
        throw ArgumentException("Expected a " + std::to_string(program_.Slots()[r].tensor.ByteLength()) +
                                "-byte readback buffer for slot '" + readback_slot + "'.");
    si_hip_plan* plan = PrepareEntry(entry);
    Upload(upload_slot, upload_bytes);
    Check(si_hip_plan_launch(plan), context_);
    Check(si_hip_readback(context_, readback_bytes.data(), buffers_[r], readback_bytes.size()), context_);
}

double HipVmExecutor::MeasureGpuMicroseconds(const std::string& entry, int repetitions)
{
    if (repetitions < 1 || repetitions > 1024)
        throw ArgumentOutOfRangeException("repetitions");
    si_hip_plan* plan = PrepareEntry(entry);
    double us = 0.0;
    Check(si_hip_plan_measure_us(plan, repetitions, &us), context_);
    return us;
}

}  // namespace sharpinference
