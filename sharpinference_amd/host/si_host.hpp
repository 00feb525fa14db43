// Host side of the HIP backend in C++: the instruction/plugin interface and
// the VM executor of the reference, restated over the C ABI of
// libsharpinference_hip (include/sharpinference_hip.h).
//
// The reference's managed host (C#) declares the operator contract in
// SharpInference.Instructions/InstructionCollection.cs (Instruction,
// signatures, adaptation, the collection registry) and runs VM programs
// through executors such as SharpInference.Backends.D3D12Vm/
// D3D12VmExecutor.cs (slots, Upload / Readback / Execute /
// MeasureGpuMicroseconds).  This header keeps those names, argument
// meanings and failure types, so the parity tests read like the
// reference's own tests:
//
//   .NET exception                   C++ exception here
//   ArgumentException                ArgumentException
//   ArgumentOutOfRangeException      ArgumentOutOfRangeException
//   InvalidOperationException        InvalidOperationException
//   InstructionAdaptationException   InstructionAdaptationException
//   NotSupportedException            NotSupportedException
//   InvalidDataException             InvalidDataException
//
// The HIP target records launch descriptors instead of shader source: an
// InstructionRecording names the C ABI operation and carries the adapted
// parameters, and the executor turns each recording into one library call
// inside a recorded plan.
#pragma once

#include "sharpinference_hip.h"

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace sharpinference {

// ---- .NET exception types --------------------------------------------------------------

struct ArgumentException : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};
struct ArgumentOutOfRangeException : ArgumentException {
    using ArgumentException::ArgumentException;
};
struct InvalidOperationException : std::logic_error {
    using std::logic_error::logic_error;
};
struct NotSupportedException : std::logic_error {
    using std::logic_error::logic_error;
};
struct InvalidDataException : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct OutOfMemoryException : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct IOException : std::runtime_error {
    using std::runtime_error::runtime_error;
};
// A HIP runtime failure (SI_HIP_ERR_DEVICE).
struct DeviceException : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// Instruction '{collection}/{name}' cannot adapt parameters: {reason}
// (InstructionCollection.cs:155-159).
struct InstructionAdaptationException : InvalidOperationException {
    InstructionAdaptationException(const std::string& collection, const std::string& name, const std::string& reason);
};

// Throws the exception that corresponds to a library status (no-op for OK).
void Check(int status, const si_hip_context* context = nullptr);

// ---- operator contract (InstructionCollection.cs) ----------------------------------------

// GraphModel.cs:63-77 (same members, same order).
enum class GraphElementType { Byte, Int32, UInt32, Float16, Float32 };
enum class GraphResourceAccess { Read, Write, ReadWrite };
// Access of a program slot (VmProgram.cs:10).
enum class VmAccess { ReadOnly, ReadWrite };

int ElementSize(GraphElementType type);
// Precision check (NumericTypeCompatibility.Satisfies, OperatorBackend.cs:106-112):
// equal types, or Float32 where Float16 is required; a type other than
// Float16 / Float32 is an ArgumentException.
bool Satisfies(GraphElementType provided, GraphElementType required);

struct InstructionTarget {
    std::string architecture;
    bool operator==(const InstructionTarget& o) const { return architecture == o.architecture; }
    bool operator!=(const InstructionTarget& o) const { return !(*this == o); }
    static InstructionTarget Hip() { return {"hip.gfx950"}; }
};

struct InstructionCollectionDescription {
    std::string id;             // GUID text
    std::string name;
    int tier;
    InstructionTarget architecture;
    bool operator==(const InstructionCollectionDescription& o) const
    {
        return id == o.id && name == o.name && tier == o.tier && architecture == o.architecture;
    }
};

struct InstructionPort {
    std::string name;
    GraphElementType element_type;
    GraphResourceAccess access;
};

struct KernelPrecisionProfile {
    GraphElementType arithmetic_type;
    GraphElementType accumulator_type;
};

struct PrecisionRequirement {
    GraphElementType minimum_arithmetic_type;
    GraphElementType minimum_accumulator_type;
};

struct InstructionSignature {
    std::vector<InstructionPort> ports;
    std::vector<std::string> attributes;
    KernelPrecisionProfile precision;
};

struct TensorDescriptor {
    GraphElementType element_type = GraphElementType::Float32;
    std::vector<int64_t> dimensions;
    uint64_t ElementCount() const;
    uint64_t ByteLength() const;
};

// InstructionTensorParameter / InstructionAttributeParameter in one value.
struct InstructionParameter {
    enum class Kind { Tensor, Attribute } kind = Kind::Tensor;
    std::string name;
    TensorDescriptor tensor;                    // Tensor
    GraphResourceAccess access = GraphResourceAccess::Read;
    std::string source;                         // Tensor: the slot it is bound to
    uint64_t byte_offset = 0;                   // Tensor: offset inside the slot
    std::string value;                          // Attribute

    static InstructionParameter Tensor(std::string name, TensorDescriptor tensor, GraphResourceAccess access,
                                       std::string source, uint64_t byte_offset = 0);
    static InstructionParameter Attribute(std::string name, std::string value);
};

// The HIP target's recording: the C ABI operation to launch and the
// adapted parameters it binds.
struct InstructionRecording {
    std::string operation;
    std::vector<InstructionParameter> parameters;
};

class IInstructionRecorder {
public:
    virtual ~IInstructionRecorder() = default;
    virtual InstructionTarget Target() const = 0;
    virtual void Record(InstructionRecording recording) = 0;
};

class Instruction {
public:
    virtual ~Instruction() = default;
    virtual std::string CollectionId() const = 0;
    virtual std::string Name() const = 0;
    virtual InstructionTarget Target() const = 0;
    virtual std::vector<InstructionSignature> Signatures() const = 0;

    // Adapt, then record (Instruction.Invoke, InstructionCollection.cs:114-122).
    void Invoke(IInstructionRecorder& recorder, const std::vector<InstructionParameter>& parameters,
                const PrecisionRequirement& precision) const;
    // The one signature the parameters match, after Validate (:124-130).
    InstructionSignature Adapt(const std::vector<InstructionParameter>& parameters,
                               const PrecisionRequirement& precision) const;
    // Signature selection (:143-172): unique names, ports matched by name,
    // element type and access, attribute set equality, precision.
    InstructionSignature GetSignature(const std::vector<InstructionParameter>& parameters,
                                      const PrecisionRequirement& precision) const;

protected:
    virtual void Validate(const std::vector<InstructionParameter>&) const {}
    virtual InstructionRecording Generate(const std::vector<InstructionParameter>& parameters) const = 0;
    [[noreturn]] void Fail(const std::string& reason) const;
};

class IInstructionCollectionProvider {
public:
    virtual ~IInstructionCollectionProvider() = default;
    virtual std::vector<InstructionCollectionDescription> QueryInstructionCollection() const = 0;
    virtual std::vector<std::shared_ptr<const Instruction>> QueryInstruction(const std::string& collection_id,
                                                                            const std::string& name) const = 0;
};

// InstructionRegistry (InstructionCollection.cs:161-230).
class InstructionRegistry : public IInstructionCollectionProvider {
public:
    explicit InstructionRegistry(std::vector<std::shared_ptr<const IInstructionCollectionProvider>> providers);
    std::vector<InstructionCollectionDescription> QueryInstructionCollection() const override { return collections_; }
    std::vector<std::shared_ptr<const Instruction>> QueryInstruction(const std::string& collection_id,
                                                                    const std::string& name) const override;
    std::shared_ptr<const Instruction> Resolve(const std::string& collection_id, const std::string& name,
                                               const InstructionTarget& target) const;

private:
    std::vector<std::shared_ptr<const IInstructionCollectionProvider>> providers_;
    std::vector<InstructionCollectionDescription> collections_;
};

// ---- the HIP quantized instruction collection -------------------------------------------

namespace HipInstructionCollectionIds {
// New collection: block-quantized matrix-vector products (the T0 mat-vec
// rejects attributes and non-dense weights, TierZeroOperationContracts.cs:70-91,161).
inline const std::string QuantizedFloat32 = "5c2f7b1e-9a4d-4f0e-8e61-3b7f2d9c4a10";
}

// quant.mat-vec: output[rows] = weight[rows, columns] . input[columns]; the
// weight port is a Byte tensor [rows, row_bytes] of GGUF blocks, attributes
// format (q8_0 | q4_0 | q4_k) and columns; port names as core.mat-vec
// (weight or matrix, input, output); FP32 arithmetic and accumulation.
class QuantizedMatVecInstruction : public Instruction {
public:
    std::string CollectionId() const override { return HipInstructionCollectionIds::QuantizedFloat32; }
    std::string Name() const override { return "quant.mat-vec"; }
    InstructionTarget Target() const override { return InstructionTarget::Hip(); }
    std::vector<InstructionSignature> Signatures() const override;

protected:
    void Validate(const std::vector<InstructionParameter>& parameters) const override;
    InstructionRecording Generate(const std::vector<InstructionParameter>& parameters) const override;
};

// quant.gather-row: output[columns] = row index[0] of table[rows, columns]
// (GpuTierZeroInstruction.cs:397-405 for a quantized table); NaN for an index
// outside the table.
class QuantizedGatherRowInstruction : public Instruction {
public:
    std::string CollectionId() const override { return HipInstructionCollectionIds::QuantizedFloat32; }
    std::string Name() const override { return "quant.gather-row"; }
    InstructionTarget Target() const override { return InstructionTarget::Hip(); }
    std::vector<InstructionSignature> Signatures() const override;

protected:
    void Validate(const std::vector<InstructionParameter>& parameters) const override;
    InstructionRecording Generate(const std::vector<InstructionParameter>& parameters) const override;
};

// quant.batch-mat-vec: output[b] = weight . input[b] for the live rows of
// control {start, valid} (transformer.batch-shared-matvec,
// GpuBatchTransformerInstructions.cs:224-279, over GGUF block rows): weight
// Byte [rows, row_bytes], input Float32 [batch, columns], control Int32 [2],
// output Float32 [batch, rows]; attributes format and columns.
class QuantizedBatchMatVecInstruction : public Instruction {
public:
    std::string CollectionId() const override { return HipInstructionCollectionIds::QuantizedFloat32; }
    std::string Name() const override { return "quant.batch-mat-vec"; }
    InstructionTarget Target() const override { return InstructionTarget::Hip(); }
    std::vector<InstructionSignature> Signatures() const override;

protected:
    void Validate(const std::vector<InstructionParameter>& parameters) const override;
    InstructionRecording Generate(const std::vector<InstructionParameter>& parameters) const override;
};

class HipQuantizedInstructions : public IInstructionCollectionProvider {
public:
    std::vector<InstructionCollectionDescription> QueryInstructionCollection() const override;
    std::vector<std::shared_ptr<const Instruction>> QueryInstruction(const std::string& collection_id,
                                                                    const std::string& name) const override;
};

// GGUF format name of the quant attribute -> GGUF type id (-1 if unknown).
int FormatId(const std::string& name);

// ---- the reference's collections on the HIP target ----------------------------------------

namespace InstructionCollectionIds {
// The reference's collection GUIDs (InstructionCollection.cs:6-12): the HIP
// target implements instructions of these collections under the same
// identity, so a program names them exactly as it does for D3D12.
inline const std::string TierZeroFloat32 = "00000000-0000-0000-0000-000000000000";
inline const std::string TransformerFloat32 = "824d0f9c-16c7-46d8-b49d-0f91d6a4ec83";
}  // namespace InstructionCollectionIds

// An instruction of one fixed identity whose signatures are given as port
// lists (FP32 arithmetic and accumulation, one attribute set); Validate and
// Generate come from the concrete instruction.
class HipFixedInstruction : public Instruction {
public:
    HipFixedInstruction(std::string collection, std::string name, std::vector<std::vector<InstructionPort>> signatures,
                        std::vector<std::string> attributes);
    std::string CollectionId() const override { return collection_; }
    std::string Name() const override { return name_; }
    InstructionTarget Target() const override { return InstructionTarget::Hip(); }
    std::vector<InstructionSignature> Signatures() const override;

protected:
    const InstructionParameter& TensorOf(const std::vector<InstructionParameter>& parameters,
                                         const std::string& name) const;
    // Attribute parsers with the reference's rules (PositiveInteger: digits
    // only and > 0; PositiveFloat: finite and > 0; GpuTransformerInstructionCollection.cs:300-311,530-540).
    int PositiveInteger(const std::vector<InstructionParameter>& parameters, const std::string& name) const;
    float PositiveFloat(const std::vector<InstructionParameter>& parameters, const std::string& name) const;

private:
    std::string collection_, name_;
    std::vector<std::vector<InstructionPort>> signatures_;
    std::vector<std::string> attributes_;
};

// T0 core.mat-vec on HIP: matrix|weight [rows, columns] Float32 or Float16,
// input Float32 [columns], output Float32 [rows] (TierZeroOperationContracts.cs:113-115,152,161;
// TierZeroInstruction.cs:100-106 adds the weight alias).
class TierZeroMatVecInstruction : public HipFixedInstruction {
public:
    TierZeroMatVecInstruction();

protected:
    void Validate(const std::vector<InstructionParameter>& parameters) const override;
    InstructionRecording Generate(const std::vector<InstructionParameter>& parameters) const override;
};

// T0 core.gather-row: table [rows, columns] Float32 or Float16, index Int32
// [1], output Float32 [columns] (TierZeroOperationContracts.cs:132-134,151,159).
class TierZeroGatherRowInstruction : public HipFixedInstruction {
public:
    TierZeroGatherRowInstruction();

protected:
    void Validate(const std::vector<InstructionParameter>& parameters) const override;
    InstructionRecording Generate(const std::vector<InstructionParameter>& parameters) const override;
};

// T0 core.tensor.batched-mat-vec: matrix [B, R, C], vector [B, C] -> output
// [B, R], Float32 (PortableTensorOperationContracts.cs:61-62,74-75).
class TierZeroBatchedMatVecInstruction : public HipFixedInstruction {
public:
    TierZeroBatchedMatVecInstruction();

protected:
    void Validate(const std::vector<InstructionParameter>& parameters) const override;
    InstructionRecording Generate(const std::vector<InstructionParameter>& parameters) const override;
};

class HipTierZeroInstructions : public IInstructionCollectionProvider {
public:
    std::vector<InstructionCollectionDescription> QueryInstructionCollection() const override;
    std::vector<std::shared_ptr<const Instruction>> QueryInstruction(const std::string& collection_id,
                                                                    const std::string& name) const override;
};

// The transformer collection (GpuTransformerInstructionCollection.cs:11-33)
// on HIP: transformer.rms-norm, residual-rms-norm, swiglu, rope-kv-write,
// grouped-query-attention and argmax, with the reference's port names,
// accesses and attributes.  rope-kv-write and grouped-query-attention take
// Float32 caches (the reference's signature) or Float16 caches (a second
// signature of this target).
class HipTransformerInstructions : public IInstructionCollectionProvider {
public:
    std::vector<InstructionCollectionDescription> QueryInstructionCollection() const override;
    std::vector<std::shared_ptr<const Instruction>> QueryInstruction(const std::string& collection_id,
                                                                    const std::string& name) const override;
};

// Every HIP collection of this library behind one registry.
std::shared_ptr<const InstructionRegistry> DefaultHipRegistry();

// The other T0 operators of the TierZeroFloat32 collection on HIP (copy,
// add, subtract, multiply, divide, maximum, exp, tanh, sigmoid, rsqrt,
// square, relu, reduce-sum, reduce-mean and the core.tensor fill,
// cast-f16-f32, reshape, slice, broadcast, reduce-last-sum / -mean,
// head-outer; TierZeroOperationContracts.cs, PortableTensorOperationContracts.cs),
// or null for another name.
std::shared_ptr<const Instruction> MakeTierZeroOpInstruction(const std::string& name);
// Launches a recording of one of those operators (si_hip_t0_*) with the
// parameters' device addresses; false when the recording is not one.
bool LaunchTierZeroOp(si_hip_context* ctx, const InstructionRecording& recording,
                      const std::function<void*(const InstructionParameter&)>& address);

// ---- program and executor (VmProgram, D3D12VmExecutor) ------------------------------------

// VmSlotScope (VmProgram.cs:9): model-lifetime, session-lifetime (KV
// caches) or per-invocation slots.
enum class VmSlotScope { Global, Session, Local };

struct HipVmSlot {
    std::string id;
    TensorDescriptor tensor;
    VmAccess access = VmAccess::ReadWrite;
    VmSlotScope scope = VmSlotScope::Global;
    std::string binding_key = {};   // empty: none
};

// A lowered program's dispatch (VmDispatch, VmProgram.cs): the kernel
// definition it instantiates (one per distinct operator), its thread group
// and grid, and an implementation variant of the instruction
// ("any_shape": a mat-vec pinned to the serial any-shape kernel).  A
// program built dispatch by dispatch leaves `definition` empty and its
// operators are written inline.  The grid is the program's record of the
// dispatch (the reference's formula); the HIP library sizes each launch
// itself from the operands.
struct HipVmKernelLaunch {
    std::string definition;
    uint32_t threads = 0;
    uint32_t groups[3] = {1, 1, 1};
    std::string implementation_variant;
};

struct HipVmDispatch {
    std::shared_ptr<const Instruction> instruction;
    InstructionRecording recording;
    PrecisionRequirement precision{GraphElementType::Float32, GraphElementType::Float32};
    KernelPrecisionProfile resolved{GraphElementType::Float32, GraphElementType::Float32};   // the adapted signature's
    HipVmKernelLaunch launch;
};

// VmStateEntry (VmProgram.cs:46): a named piece of session state and its slot.
struct HipVmStateEntry {
    std::string name;
    std::string slot;
};

// Slots and named entries; each entry is a list of dispatches separated by
// barriers (every dispatch here is followed by one, as in the reference's
// generated schedules).
class HipVmProgram {
public:
    void AddSlot(HipVmSlot slot);
    // Invokes the instruction on the entry's recorder.  Binding rules
    // (D3D12VmSchedule.cs:74-99): every tensor names an existing slot and
    // fits inside it at its byte offset; a parameter that writes (Write or
    // ReadWrite) needs a ReadWrite slot; writing parameters of one dispatch
    // may not overlap others (NotSupportedException).
    void AddDispatch(const std::string& entry, std::shared_ptr<const Instruction> instruction,
                     const std::vector<InstructionParameter>& parameters, const PrecisionRequirement& precision);
    // AddDispatch for a lowered program: the dispatch also records its
    // kernel definition and grid, and an implementation variant replaces the
    // recording's C ABI operation ("any_shape" on a mat-vec: the serial
    // any-shape kernel); another variant raises NotSupportedException.
    void AddKernelDispatch(const std::string& entry, std::shared_ptr<const Instruction> instruction,
                           const std::vector<InstructionParameter>& parameters, const PrecisionRequirement& precision,
                           const HipVmKernelLaunch& launch);

    const std::vector<HipVmSlot>& Slots() const { return slots_; }
    const std::map<std::string, std::vector<HipVmDispatch>>& Entries() const { return entries_; }
    int SlotIndex(const std::string& id) const;   // -1 if absent

    // Program identity and session state (VmProgram name / abi / state).
    std::string name = "hip-program", abi = "hip.fp32";
    std::string state_schema = "none";
    int state_version = 1;
    std::vector<HipVmStateEntry> state;

private:
    std::vector<HipVmSlot> slots_;
    std::map<std::string, std::vector<HipVmDispatch>> entries_;
};

// ---- VmProgram XML and artifacts (VmProgramXml.cs, D3D12VmArtifact.cs) ----------------------

// The reference's VmProgram XML (VmProgramXml.cs:13-41) with target "Hip":
// slots as written; each entry as an Orchestration definition whose
// parameters are the entry's distinct slot views (the whole slot by its id,
// a narrower view such as control's position word by its port name), an
// Operator node per dispatch (collection GUID, name, arguments, precision,
// resolved precision, execution configuration hip.gfx950 / its C ABI
// operation, sorted attributes and port accesses) followed by a Barrier
// node over the parameters it writes, and an Entry binding each parameter to
// its slot and byte offset.
std::string SerializeVmProgram(const HipVmProgram& program);
// The inverse, with the reference's reader rules (VmProgramXml.cs:43-107,
// 236-296): no DTD, comments and processing instructions ignored, at most
// 16 Mi characters, 100000 elements and nesting 64, only the schema's
// elements and attributes, no text content, enums by exact name.  Every
// operator is resolved on the HIP target through `registry` and re-adapted
// by AddDispatch.  Malformed input raises InvalidDataException.
HipVmProgram DeserializeVmProgram(const std::string& xml,
                                  const std::shared_ptr<const InstructionRegistry>& registry = nullptr);

// HIP program artifact (D3D12VmArtifact.cs:90-148 for this target): a ZIP
// holding program.xml and manifest.json = {"Manifest": <manifest JSON>,
// "Sha256": <its hash>}, the manifest naming the format version, the
// backend ABI (HipVmArtifactAbi), the target "hip.gfx950", the C ABI
// version of libsharpinference_hip it was exported against and program.xml's
// SHA-256.  Kernels are the library's code objects, so the archive holds no
// kernel modules.  Import checks sizes, entry names, both hashes, version,
// ABI, target and library ABI, then deserializes the program.  Hashes detect
// corruption; they are not a signature.
inline const std::string HipVmArtifactAbi = "SharpInference.HipVm.c-abi-launch.ic-precision.v1";
std::vector<uint8_t> ExportHipVmArtifact(const HipVmProgram& program);
HipVmProgram ImportHipVmArtifact(const std::vector<uint8_t>& archive,
                                 const std::shared_ptr<const InstructionRegistry>& registry = nullptr);
// SHA-256 of bytes as 64 upper-case hex digits (Convert.ToHexString(SHA256.HashData)).
std::string Sha256Hex(const void* data, size_t length);

// The executor of a HipVmProgram on one device (D3D12VmExecutor.cs): one
// persistent device buffer per slot, exact-size uploads, entries recorded
// once into plans and replayed with one submission.
//
// Dispatch fusion (on unless switched off): when an entry is recorded, a
// mat-vec whose input comes from the dispatch just before it takes that
// dispatch's work into its own launch, as the reference's graph optimizer
// elides a cast its consumer can absorb (VmGraphOptimizer.cs:198-299):
//   rms-norm -> mat-vec            : one mat-vec with the RMSNorm fused in;
//   swiglu -> mat-vec              : one mat-vec with SwiGLU fused in;
//   mat-vec -> residual-rms-norm -> mat-vec : the first mat-vec adds the
//                                    residual into the updated hidden state,
//                                    the second fuses the RMSNorm.
// Only when every intermediate the fused launches no longer write (the
// normalised vector, the SwiGLU output, the first product) is overwritten
// later in the entry before anything reads it, so no dispatch of the entry
// and no read-back after it observes a difference beyond FP32 rounding (the
// fused RMSNorm scales each row's sum instead of each input).
class HipVmExecutor {
public:
    explicit HipVmExecutor(HipVmProgram program, int device = 0);
    ~HipVmExecutor();
    HipVmExecutor(const HipVmExecutor&) = delete;
    HipVmExecutor& operator=(const HipVmExecutor&) = delete;

    const HipVmProgram& Program() const { return program_; }
    void Upload(const std::string& slot, const void* bytes, uint64_t length);
    void Upload(const std::string& slot, const std::vector<uint8_t>& bytes) { Upload(slot, bytes.data(), bytes.size()); }
    std::vector<uint8_t> Readback(const std::string& slot);
    void Execute(const std::string& entry);
    // Uploads one control slot, replays the entry, reads one result slot
    // (D3D12VmExecutor.cs:298).
    void ExecuteWithTransfers(const std::string& entry, const std::string& upload_slot,
                              const std::vector<uint8_t>& upload_bytes, const std::string& readback_slot,
                              std::vector<uint8_t>& readback_bytes);
    // GPU microseconds per replay over `repetitions` (1..1024) back-to-back
    // replays (D3D12VmExecutor.cs:452-478).
    double MeasureGpuMicroseconds(const std::string& entry, int repetitions = 8);
    // Switches dispatch fusion (recorded plans are dropped and re-recorded).
    void SetDispatchFusion(bool on);
    bool DispatchFusion() const { return fuse_; }
    // Launches one recording of `entry` makes with the current fusion setting.
    int LaunchCount(const std::string& entry);

private:
    si_hip_plan* PrepareEntry(const std::string& entry);
    void Launch(const InstructionRecording& recording);
    void* Address(const InstructionParameter& parameter) const;
    // The fused group starting at dispatch i: its dispatch count (0: none),
    // and, when `launch`, the launches it makes (their count in *launches).
    size_t FuseAt(const std::vector<HipVmDispatch>& ds, size_t i, bool launch, int* launches);
    void LaunchGemvFused(const InstructionRecording& gemv, const void* x, void* y, const void* residual, int xform,
                         const void* norm_weight, float eps);
    void LaunchBatchAttentionFused(const InstructionRecording& scores, const InstructionRecording& values);
    bool fuse_ = true;

    HipVmProgram program_;
    si_hip_context* context_ = nullptr;
    std::vector<void*> buffers_;
    void* scratch_ = nullptr;   // the executor's own device scratch (argmax partials)
    std::map<std::string, si_hip_plan*> plans_;
};

// ---- the Phi-4 decode program, dispatch by dispatch --------------------------------------

// Shapes and storage of a Phi-4 decode program.  Formats are GGUF type ids
// (Q8_0 / Q4_0 / Q4_K weights are Byte rows dispatched to quant.mat-vec,
// F16 / F32 weights typed tensors dispatched to core.mat-vec); the cache is
// Float32 (the reference's) or Float16.
struct Phi4ProgramShape {
    int layers = 32, hidden = 3072, heads = 24, kv_heads = 8, head_dim = 128, rotary_dim = 96, ffn = 8192;
    int vocab = 200064, context = 4096;
    int weight_format = SI_HIP_Q4_K, embed_format = SI_HIP_Q8_0, head_format = SI_HIP_Q8_0;
    bool tied = false;        // project onto token_embedding (the reference model) instead of output_weight
    GraphElementType cache_type = GraphElementType::Float16;
    float rms_eps = 1e-5f, rope_base = 10000.0f, rope_scale = 1.0f;
    int prompt_rows = 0;      // > 0: the prefill entry over fused_embeddings [prompt_rows, hidden]
};

// The decode program of Phi4D3D12TextSession.Build (Phi4D3D12TextSession.cs:
// 391-426, 866-919) as a HipVmProgram: slots token_embedding, output_weight
// (untied), output_norm, rope_frequencies, attn_norm_{l}, ffn_norm_{l},
// qkv_weight_{l}, attn_output_weight_{l}, ffn_up_weight_{l},
// ffn_down_weight_{l}, key_cache_{l}, value_cache_{l}, control ([token,
// position]), hidden, hidden_after_attention, normalized, qkv, query,
// attention, projected, gate_up, activated, down, logits, next_token; entry
// "decode" = embedding gather, rms-norm, per layer qkv mat-vec, rope-kv-write,
// grouped-query-attention, output mat-vec, residual-rms-norm, up mat-vec,
// swiglu, down mat-vec, residual-rms-norm (onto the next layer's attention
// norm, the output norm after the last), then the vocabulary mat-vec and
// argmax: 2 + 9 * layers + 2 dispatches.
//
// With prompt_rows > 0 the program also holds the reference's prefill entry
// "prefill_fused_16" (Phi4D3D12TextSession.cs:428-504, 952-1168): slot
// fused_embeddings [prompt_rows, hidden] (FP32 prompt embeddings), control
// read as [start, valid], batch slots of 16 rows (batch_hidden,
// batch_normalized, batch_qkv, batch_query, batch_scores and
// batch_probabilities [16, heads, context], batch_attention,
// batch_projected, batch_hidden_after_attention, batch_gate_up,
// batch_activated, batch_down, batch_last [hidden]); dispatches = batch
// gather, batch rms-norm, per layer the batched qkv product, batch
// rope-kv-write, gqa-scores, causal-softmax, gqa-values, output product,
// residual-rms-norm, up product, swiglu, down product, residual-rms-norm,
// then batch select-last, the vocabulary mat-vec and argmax: 2 + 11 *
// layers + 3 dispatches.  It writes the same caches as "decode".
HipVmProgram BuildPhi4DecodeProgram(const Phi4ProgramShape& shape);
// rope_frequencies contents: 1 / base^(2i / rotary) for i < rotary / 2
// (Phi4D3D12TextSession.cs:395-397).
std::vector<float> Phi4RopeFrequencies(const Phi4ProgramShape& shape);

}  // namespace sharpinference
