// Logical graphs and their lowering to HIP VM programs.
//
// The reference describes a model step as a LogicalGraph of portable
// operations (SharpInference.Graphs/GraphModel.cs: resources with kind,
// lifetime and tensor; nodes binding ports to resources), validates it
// against the T0 operation contracts (TierZeroOperationContracts.cs,
// PortableTensorOperationContracts.cs) and lowers it to a VmProgram
// (SharpInference.Vm.Optimization/VmGraphOptimizer.cs): weight views and
// cast elision, local storage reuse, one definition per distinct operator,
// one dispatch per node followed by a barrier over what it writes, and the
// GPU mat-vec selection of GpuMatVecOptimization.cs.  This header restates
// that path for the HIP target: the lowered program runs on HipVmExecutor
// operator by operator.
//
// Block-quantized weights (GGUF Q8_0 / Q4_0 / Q4_K) have no element type in
// the reference's graphs, which accept FP16 / FP32 weights only
// (PortableRwkv7GraphProvider.cs:43-44).  Here a quantized tensor is a Byte
// weight resource [rows, row_bytes] in its GGUF block layout, and a
// projection or embedding gather over it is a quant.mat-vec /
// quant.gather-row node (attributes format and columns) of the HIP
// quantized collection; every other node is unchanged.
#pragma once

#include "si_host.hpp"

#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace sharpinference {

// ---- logical graph (GraphModel.cs) -----------------------------------------------------------

// GraphModel.cs:36-61 (same members, same order).
enum class GraphResourceKind { Input, Output, Weight, SessionState, TokenTransient, Temporary, Constant };
enum class GraphResourceLifetime { External, Model, Session, Token, Invocation };
enum class GraphResourceScope { Global, Session, Local };

struct GraphResource {
    std::string id;
    std::string name;
    GraphResourceKind kind = GraphResourceKind::Temporary;
    GraphResourceLifetime lifetime = GraphResourceLifetime::Invocation;
    TensorDescriptor tensor;
    std::string binding_key;   // weights: the model tensor's name
    // GraphResource.Scope (GraphModel.cs:246-254).
    GraphResourceScope Scope() const;
};

struct NodeResourceBinding {
    std::string port;
    std::string resource;
    GraphResourceAccess access = GraphResourceAccess::Read;
};

struct LogicalNode {
    std::string id;
    std::string operation;     // e.g. "core.add", "core.tensor.broadcast", "quant.mat-vec"
    int version = 1;
    std::vector<NodeResourceBinding> resources;
    std::vector<std::string> dependencies;
    std::map<std::string, std::string> attributes;
    PrecisionRequirement requirements{GraphElementType::Float32, GraphElementType::Float32};

    const NodeResourceBinding* Binding(const std::string& port) const;
};

struct GraphStateEntry {
    std::string name;
    std::string resource;
};

struct LogicalGraph {
    // GraphIdentity / GraphModelSignature (the parts a program keeps).
    std::string name;
    std::string architecture;
    std::string state_abi;      // "rwkv-7.state.fp32@1"
    std::string state_schema;   // "RWKV7_State"
    std::vector<GraphResource> resources;
    std::vector<LogicalNode> nodes;
    std::vector<std::string> inputs, outputs;
    std::vector<GraphStateEntry> state;

    const GraphResource& Resource(const std::string& id) const;   // InvalidDataException if absent
    const GraphResource* FindResource(const std::string& id) const;

private:
    mutable std::map<std::string, size_t> index_;   // resource id -> position, extended as resources grow
};

// GraphValidator + TierZeroOperationContracts.ValidateGraph: unique ids,
// every binding names a resource, and each node obeys its operation's
// contract (ports, accesses, attributes, element types, dimensions; no
// write to an input, weight or constant; no output that is also an input).
// Raises InvalidDataException (contract violations) or NotSupportedException
// (an operation or element types outside the contracts).
void ValidateGraph(const LogicalGraph& graph);

// ---- the RWKV-7 forward-token graph (PortableRwkv7GraphProvider.cs) --------------------------

// One tensor of a model's catalog: GGUF type id (SI_HIP_F32, SI_HIP_F16,
// SI_HIP_Q8_0, SI_HIP_Q4_0, SI_HIP_Q4_K) and the catalog's dimensions
// (GGML order: a matrix is [input, output]).
struct ModelTensor {
    int type = SI_HIP_F32;
    std::vector<int64_t> dims;
};

// IModelTensorCatalog (the parts the graph provider reads).
struct ModelTensorCatalog {
    int64_t vocabulary = 0;
    int64_t embedding = 0;
    int64_t layers = 0;
    std::map<std::string, ModelTensor> tensors;
};

// PortableRwkv7GraphProvider.Build (:13-295): the unfused single-token
// graph "rwkv7.forward-token.portable" — token [1] Int32 in, logits
// [vocabulary] out, per layer the session state att-previous, ffn-previous
// and wkv [heads, head, head] — node by node in the reference's order and
// with its node and resource ids ("portable.NNNNN", "weight.<name>",
// "state.<layer>.<suffix>").  Matrices may be FP16 / FP32 (as in the
// reference) or block-quantized (quant.mat-vec / quant.gather-row nodes).
// Catalog errors raise InvalidDataException with the reference's messages.
LogicalGraph BuildRwkv7Graph(const ModelTensorCatalog& tensors);

// ---- GPU mat-vec selection (GpuMatVecOptimization.cs) ----------------------------------------

enum class GpuMatVecMode { Serial, Cooperative, Profile, Default };

// The HIP cooperative (tiled) mat-vec: its identity in cost profiles and its
// workgroup size.
namespace HipMatVecExecution {
inline const std::string ImplementationFingerprint = "hip.gfx950.gemv-tiled@1";
constexpr uint32_t Threads = 256;
}

// One offline measurement (TierOneCostProfile's mat-vec entries).
struct MatVecCostMeasurement {
    std::string operation = "core.mat-vec";
    std::string implementation_fingerprint;
    std::string shape;           // GpuMatVecOptimizationSettings::Shape
    std::string input_aliases = "0,1";
    uint32_t threads_per_group = 0;
    bool reuse_local_storage = true;
    double conservative_saving_microseconds = 0.0;
};

struct MatVecCostProfile {
    std::string environment_fingerprint;
    int64_t measured_at_unix_seconds = 0;
    std::vector<MatVecCostMeasurement> measurements;
};

struct HipVmOptimizationOptions;

class GpuMatVecOptimizationSettings {
public:
    // Profile mode needs a profile and a non-blank current fingerprint; the
    // other modes accept neither (ArgumentException), as :10-19.
    explicit GpuMatVecOptimizationSettings(GpuMatVecMode mode, std::optional<MatVecCostProfile> profile = std::nullopt,
                                           std::optional<std::string> environment_fingerprint = std::nullopt);
    GpuMatVecMode Mode() const { return mode_; }
    // "<matrix dims joined by x>|<matrix type>,<input type>,<output type>" (:26-32).
    static std::string Shape(const std::vector<InstructionParameter>& parameters);
    // (cooperative, diagnostic) for one mat-vec node (:34-59); `now` in Unix seconds.
    std::pair<bool, std::string> Select(const std::vector<InstructionParameter>& parameters,
                                        const HipVmOptimizationOptions& options, int64_t now) const;

private:
    GpuMatVecMode mode_;
    std::optional<MatVecCostProfile> profile_;
    std::optional<std::string> fingerprint_;
};

struct GpuMatVecOptimizationReport {
    int calls = 0;
    int cooperative_calls = 0;
    std::vector<std::string> diagnostics;   // distinct, ordinal order
};

// ---- lowering (VmGraphOptimizer.cs) -------------------------------------------------------------

struct HipVmOptimizationOptions {
    bool reuse_local_storage = true;
    uint32_t threads_per_group = 64;    // 1..1024
    bool native_half_weights = true;    // FP16 weights feed mat-vec / gather-row / batched-mat-vec directly
    bool weight_views = true;           // reshapes (and casts) of weights become views of the weight slot
    std::optional<GpuMatVecOptimizationSettings> gpu_matvec;
    int64_t now_unix_seconds = 0;       // profile freshness; 0: the system clock
};

// One lowered node: its definition, execution configuration and grid.
struct HipVmNodeReport {
    std::string node;
    std::string operation;
    std::string definition;         // "op.NNNN"
    std::string implementation;     // the C ABI operation the executor launches
    uint32_t threads = 0;
    uint32_t groups[3] = {1, 1, 1};
    bool matvec = false;
    bool cooperative = false;
    std::string diagnostic;         // mat-vec nodes: the selection's diagnostic
};

struct HipVmOptimizationResult {
    HipVmProgram program;
    GpuMatVecOptimizationReport matvec;
    std::vector<HipVmNodeReport> nodes;
    int removed_nodes = 0;          // casts and reshapes lowered to views
    int local_slots = 0;
    int definitions = 0;
};

// VmGraphOptimizer.OptimizeWithReport (:17-196) for the HIP target:
// validate; lower weight views (:198-299); plan local storage
// (GraphResourceAllocator.PlanLocal: a local intermediate shares a slot
// with earlier ones of the same type and dimensions whose uses are all
// ordered before its own); one slot per remaining resource; then per node
// one definition per distinct operator key (name, target, threads,
// implementation, precision, parameter types and dimensions, sorted
// attributes), one dispatch of the entry "forward" with its grid and one
// barrier over the slots it writes.  Mat-vec nodes (core.mat-vec and
// quant.mat-vec) take the cooperative tiled kernel or the serial any-shape
// kernel as the settings select (default: cooperative).
HipVmOptimizationResult OptimizeWithReport(const LogicalGraph& graph, const HipVmOptimizationOptions& options = {},
                                           const std::shared_ptr<const InstructionRegistry>& registry = nullptr);

// The report as JSON text: matvec {calls, cooperativeCalls, diagnostics},
// removedNodes, localSlots, definitions and per node {node, operation,
// definition, implementation, threads, groups, cooperative, diagnostic}.
std::string OptimizationReportJson(const HipVmOptimizationResult& result);
// A JSON string literal of `s` (quotes, backslashes and control characters escaped).
std::string JsonString(const std::string& s);

}  // namespace sharpinference
