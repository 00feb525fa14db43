// Tests of the C++ host interface (sharpinference_amd/host/si_host.hpp):
// the instruction contract and registry, program binding rules, and the VM
// executor running quantized mat-vec and gather-row programs on the GPU.
//
// Mirrors SharpInference.Tests/GpuMatVecTests.cs for block-quantized
// weights: tails, views with sentinel padding and repeated invocation
// (:13-39, :283-310), non-finite sums (:54-67), compiler rejections
// (:87-114), resident timestamp measurement (:116-127) and span upload
// (:129-142).  Expected values come from the oracle's fp64 product over the
// exactly dequantised weights (test infrastructure, linked only here).
//
//   test_host cpu    contract, registry and binding tests (no device)
//   test_host gpu    executor tests on device 0
#include "si_host.hpp"

#include "oracle.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <functional>
#include <sstream>
#include <string>
#include <typeinfo>
#include <vector>

using namespace sharpinference;

namespace {

struct TestCase {
    const char* group;
    const char* name;
    std::function<void()> body;
};

std::vector<TestCase>& Registry()
{
    static std::vector<TestCase> tests;
    return tests;
}

struct Register {
    Register(const char* group, const char* name, std::function<void()> body)
    {
        Registry().push_back({group, name, std::move(body)});
    }
};

struct Failure : std::runtime_error {
    using std::runtime_error::runtime_error;
};

#define TEST(group, name)                                                                                         \
    void name();                                                                                                  \
    const Register register_##name(#group, #name, name);                                                         \
    void name()

#define ASSERT_TRUE(cond)                                                                                         \
    do {                                                                                                          \
        if (!(cond))                                                                                              \
            throw Failure(std::string(__FILE__ ":") + std::to_string(__LINE__) + ": " #cond);                     \
    } while (0)

// Assert.Throws<T>: the exact exception type, not a subclass.
template <typename T, typename F>
void ThrowsExactly(F&& f, const char* what, int line)
{
    try {
        f();
    } catch (const std::exception& e) {
        if (typeid(e) == typeid(T))
            return;
        throw Failure(std::string("line ") + std::to_string(line) + ": " + what + " threw " + typeid(e).name() +
                      " (" + e.what() + "), expected " + typeid(T).name());
    }
    throw Failure(std::string("line ") + std::to_string(line) + ": " + what + " did not throw");
}
#define ASSERT_THROWS(T, expr) ThrowsExactly<T>([&] { (void)(expr); }, #expr, __LINE__)

const PrecisionRequirement kFp32{GraphElementType::Float32, GraphElementType::Float32};

std::shared_ptr<const InstructionRegistry> DefaultRegistry()
{
    return std::make_shared<InstructionRegistry>(
        std::vector<std::shared_ptr<const IInstructionCollectionProvider>>{std::make_shared<HipQuantizedInstructions>()});
}

std::shared_ptr<const Instruction> MatVec()
{
    return DefaultRegistry()->Resolve(HipInstructionCollectionIds::QuantizedFloat32, "quant.mat-vec",
                                      InstructionTarget::Hip());
}

std::shared_ptr<const Instruction> GatherRow()
{
    return DefaultRegistry()->Resolve(HipInstructionCollectionIds::QuantizedFloat32, "quant.gather-row",
                                      InstructionTarget::Hip());
}

int Elems(int fmt) { return fmt == SI_HIP_Q4_K ? 256 : 32; }

const char* Name(int fmt) { return fmt == SI_HIP_Q8_0 ? "q8_0" : fmt == SI_HIP_Q4_0 ? "q4_0" : "q4_k"; }

uint64_t RowBytes(int fmt, int64_t columns)
{
    uint64_t b = 0;
    Check(si_hip_tensor_bytes(fmt, 1, columns, &b));
    return b;
}

TensorDescriptor U8(int64_t rows, int64_t bytes) { return {GraphElementType::Byte, {rows, bytes}}; }
TensorDescriptor F32(int64_t n) { return {GraphElementType::Float32, {n}}; }

// The parameters of one quant.mat-vec dispatch over a view `padding`
// elements into each slot (weight padding counts bytes).
std::vector<InstructionParameter> MatVecParameters(int fmt, int64_t rows, int64_t columns, int64_t padding,
                                                   const char* weight_port = "weight")
{
    return {InstructionParameter::Tensor(weight_port, U8(rows, RowBytes(fmt, columns)), GraphResourceAccess::Read,
                                         "weight", padding),
            InstructionParameter::Tensor("input", F32(columns), GraphResourceAccess::Read, "input", 4 * padding),
            InstructionParameter::Tensor("output", F32(rows), GraphResourceAccess::Write, "output", 4 * padding),
            InstructionParameter::Attribute("format", Name(fmt)),
            InstructionParameter::Attribute("columns", std::to_string(columns))};
}

// GpuMatVecReferencePrograms.Create(rows, columns, ..., padding, weightPort)
// for a block-quantized weight: three slots, one "forward" entry.
HipVmProgram MatVecProgram(int fmt, int64_t rows, int64_t columns, int64_t padding = 0,
                           const char* weight_port = "weight")
{
    HipVmProgram p;
    p.AddSlot({"weight", U8(1, static_cast<int64_t>(rows * RowBytes(fmt, columns)) + 2 * padding),
               VmAccess::ReadOnly});
    p.AddSlot({"input", F32(columns + 2 * padding), VmAccess::ReadOnly});
    p.AddSlot({"output", F32(rows + 2 * padding), VmAccess::ReadWrite});
    p.AddDispatch("forward", MatVec(), MatVecParameters(fmt, rows, columns, padding, weight_port), kFp32);
    return p;
}

HipVmProgram GatherProgram(int fmt, int64_t rows, int64_t columns)
{
    HipVmProgram p;
    p.AddSlot({"table", U8(rows, RowBytes(fmt, columns)), VmAccess::ReadOnly});
    p.AddSlot({"index", {GraphElementType::Int32, {1}}, VmAccess::ReadWrite});
    p.AddSlot({"output", F32(columns), VmAccess::ReadWrite});
    p.AddDispatch("forward", GatherRow(),
                  {InstructionParameter::Tensor("table", U8(rows, RowBytes(fmt, columns)), GraphResourceAccess::Read,
                                                "table"),
                   InstructionParameter::Tensor("index", {GraphElementType::Int32, {1}}, GraphResourceAccess::Read,
                                                "index"),
                   InstructionParameter::Tensor("output", F32(columns), GraphResourceAccess::Write, "output"),
                   InstructionParameter::Attribute("format", Name(fmt)),
                   InstructionParameter::Attribute("columns", std::to_string(columns))},
                  kFp32);
    return p;
}

std::vector<uint8_t> Quant(int fmt, uint64_t seed, int64_t rows, int64_t columns)
{
    std::vector<uint8_t> w(rows * RowBytes(fmt, columns));
    orc_gen_quant(fmt, seed, rows, columns, 0.02, w.data());
    return w;
}

// A [rows, columns] matrix whose every weight decodes to exactly 1.
std::vector<uint8_t> Ones(int fmt, int64_t rows, int64_t columns)
{
    const int64_t blocks = rows * columns / Elems(fmt);
    std::vector<uint8_t> w;
    for (int64_t b = 0; b < blocks; b++) {
        if (fmt == SI_HIP_Q8_0) {           // d = 1, q = 1
            w.insert(w.end(), {0x00, 0x3c});
            w.insert(w.end(), 32, 0x01);
        } else if (fmt == SI_HIP_Q4_0) {    // d = 1, q - 8 = 1
            w.insert(w.end(), {0x00, 0x3c});
            w.insert(w.end(), 16, 0x99);
        } else {                            // d = 1, dmin = 0, sc = 1, m = 0, q = 1
            w.insert(w.end(), {0x00, 0x3c, 0x00, 0x00, 1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1});
            w.insert(w.end(), 128, 0x11);
        }
    }
    return w;
}

template <typename T>
std::vector<uint8_t> Bytes(const std::vector<T>& v)
{
    std::vector<uint8_t> b(v.size() * sizeof(T));
    std::memcpy(b.data(), v.data(), b.size());
    return b;
}

std::vector<float> Floats(const std::vector<uint8_t>& b)
{
    std::vector<float> v(b.size() / 4);
    std::memcpy(v.data(), b.data(), b.size());
    return v;
}

// The GEMV gate: |y - t| <= 1e-3 * max(|t|, rms(t)) elementwise and
// ||y - t|| / ||t|| <= 1e-5.
void AssertGemvClose(const float* y, const std::vector<double>& t)
{
    double ss = 0, es = 0;
    for (double v : t)
        ss += v * v;
    const double rms = std::sqrt(ss / t.size());
    for (size_t i = 0; i < t.size(); i++) {
        const double e = std::fabs(y[i] - t[i]);
        if (!(e <= 1e-3 * std::max(std::fabs(t[i]), rms)))
            throw Failure("row " + std::to_string(i) + ": " + std::to_string(y[i]) + " vs " + std::to_string(t[i]));
        es += e * e;
    }
    if (ss > 0 && !(std::sqrt(es / ss) <= 1e-5))
        throw Failure("L2-relative error " + std::to_string(std::sqrt(es / ss)));
}

// ---- contract and registry (no device) ---------------------------------------------------

TEST(cpu, RegistryResolvesTheQuantizedCollection)
{
    const auto registry = DefaultRegistry();
    const auto collections = registry->QueryInstructionCollection();
    ASSERT_TRUE(collections.size() == 1);
    ASSERT_TRUE(collections[0].id == HipInstructionCollectionIds::QuantizedFloat32);
    ASSERT_TRUE(collections[0].architecture == InstructionTarget::Hip());
    ASSERT_TRUE(MatVec()->Name() == "quant.mat-vec");
    ASSERT_TRUE(GatherRow()->Name() == "quant.gather-row");
    ASSERT_THROWS(NotSupportedException, registry->QueryInstruction("00000000-0000-0000-0000-000000000000", "x"));
    ASSERT_THROWS(ArgumentException, registry->QueryInstruction(HipInstructionCollectionIds::QuantizedFloat32, " "));
    ASSERT_THROWS(NotSupportedException,
                  registry->Resolve(HipInstructionCollectionIds::QuantizedFloat32, "core.mat-vec", InstructionTarget::Hip()));
    ASSERT_THROWS(NotSupportedException, registry->Resolve(HipInstructionCollectionIds::QuantizedFloat32,
                                                           "quant.mat-vec", InstructionTarget{"direct3d12"}));
    ASSERT_TRUE(registry->QueryInstruction(HipInstructionCollectionIds::QuantizedFloat32, "quant.other").empty());
}

struct FixedProvider : IInstructionCollectionProvider {
    std::vector<InstructionCollectionDescription> descriptions;
    std::vector<std::shared_ptr<const Instruction>> instructions;
    std::vector<InstructionCollectionDescription> QueryInstructionCollection() const override { return descriptions; }
    std::vector<std::shared_ptr<const Instruction>> QueryInstruction(const std::string&,
                                                                    const std::string&) const override
    {
        return instructions;
    }
};

struct RenamedMatVec : QuantizedMatVecInstruction {
    std::string Name() const override { return "quant.renamed"; }
};

TEST(cpu, RegistryRejectsConflictsForeignIdentitiesAndAmbiguity)
{
    using Providers = std::vector<std::shared_ptr<const IInstructionCollectionProvider>>;
    ASSERT_THROWS(ArgumentException, InstructionRegistry(Providers{nullptr}));
    auto renamed = std::make_shared<FixedProvider>();
    renamed->descriptions = {{HipInstructionCollectionIds::QuantizedFloat32, "HIP quantized products v2", 0,
                              InstructionTarget::Hip()}};
    ASSERT_THROWS(InvalidDataException,
                  InstructionRegistry(Providers{std::make_shared<HipQuantizedInstructions>(), renamed}));
    auto nameless = std::make_shared<FixedProvider>();
    nameless->descriptions = {{"11111111-2222-3333-4444-555555555555", " ", 0, InstructionTarget::Hip()}};
    ASSERT_THROWS(InvalidDataException, InstructionRegistry(Providers{nameless}));
    auto foreign = std::make_shared<FixedProvider>();
    foreign->descriptions = {{HipInstructionCollectionIds::QuantizedFloat32, "HIP quantized products", 0,
                              InstructionTarget::Hip()}};
    foreign->instructions = {std::make_shared<RenamedMatVec>()};
    ASSERT_THROWS(InvalidDataException, InstructionRegistry(Providers{foreign}).QueryInstruction(
                                            HipInstructionCollectionIds::QuantizedFloat32, "quant.mat-vec"));
    auto twice = std::make_shared<FixedProvider>();
    twice->descriptions = foreign->descriptions;
    twice->instructions = {std::make_shared<QuantizedMatVecInstruction>(),
                           std::make_shared<QuantizedMatVecInstruction>()};
    ASSERT_THROWS(InvalidDataException, InstructionRegistry(Providers{twice}).QueryInstruction(
                                            HipInstructionCollectionIds::QuantizedFloat32, "quant.mat-vec"));
}

TEST(cpu, AdaptationSelectsTheSignatureAndRejectsMismatches)
{
    const auto mv = MatVec();
    const auto ok = MatVecParameters(SI_HIP_Q4_K, 7, 512, 0);
    ASSERT_TRUE(mv->Adapt(ok, kFp32).ports[0].name == "weight");
    ASSERT_TRUE(mv->Adapt(MatVecParameters(SI_HIP_Q8_0, 7, 64, 0, "matrix"), kFp32).ports[0].name == "matrix");
    // a weaker requirement is satisfied by FP32 arithmetic
    ASSERT_TRUE(mv->Adapt(ok, {GraphElementType::Float16, GraphElementType::Float16}).precision.arithmetic_type ==
                GraphElementType::Float32);
    auto with = [&](std::function<void(std::vector<InstructionParameter>&)> change) {
        auto p = ok;
        change(p);
        return p;
    };
    using P = std::vector<InstructionParameter>;
    ASSERT_THROWS(InstructionAdaptationException, mv->Adapt(with([](P& p) { p.pop_back(); }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException, mv->Adapt(with([](P& p) { p.push_back(p[3]); }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException,
                  mv->Adapt(with([](P& p) { p[0].tensor.element_type = GraphElementType::Float32; }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException,
                  mv->Adapt(with([](P& p) { p[2].access = GraphResourceAccess::Read; }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException,
                  mv->Adapt(with([](P& p) { p[0].name = "matrix2"; }), kFp32));
    // a requirement that is not a floating-point type (OperatorBackend.cs:143-149)
    ASSERT_THROWS(ArgumentException, mv->Adapt(ok, {GraphElementType::Int32, GraphElementType::Float32}));
    ASSERT_TRUE(Satisfies(GraphElementType::Float32, GraphElementType::Float16));
    ASSERT_TRUE(!Satisfies(GraphElementType::Float16, GraphElementType::Float32));
    // Validate: format, columns, and tensor shapes
    ASSERT_THROWS(InstructionAdaptationException, mv->Adapt(with([](P& p) { p[3].value = "q5_0"; }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException, mv->Adapt(with([](P& p) { p[4].value = "500"; }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException, mv->Adapt(with([](P& p) { p[4].value = "512x"; }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException, mv->Adapt(with([](P& p) { p[4].value = "-256"; }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException,
                  mv->Adapt(with([](P& p) { p[0].tensor.dimensions = {7, 287}; }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException,
                  mv->Adapt(with([](P& p) { p[1].tensor.dimensions = {511}; }), kFp32));
    ASSERT_THROWS(InstructionAdaptationException,
                  mv->Adapt(with([](P& p) { p[2].tensor.dimensions = {8}; }), kFp32));
    try {
        mv->Adapt(with([](P& p) { p[3].value = "f16"; }), kFp32);
        throw Failure("f16 format adapted");
    } catch (const InstructionAdaptationException& e) {
        const std::string m = e.what();
        ASSERT_TRUE(m.find("Instruction '" + HipInstructionCollectionIds::QuantizedFloat32 + "/quant.mat-vec'") == 0);
    }
}

// An FP16-precision instruction: an FP32 requirement cannot be met.
struct HalfPrecisionMatVec : QuantizedMatVecInstruction {
    std::vector<InstructionSignature> Signatures() const override
    {
        auto s = QuantizedMatVecInstruction::Signatures();
        for (auto& sig : s)
            sig.precision = {GraphElementType::Float16, GraphElementType::Float16};
        return s;
    }
};

TEST(cpu, PrecisionRequirementsAboveTheSignatureAreRejectedWithTheProvidedProfiles)
{
    HalfPrecisionMatVec half;
    const auto p = MatVecParameters(SI_HIP_Q8_0, 3, 64, 0);
    ASSERT_TRUE(half.Adapt(p, {GraphElementType::Float16, GraphElementType::Float16}).precision.arithmetic_type ==
                GraphElementType::Float16);
    try {
        half.Adapt(p, kFp32);
        throw Failure("an FP32 requirement adapted to an FP16 signature");
    } catch (const InstructionAdaptationException& e) {
        const std::string m = e.what();
        ASSERT_TRUE(m.find("On hip.gfx950, required arithmetic=Float32, accumulator=Float32; provided "
                           "arithmetic=Float16, accumulator=Float16") != std::string::npos);
    }
}

// The enums carry the reference's members in its order (GraphModel.cs:63-77,
// VmProgram.cs:10), so values cross a managed binding unchanged.
TEST(cpu, ElementTypeAndAccessEnumsMatchTheReference)
{
    ASSERT_TRUE(static_cast<int>(GraphElementType::Byte) == 0 && static_cast<int>(GraphElementType::Int32) == 1 &&
                static_cast<int>(GraphElementType::UInt32) == 2 && static_cast<int>(GraphElementType::Float16) == 3 &&
                static_cast<int>(GraphElementType::Float32) == 4);
    ASSERT_TRUE(static_cast<int>(GraphResourceAccess::Read) == 0 && static_cast<int>(GraphResourceAccess::Write) == 1 &&
                static_cast<int>(GraphResourceAccess::ReadWrite) == 2);
    ASSERT_TRUE(static_cast<int>(VmAccess::ReadOnly) == 0 && static_cast<int>(VmAccess::ReadWrite) == 1);
    ASSERT_TRUE(ElementSize(GraphElementType::Byte) == 1 && ElementSize(GraphElementType::Int32) == 4 &&
                ElementSize(GraphElementType::UInt32) == 4 && ElementSize(GraphElementType::Float16) == 2 &&
                ElementSize(GraphElementType::Float32) == 4);
    // only floating-point types are precisions (OperatorBackend.cs:143-149)
    ASSERT_THROWS(ArgumentException, Satisfies(GraphElementType::UInt32, GraphElementType::Float32));
    ASSERT_THROWS(ArgumentException, Satisfies(GraphElementType::Float32, GraphElementType::Byte));
}

// A Write port accepts a Write or a ReadWrite parameter and rejects a Read
// one; a Read port accepts any access (InstructionCollection.cs:163-165).
TEST(cpu, WritePortsAcceptWriteAndReadWriteParameters)
{
    const auto mv = MatVec();
    ASSERT_TRUE(mv->Signatures()[0].ports[2].access == GraphResourceAccess::Write);
    auto p = MatVecParameters(SI_HIP_Q8_0, 7, 64, 0);
    for (GraphResourceAccess a : {GraphResourceAccess::Write, GraphResourceAccess::ReadWrite}) {
        p[2].access = a;
        ASSERT_TRUE(mv->Adapt(p, kFp32).ports[2].name == "output");
    }
    p[2].access = GraphResourceAccess::Read;
    ASSERT_THROWS(InstructionAdaptationException, mv->Adapt(p, kFp32));
    p[2].access = GraphResourceAccess::Write;
    p[1].access = GraphResourceAccess::ReadWrite;    // more access than a Read port asks for
    ASSERT_TRUE(mv->Adapt(p, kFp32).ports[1].name == "input");
}

// An instruction with UInt32 ports: a UInt32 tensor adapts, an Int32 tensor
// of the same shape does not (the element type is matched exactly).
struct UInt32CopyInstruction : Instruction {
    std::string CollectionId() const override { return HipInstructionCollectionIds::QuantizedFloat32; }
    std::string Name() const override { return "test.copy-u32"; }
    InstructionTarget Target() const override { return InstructionTarget::Hip(); }
    std::vector<InstructionSignature> Signatures() const override
    {
        return {{{{"input", GraphElementType::UInt32, GraphResourceAccess::Read},
                  {"output", GraphElementType::UInt32, GraphResourceAccess::Write}},
                 {},
                 {GraphElementType::Float32, GraphElementType::Float32}}};
    }

protected:
    InstructionRecording Generate(const std::vector<InstructionParameter>& parameters) const override
    {
        return {"copy", parameters};
    }
};

TEST(cpu, UInt32TensorsAdaptByExactElementType)
{
    UInt32CopyInstruction copy;
    const TensorDescriptor u32{GraphElementType::UInt32, {5, 3}};
    ASSERT_TRUE(u32.ByteLength() == 60);
    std::vector<InstructionParameter> p{
        InstructionParameter::Tensor("input", u32, GraphResourceAccess::Read, "a"),
        InstructionParameter::Tensor("output", u32, GraphResourceAccess::Write, "b")};
    ASSERT_TRUE(copy.Adapt(p, kFp32).ports[0].element_type == GraphElementType::UInt32);
    p[0].tensor.element_type = GraphElementType::Int32;
    ASSERT_THROWS(InstructionAdaptationException, copy.Adapt(p, kFp32));
    // bound into a program: the UInt32 view must fit its slot, and a write
    // into a read-only slot is rejected
    HipVmProgram program;
    program.AddSlot({"a", u32, VmAccess::ReadOnly});
    program.AddSlot({"b", {GraphElementType::UInt32, {15}}, VmAccess::ReadOnly});
    auto q = p;
    q[0].tensor.element_type = GraphElementType::UInt32;
    ASSERT_THROWS(InvalidDataException, program.AddDispatch("forward", std::make_shared<UInt32CopyInstruction>(), q, kFp32));
    program.AddSlot({"c", {GraphElementType::UInt32, {15}}, VmAccess::ReadWrite});
    q[1].source = "c";
    program.AddDispatch("forward", std::make_shared<UInt32CopyInstruction>(), q, kFp32);
    ASSERT_TRUE(program.Entries().at("forward").size() == 1);
}

struct OtherTargetRecorder : IInstructionRecorder {
    InstructionTarget Target() const override { return {"direct3d12"}; }
    void Record(InstructionRecording) override { throw Failure("recorded on a foreign target"); }
};

TEST(cpu, InvokeRequiresTheRecordersTarget)
{
    OtherTargetRecorder r;
    ASSERT_THROWS(InstructionAdaptationException, MatVec()->Invoke(r, MatVecParameters(SI_HIP_Q8_0, 3, 64, 0), kFp32));
}

TEST(cpu, ProgramRejectsUnknownSlotsOversizedViewsWritesToReadSlotsAndAliasing)
{
    auto program = MatVecProgram(SI_HIP_Q8_0, 7, 65 * 32, 3);
    ASSERT_TRUE(program.Entries().at("forward").size() == 1);
    ASSERT_TRUE(program.Entries().at("forward")[0].recording.operation == "si_hip_gemv");
    ASSERT_THROWS(InvalidDataException, program.AddSlot({"input", F32(4), VmAccess::ReadOnly}));
    ASSERT_THROWS(InvalidDataException, program.AddSlot({"empty", F32(0), VmAccess::ReadOnly}));
    auto p = MatVecParameters(SI_HIP_Q8_0, 7, 65 * 32, 3);
    auto unknown = p;
    unknown[1].source = "missing";
    ASSERT_THROWS(ArgumentException, program.AddDispatch("second", MatVec(), unknown, kFp32));
    auto oversized = p;
    oversized[2].byte_offset = 4 * 7;       // 7 + 7 > 7 + 2 * 3 floats
    ASSERT_THROWS(InvalidDataException, program.AddDispatch("second", MatVec(), oversized, kFp32));
    auto readonly = p;
    readonly[2].source = "input";
    ASSERT_THROWS(InvalidDataException, program.AddDispatch("second", MatVec(), readonly, kFp32));
    // the output aliasing the input inside one writable slot
    HipVmProgram shared;
    shared.AddSlot({"weight", U8(7, RowBytes(SI_HIP_Q8_0, 64)), VmAccess::ReadOnly});
    shared.AddSlot({"buffer", F32(64), VmAccess::ReadWrite});
    auto aliased = MatVecParameters(SI_HIP_Q8_0, 7, 64, 0);
    aliased[1].source = aliased[2].source = "buffer";
    aliased[2].byte_offset = 4 * 32;
    ASSERT_THROWS(NotSupportedException, shared.AddDispatch("forward", MatVec(), aliased, kFp32));
    aliased[2].byte_offset = 4 * 58;        // 58 + 7 floats do not fit in the 64-float slot
    ASSERT_THROWS(InvalidDataException, shared.AddDispatch("forward", MatVec(), aliased, kFp32));
    ASSERT_THROWS(ArgumentException, shared.AddDispatch("forward", nullptr, p, kFp32));
    ASSERT_THROWS(ArgumentException, shared.AddDispatch(" ", MatVec(), p, kFp32));
    // a rejected dispatch leaves the program unchanged
    ASSERT_TRUE(shared.Entries().empty());
}

// The reference's collections resolve on the HIP target under their own
// identities (InstructionCollection.cs:6-12, GpuTransformerInstructionCollection.cs:11-44).
TEST(cpu, ReferenceCollectionsResolveOnTheHipTarget)
{
    const auto reg = DefaultHipRegistry();
    const auto& T = InstructionCollectionIds::TransformerFloat32;
    for (const char* n : {"transformer.rms-norm", "transformer.residual-rms-norm", "transformer.swiglu",
                          "transformer.rope-kv-write", "transformer.grouped-query-attention", "transformer.argmax"})
        ASSERT_TRUE(reg->Resolve(T, n, InstructionTarget::Hip())->Name() == n);
    for (const char* n : {"core.mat-vec", "core.gather-row", "core.tensor.batched-mat-vec"})
        ASSERT_TRUE(reg->Resolve(InstructionCollectionIds::TierZeroFloat32, n, InstructionTarget::Hip())->Name() == n);
    ASSERT_THROWS(NotSupportedException, reg->Resolve(T, "transformer.rms-norm", {"direct3d12"}));
    ASSERT_TRUE(reg->QueryInstruction(T, "transformer.gqa-scores").empty());
    // the transformer ports carry the reference's names, types and accesses
    const auto rope = reg->Resolve(T, "transformer.rope-kv-write", InstructionTarget::Hip());
    const auto sig = rope->Signatures()[0];
    ASSERT_TRUE(sig.ports.size() == 6 && sig.ports[1].name == "position" &&
                sig.ports[1].element_type == GraphElementType::Int32 && sig.ports[4].name == "key_cache" &&
                sig.ports[4].access == GraphResourceAccess::Write);
    ASSERT_TRUE((sig.attributes == std::vector<std::string>{"head_size", "rotary_size", "rope_scale"}));
}

TEST(cpu, TransformerInstructionsAdaptWithTheReferenceRules)
{
    const auto reg = DefaultHipRegistry();
    const auto& T = InstructionCollectionIds::TransformerFloat32;
    using P = InstructionParameter;
    const auto f32 = [](std::vector<int64_t> d) { return TensorDescriptor{GraphElementType::Float32, std::move(d)}; };
    const auto rms = reg->Resolve(T, "transformer.rms-norm", InstructionTarget::Hip());
    std::vector<P> p{P::Tensor("input", f32({64}), GraphResourceAccess::Read, "a"),
                     P::Tensor("weight", f32({64}), GraphResourceAccess::Read, "b"),
                     P::Tensor("output", f32({64}), GraphResourceAccess::Write, "c"), P::Attribute("epsilon", "1e-05")};
    rms->Adapt(p, kFp32);
    for (const char* bad : {"0", "-1", "nan", "inf", "1e-5x", ""}) {
        auto q = p;
        q[3].value = bad;
        ASSERT_THROWS(InstructionAdaptationException, rms->Adapt(q, kFp32));
    }
    const auto gqa = reg->Resolve(T, "transformer.grouped-query-attention", InstructionTarget::Hip());
    const auto cache = [](GraphElementType t) { return TensorDescriptor{t, {16, 2, 128}}; };
    for (GraphElementType t : {GraphElementType::Float32, GraphElementType::Float16}) {
        std::vector<P> g{P::Tensor("query", f32({8 * 128}), GraphResourceAccess::Read, "q"),
                         P::Tensor("key_cache", cache(t), GraphResourceAccess::Read, "k"),
                         P::Tensor("value_cache", cache(t), GraphResourceAccess::Read, "v"),
                         P::Tensor("position", {GraphElementType::Int32, {1}}, GraphResourceAccess::Read, "p"),
                         P::Tensor("output", f32({8 * 128}), GraphResourceAccess::Write, "o")};
        ASSERT_TRUE(gqa->Adapt(g, kFp32).ports[1].element_type == t);
        auto bad = g;
        bad[0].tensor = f32({6 * 128});   // query and output heads differ
        ASSERT_THROWS(InstructionAdaptationException, gqa->Adapt(bad, kFp32));
        bad[4].tensor = f32({6 * 128});   // 6 query heads over 2 KV heads
        gqa->Adapt(bad, kFp32);
        bad[1].tensor = bad[2].tensor = TensorDescriptor{t, {16, 4, 128}};
        ASSERT_THROWS(InstructionAdaptationException, gqa->Adapt(bad, kFp32));   // 6 heads over 4 KV heads
        bad = g;
        bad[2].tensor = TensorDescriptor{t, {16, 2, 64}};
        ASSERT_THROWS(InstructionAdaptationException, gqa->Adapt(bad, kFp32));   // mismatched caches
    }
}

TEST(cpu, Phi4ProgramFollowsTheReferenceDispatchOrder)
{
    Phi4ProgramShape s;
    s.layers = 2;
    s.hidden = 1024;
    s.heads = 8;
    s.kv_heads = 2;
    s.ffn = 2048;
    s.vocab = 100;
    s.context = 32;
    const auto p = BuildPhi4DecodeProgram(s);
    const auto& d = p.Entries().at("decode");
    ASSERT_TRUE(d.size() == 2 + 9 * 2 + 2);
    std::vector<std::string> names;
    for (const auto& x : d)
        names.push_back(x.instruction->Name());
    const std::vector<std::string> layer{"quant.mat-vec",    "transformer.rope-kv-write",
                                         "transformer.grouped-query-attention", "quant.mat-vec",
                                         "transformer.residual-rms-norm",       "quant.mat-vec",
                                         "transformer.swiglu",                  "quant.mat-vec",
                                         "transformer.residual-rms-norm"};
    std::vector<std::string> want{"quant.gather-row", "transformer.rms-norm"};
    for (int l = 0; l < 2; l++)
        want.insert(want.end(), layer.begin(), layer.end());
    want.push_back("quant.mat-vec");
    want.push_back("transformer.argmax");
    ASSERT_TRUE(names == want);
    // the second residual-rms-norm of layer 0 normalises onto layer 1's attention norm
    const auto& r = d[2 + 8].recording.parameters;
    bool onto_next = false;
    for (const auto& q : r)
        onto_next |= q.name == "weight" && q.source == "attn_norm_1";
    ASSERT_TRUE(onto_next);
    // dense weights dispatch the T0 mat-vec and gather over typed slots; the
    // tied head projects onto the embedding table
    s.weight_format = s.embed_format = s.head_format = SI_HIP_F16;
    s.tied = true;
    s.cache_type = GraphElementType::Float32;
    const auto dense = BuildPhi4DecodeProgram(s);
    const auto& dd = dense.Entries().at("decode");
    ASSERT_TRUE(dd.front().instruction->Name() == "core.gather-row" &&
                dd.front().instruction->CollectionId() == InstructionCollectionIds::TierZeroFloat32);
    ASSERT_TRUE(dd[2].instruction->Name() == "core.mat-vec");
    ASSERT_TRUE(dense.SlotIndex("output_weight") < 0 &&
                dense.Slots()[dense.SlotIndex("qkv_weight_0")].tensor.element_type == GraphElementType::Float16 &&
                dense.Slots()[dense.SlotIndex("key_cache_1")].tensor.element_type == GraphElementType::Float32);
    bool head_on_embedding = false;
    for (const auto& q : dd[dd.size() - 2].recording.parameters)
        head_on_embedding |= q.name == "weight" && q.source == "token_embedding";
    ASSERT_TRUE(head_on_embedding);
    auto bad = s;
    bad.hidden = 1000;
    ASSERT_THROWS(ArgumentException, BuildPhi4DecodeProgram(bad));
    bad = s;
    bad.rotary_dim = 97;
    ASSERT_THROWS(ArgumentException, BuildPhi4DecodeProgram(bad));
    bad = s;
    bad.head_format = SI_HIP_Q8_0;   // tied head in another format
    ASSERT_THROWS(ArgumentException, BuildPhi4DecodeProgram(bad));
    const auto f = Phi4RopeFrequencies(Phi4ProgramShape{});
    ASSERT_TRUE(f.size() == 48 && f[0] == 1.0f && std::fabs(f[47] - 1.0f / std::pow(10000.0f, 94.0f / 96.0f)) < 1e-12f);
}

TEST(cpu, BatchInstructionsAdaptWithTheReferenceRules)
{
    // GpuBatchTransformerInstructions.cs:12-96 shape rules, :101-679 per op
    const auto reg = DefaultHipRegistry();
    const auto& T = InstructionCollectionIds::TransformerFloat32;
    using P = InstructionParameter;
    const auto R = GraphResourceAccess::Read, W = GraphResourceAccess::Write;
    const auto f32 = [](std::vector<int64_t> d) { return TensorDescriptor{GraphElementType::Float32, std::move(d)}; };
    const TensorDescriptor ctl{GraphElementType::Int32, {2}};
    const auto rms = reg->Resolve(T, "transformer.batch-rms-norm", InstructionTarget::Hip());
    std::vector<P> p{P::Tensor("input", f32({16, 64}), R, "a"), P::Tensor("weight", f32({64}), R, "b"),
                     P::Tensor("control", ctl, R, "c"), P::Tensor("output", f32({16, 64}), W, "d"),
                     P::Attribute("epsilon", "1e-05")};
    rms->Adapt(p, kFp32);
    auto bad = p;
    bad[0].tensor = f32({16 * 64});            // 'input' must have rank 2
    ASSERT_THROWS(InstructionAdaptationException, rms->Adapt(bad, kFp32));
    bad = p;
    bad[3].tensor = f32({8, 64});              // input and output shapes differ
    ASSERT_THROWS(InstructionAdaptationException, rms->Adapt(bad, kFp32));
    bad = p;
    bad[2].tensor = TensorDescriptor{GraphElementType::Int32, {3}};   // control [3]
    ASSERT_THROWS(InstructionAdaptationException, rms->Adapt(bad, kFp32));
    bad = p;
    bad[0].tensor = bad[3].tensor = f32({17, 64});   // more rows than the HIP batch
    ASSERT_THROWS(InstructionAdaptationException, rms->Adapt(bad, kFp32));

    // the shared mat-vec: F16 (the reference) and F32 weights; block formats go to quant.batch-mat-vec
    const auto bmv = reg->Resolve(T, "transformer.batch-shared-matvec", InstructionTarget::Hip());
    for (GraphElementType wt : {GraphElementType::Float16, GraphElementType::Float32}) {
        std::vector<P> m{P::Tensor("weight", TensorDescriptor{wt, {96, 64}}, R, "w"),
                         P::Tensor("input", f32({16, 64}), R, "x"), P::Tensor("control", ctl, R, "c"),
                         P::Tensor("output", f32({16, 96}), W, "y")};
        ASSERT_TRUE(bmv->Adapt(m, kFp32).ports[0].element_type == wt);
        auto wrong = m;
        wrong[3].tensor = f32({16, 95});        // output [B,O] mismatch
        ASSERT_THROWS(InstructionAdaptationException, bmv->Adapt(wrong, kFp32));
    }
    const auto qbmv = reg->Resolve(HipInstructionCollectionIds::QuantizedFloat32, "quant.batch-mat-vec",
                                   InstructionTarget::Hip());
    std::vector<P> q{P::Tensor("weight", TensorDescriptor{GraphElementType::Byte, {96, 36}}, R, "w"),
                     P::Tensor("input", f32({16, 64}), R, "x"), P::Tensor("control", ctl, R, "c"),
                     P::Tensor("output", f32({16, 96}), W, "y"), P::Attribute("format", "q4_0"),
                     P::Attribute("columns", "64")};
    qbmv->Adapt(q, kFp32);
    auto wq = q;
    wq[5].value = "128";                        // 36-byte rows hold 64 Q4_0 columns
    ASSERT_THROWS(InstructionAdaptationException, qbmv->Adapt(wq, kFp32));

    // rope-kv-write: qkv width = query + 2 kv, frequencies [rotary/2]
    const auto rope = reg->Resolve(T, "transformer.batch-rope-kv-write", InstructionTarget::Hip());
    const auto cache = [](GraphElementType t) { return TensorDescriptor{t, {32, 2, 128}}; };
    for (GraphElementType t : {GraphElementType::Float32, GraphElementType::Float16}) {
        std::vector<P> r{P::Tensor("qkv", f32({16, 8 * 128 + 2 * 256}), R, "qkv"), P::Tensor("control", ctl, R, "c"),
                         P::Tensor("frequencies", f32({48}), R, "f"), P::Tensor("query", f32({16, 8 * 128}), W, "q"),
                         P::Tensor("key_cache", cache(t), W, "k"), P::Tensor("value_cache", cache(t), W, "v"),
                         P::Attribute("head_size", "128"), P::Attribute("rotary_size", "96"),
                         P::Attribute("rope_scale", "1.19")};
        rope->Adapt(r, kFp32);
        auto wr = r;
        wr[2].tensor = f32({47});
        ASSERT_THROWS(InstructionAdaptationException, rope->Adapt(wr, kFp32));
        wr = r;
        wr[0].tensor = f32({16, 8 * 128 + 256});
        ASSERT_THROWS(InstructionAdaptationException, rope->Adapt(wr, kFp32));
    }
    // scores [B, qheads, context] over a matching cache; values output [B, qheads * head]
    const auto scores = reg->Resolve(T, "transformer.batch-gqa-scores", InstructionTarget::Hip());
    std::vector<P> sc{P::Tensor("query", f32({16, 8 * 128}), R, "q"),
                      P::Tensor("key_cache", cache(GraphElementType::Float32), R, "k"),
                      P::Tensor("control", ctl, R, "c"), P::Tensor("scores", f32({16, 8, 32}), W, "s")};
    scores->Adapt(sc, kFp32);
    auto ws = sc;
    ws[3].tensor = f32({16, 8, 31});            // context column count differs from the cache
    ASSERT_THROWS(InstructionAdaptationException, scores->Adapt(ws, kFp32));
    const auto values = reg->Resolve(T, "transformer.batch-gqa-values", InstructionTarget::Hip());
    std::vector<P> va{P::Tensor("probabilities", f32({16, 8, 32}), R, "p"),
                      P::Tensor("value_cache", cache(GraphElementType::Float16), R, "v"),
                      P::Tensor("control", ctl, R, "c"), P::Tensor("output", f32({16, 8 * 128}), W, "o")};
    values->Adapt(va, kFp32);
    auto wv = va;
    wv[0].tensor = f32({16, 6, 32});            // 6 query heads, output holds 8
    ASSERT_THROWS(InstructionAdaptationException, values->Adapt(wv, kFp32));
    const auto last = reg->Resolve(T, "transformer.batch-select-last", InstructionTarget::Hip());
    std::vector<P> sl{P::Tensor("input", f32({16, 64}), R, "x"), P::Tensor("control", ctl, R, "c"),
                      P::Tensor("output", f32({63}), W, "y")};
    ASSERT_THROWS(InstructionAdaptationException, last->Adapt(sl, kFp32));
}

TEST(cpu, Phi4PrefillEntryFollowsTheReferenceDispatchOrder)
{
    Phi4ProgramShape s;
    s.layers = 2;
    s.hidden = 1024;
    s.heads = 8;
    s.kv_heads = 2;
    s.ffn = 2048;
    s.vocab = 100;
    s.context = 64;
    s.prompt_rows = 40;
    const auto p = BuildPhi4DecodeProgram(s);
    ASSERT_TRUE(p.Entries().at("decode").size() == 2 + 9 * 2 + 2);
    const auto& d = p.Entries().at("prefill_fused_16");
    ASSERT_TRUE(d.size() == 2 + 11 * 2 + 3);
    std::vector<std::string> names;
    for (const auto& x : d)
        names.push_back(x.instruction->Name());
    const std::vector<std::string> layer{
        "quant.batch-mat-vec",         "transformer.batch-rope-kv-write",       "transformer.batch-gqa-scores",
        "transformer.batch-causal-softmax", "transformer.batch-gqa-values",     "quant.batch-mat-vec",
        "transformer.batch-residual-rms-norm", "quant.batch-mat-vec",           "transformer.batch-swiglu",
        "quant.batch-mat-vec",         "transformer.batch-residual-rms-norm"};
    std::vector<std::string> want{"transformer.batch-gather-rows", "transformer.batch-rms-norm"};
    for (int l = 0; l < 2; l++)
        want.insert(want.end(), layer.begin(), layer.end());
    want.insert(want.end(), {"transformer.batch-select-last", "quant.mat-vec", "transformer.argmax"});
    ASSERT_TRUE(names == want);
    // the batch slots and the shared caches / control
    ASSERT_TRUE(p.Slots()[p.SlotIndex("fused_embeddings")].tensor.dimensions == std::vector<int64_t>({40, 1024}));
    ASSERT_TRUE(p.Slots()[p.SlotIndex("batch_scores")].tensor.dimensions == std::vector<int64_t>({16, 8, 64}));
    bool writes_layer_cache = false;
    for (const auto& q : d[3].recording.parameters)
        writes_layer_cache |= q.name == "key_cache" && q.source == "key_cache_0";
    ASSERT_TRUE(writes_layer_cache);
    // dense weights use the transformer collection's shared mat-vec
    s.weight_format = s.embed_format = s.head_format = SI_HIP_F16;
    const auto dense = BuildPhi4DecodeProgram(s);
    ASSERT_TRUE(dense.Entries().at("prefill_fused_16")[2].instruction->Name() == "transformer.batch-shared-matvec");
    auto bad = s;
    bad.prompt_rows = 65;                        // longer than the context
    ASSERT_THROWS(ArgumentException, BuildPhi4DecodeProgram(bad));
}

// Everything a program's execution depends on, in entry and dispatch order.
std::string Fingerprint(const HipVmProgram& p)
{
    std::ostringstream o;
    o << p.name << '|' << p.abi << '|' << p.state_schema << '|' << p.state_version << '\n';
    for (const auto& s : p.state)
        o << "state " << s.name << '=' << s.slot << '\n';
    for (const auto& s : p.Slots()) {
        o << "slot " << s.id << ' ' << static_cast<int>(s.scope) << ' ' << static_cast<int>(s.access) << ' '
          << static_cast<int>(s.tensor.element_type) << ' ' << s.binding_key;
        for (auto d : s.tensor.dimensions)
            o << ',' << d;
        o << '\n';
    }
    for (const auto& [entry, ds] : p.Entries())
        for (const auto& d : ds) {
            o << entry << ' ' << d.instruction->CollectionId() << ' ' << d.instruction->Name() << ' '
              << d.recording.operation << ' ' << static_cast<int>(d.precision.minimum_arithmetic_type)
              << static_cast<int>(d.resolved.accumulator_type);
            auto ps = d.recording.parameters;
            std::sort(ps.begin(), ps.end(), [](const auto& a, const auto& b) { return a.name < b.name; });
            for (const auto& q : ps) {
                o << " [" << q.name << ':' << static_cast<int>(q.kind) << ':' << q.value << ':' << q.source << '@'
                  << q.byte_offset << ':' << static_cast<int>(q.access) << ':'
                  << static_cast<int>(q.tensor.element_type);
                for (auto x : q.tensor.dimensions)
                    o << ',' << x;
                o << ']';
            }
            o << '\n';
        }
    return o.str();
}

TEST(cpu, VmProgramXmlRoundTripsThePhi4Program)
{
    Phi4ProgramShape s;
    s.layers = 2;
    s.hidden = 1024;
    s.heads = 8;
    s.kv_heads = 2;
    s.ffn = 2048;
    s.vocab = 100;
    s.context = 64;
    s.prompt_rows = 20;
    const auto p = BuildPhi4DecodeProgram(s);
    const std::string xml = SerializeVmProgram(p);
    ASSERT_TRUE(xml.rfind("<VmProgram name=\"phi4-hip-decode\" abi=\"phi4.decode.fp16\" target=\"Hip\">", 0) == 0);
    // control's token and position words are parameters of their own, bound at byte offsets 0 and 4
    ASSERT_TRUE(xml.find("<Argument parameter=\"position\" source=\"control\" byteOffset=\"4\" />") != std::string::npos);
    ASSERT_TRUE(xml.find("<Port name=\"key_cache\" access=\"Write\" />") != std::string::npos);
    const auto q = DeserializeVmProgram(xml);
    ASSERT_TRUE(Fingerprint(q) == Fingerprint(p));
    ASSERT_TRUE(SerializeVmProgram(q) == xml);
    // dense weights, FP32 caches, no prefill entry
    s.weight_format = s.embed_format = s.head_format = SI_HIP_F32;
    s.tied = true;
    s.cache_type = GraphElementType::Float32;
    s.prompt_rows = 0;
    const auto d = BuildPhi4DecodeProgram(s);
    ASSERT_TRUE(Fingerprint(DeserializeVmProgram(SerializeVmProgram(d))) == Fingerprint(d));
}

TEST(cpu, VmProgramXmlReaderRejectsWhatTheReferenceRejects)
{
    const std::string good = SerializeVmProgram(MatVecProgram(SI_HIP_Q8_0, 3, 32));
    DeserializeVmProgram(good);
    const auto edit = [&](const std::string& from, const std::string& to) {
        std::string x = good;
        const size_t i = x.find(from);
        if (i == std::string::npos)
            throw Failure("fixture text not found: " + from);
        return x.replace(i, from.size(), to);
    };
    const std::vector<std::string> bad{
        "<!DOCTYPE VmProgram [<!ENTITY x \"y\">]>" + good,       // DTD processing is prohibited
        edit("<Slots>", "<Slots>text"),                            // text content
        edit("<Slots>", "<Slots><Extra />"),                      // unknown element
        edit("<Slots>", "<Slots extra=\"1\">"),                   // unknown attribute
        edit("target=\"Hip\"", "target=\"Direct3D12\""),         // another target
        edit("scope=\"Global\"", "scope=\"global\""),             // enum names are exact
        edit("elementType=\"Byte\"", "elementType=\"Int8\""),
        edit("kind=\"Orchestration\"", "kind=\"Kernel\""),        // the HIP executor runs orchestrations
        edit("<Dimension size=\"3\" />", "<Dimension size=\"0\" />"),
        edit("<Slots>", "<Slots><Slot id=\"a\" scope=\"Global\" access=\"ReadOnly\" access=\"ReadOnly\" /></Slots><Slots>"),
        edit("<State ", "<State xmlns:z=\"urn:z\" z:a=\"1\" "),   // namespaced attribute
        edit(" />", " &bogus; />"),                               // undeclared entity
        good.substr(0, good.size() - 3),                           // truncated
        edit("5c2f7b1e-9a4d-4f0e-8e61-3b7f2d9c4a10", "5c2f7b1e-9a4d-4f0e-8e61-3b7f2d9c4a11"),   // unknown collection
        std::string(64 + 2, '<'),
    };
    int i = 0;
    for (const auto& x : bad) {
        bool threw = false;
        try {
            DeserializeVmProgram(x);
        } catch (const std::exception&) {
            threw = true;
        }
        if (!threw)
            throw Failure("malformed case " + std::to_string(i) + " was accepted");
        i++;
    }
    // nesting beyond 64 levels
    std::string deep = "<VmProgram name=\"a\" abi=\"b\" target=\"Hip\">";
    for (int k = 0; k < 70; k++)
        deep += "<Slots>";
    ASSERT_THROWS(InvalidDataException, DeserializeVmProgram(deep));
    // comments and processing instructions are ignored
    DeserializeVmProgram("<?xml version=\"1.0\"?><!-- c -->" + good + "<!-- d -->");
}

TEST(cpu, HipArtifactRoundTripsAndDetectsCorruption)
{
    ASSERT_TRUE(Sha256Hex("", 0) == "E3B0C44298FC1C149AFBF4C8996FB92427AE41E4649B934CA495991B7852B855");
    ASSERT_TRUE(Sha256Hex("abc", 3) == "BA7816BF8F01CFEA414140DE5DAE2223B00361A396177A9CB410FF61F20015AD");
    const std::string m56 = "abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq";
    ASSERT_TRUE(Sha256Hex(m56.data(), m56.size()) ==
                "248D6A61D20638B8E5C026930C3E6039A33CE45964FF2167F6ECEDD419DB06C1");
    Phi4ProgramShape s;
    s.layers = 1;
    s.hidden = 1024;
    s.heads = 8;
    s.kv_heads = 2;
    s.ffn = 2048;
    s.vocab = 64;
    s.context = 32;
    const auto p = BuildPhi4DecodeProgram(s);
    const auto a = ExportHipVmArtifact(p);
    ASSERT_TRUE(a.size() > 4 && a[0] == 'P' && a[1] == 'K');
    ASSERT_TRUE(Fingerprint(ImportHipVmArtifact(a)) == Fingerprint(p));
    // a flipped byte inside program.xml: the stored entry's CRC or the program hash rejects it
    auto c = a;
    c[200] ^= 0x20;
    ASSERT_THROWS(InvalidDataException, ImportHipVmArtifact(c));
    // the envelope hash covers the manifest
    std::string t(a.begin(), a.end());
    const size_t at = t.find("c-abi-launch");
    ASSERT_TRUE(at != std::string::npos);
    auto d = a;
    d[at] = 'C';
    ASSERT_THROWS(InvalidDataException, ImportHipVmArtifact(d));
    ASSERT_THROWS(InvalidDataException, ImportHipVmArtifact(std::vector<uint8_t>(a.begin(), a.begin() + 40)));
}

TEST(cpu, ExecutorWithoutADeviceFailsLoudly)
{
    int n = 0;
    if (si_hip_device_count(&n) == SI_HIP_OK && n > 0)
        return;   // a device is present: the GPU group covers the executor
    ASSERT_THROWS(DeviceException, HipVmExecutor(MatVecProgram(SI_HIP_Q8_0, 3, 32)));
}

// ---- executor (device 0) -----------------------------------------------------------------

// Execute (GpuMatVecTests.cs:283-310): every slot is filled with 13 outside
// the views, executed three times, the padding is left untouched and the
// inputs read back unchanged.
void ExecuteView(int fmt, int64_t rows, int64_t columns, const char* weight_port, uint64_t seed)
{
    const int64_t padding = 3;
    auto program = MatVecProgram(fmt, rows, columns, padding, weight_port);
    HipVmExecutor executor(program);
    const auto w = Quant(fmt, seed, rows, columns);
    std::vector<float> x(columns);
    orc_gen_normal_f32(seed + 1, columns, 0.0, 1.0, x.data());
    std::vector<uint8_t> weight(w.size() + 2 * padding, 13);
    std::copy(w.begin(), w.end(), weight.begin() + padding);
    std::vector<float> input(columns + 2 * padding, 13.0f), output(rows + 2 * padding, 13.0f);
    std::copy(x.begin(), x.end(), input.begin() + padding);
    executor.Upload("weight", weight);
    executor.Upload("input", Bytes(input));
    executor.Upload("output", Bytes(output));
    std::vector<double> t(rows);
    Check(orc_gemv_f64(fmt, w.data(), x.data(), t.data(), rows, columns) == 0 ? SI_HIP_OK : SI_HIP_ERR_ARGUMENT);
    for (int repeat = 0; repeat < 3; repeat++) {
        executor.Execute("forward");
        const auto actual = Floats(executor.Readback("output"));
        for (int64_t i = 0; i < padding; i++)
            ASSERT_TRUE(actual[i] == 13.0f && actual[rows + padding + i] == 13.0f);
        AssertGemvClose(actual.data() + padding, t);
    }
    ASSERT_TRUE(executor.Readback("weight") == weight);
    ASSERT_TRUE(executor.Readback("input") == Bytes(input));
    // a new input is read by the recorded entry
    for (auto& v : x)
        v = -2.0f * v;
    std::copy(x.begin(), x.end(), input.begin() + padding);
    executor.Upload("input", Bytes(input));
    executor.Execute("forward");
    Check(orc_gemv_f64(fmt, w.data(), x.data(), t.data(), rows, columns) == 0 ? SI_HIP_OK : SI_HIP_ERR_ARGUMENT);
    AssertGemvClose(Floats(executor.Readback("output")).data() + padding, t);
}

TEST(gpu, QuantizedSignaturesHandleTailsViewsAndRepeatedInvocation)
{
    // (rows, blocks per row), as (rows, columns) of GpuMatVecTests.cs:14-21
    const int64_t shapes[][2] = {{1, 1}, {7, 17}, {7, 63}, {7, 64}, {7, 65}, {3, -1}, {65536, 3}, {65537, 3}};
    uint64_t seed = 500;
    for (int fmt : {SI_HIP_Q8_0, SI_HIP_Q4_0, SI_HIP_Q4_K})
        for (const auto& s : shapes) {
            const int64_t columns = s[1] < 0 ? 4096 : s[1] * Elems(fmt);
            std::printf("    %s %lld x %lld\n", Name(fmt), static_cast<long long>(s[0]),
                        static_cast<long long>(columns));
            std::fflush(stdout);
            ExecuteView(fmt, s[0], columns, (seed / 2) % 2 ? "matrix" : "weight", seed);
            seed += 2;
        }
}

TEST(gpu, AlignedSlotsMeetTheGate)
{
    // Views at offset 0 of 256-byte aligned slots: the 3072-column product
    // runs on the tiled kernel (the views above run on the any-shape ones).
    for (int fmt : {SI_HIP_Q8_0, SI_HIP_Q4_0, SI_HIP_Q4_K}) {
        const int64_t rows = 3072, columns = 3072;
        HipVmExecutor executor(MatVecProgram(fmt, rows, columns));
        const auto w = Quant(fmt, 900 + fmt, rows, columns);
        std::vector<float> x(columns);
        orc_gen_normal_f32(901 + fmt, columns, 0.0, 1.0, x.data());
        executor.Upload("weight", w);
        executor.Upload("input", Bytes(x));
        executor.Execute("forward");
        std::vector<double> t(rows);
        orc_gemv_f64(fmt, w.data(), x.data(), t.data(), rows, columns);
        AssertGemvClose(Floats(executor.Readback("output")).data(), t);
    }
}

TEST(gpu, QuantizedNonfiniteSumsRetainClassification)
{
    const float inf = INFINITY;
    const std::vector<std::vector<float>> inputs = {{inf, 1}, {-inf, 1}, {inf, -inf}, {NAN, 1}};
    for (int fmt : {SI_HIP_Q8_0, SI_HIP_Q4_0, SI_HIP_Q4_K})
        for (int64_t columns : {int64_t(Elems(fmt)), int64_t(3072)}) {
            HipVmExecutor executor(MatVecProgram(fmt, 3, columns));
            executor.Upload("weight", Ones(fmt, 3, columns));
            for (const auto& head : inputs) {
                std::vector<float> x(columns, 0.0f);
                std::copy(head.begin(), head.end(), x.begin());
                executor.Upload("input", Bytes(x));
                executor.Execute("forward");
                const float expected = head[0] + head[1];
                for (float v : Floats(executor.Readback("output")))
                    ASSERT_TRUE(std::isnan(expected) ? std::isnan(v) : v == expected);
            }
        }
}

TEST(gpu, ResidentTimestampMeasurementExecutesAndRejectsInvalidRequests)
{
    HipVmExecutor executor(MatVecProgram(SI_HIP_Q8_0, 3, 65 * 32));
    executor.Upload("weight", Ones(SI_HIP_Q8_0, 3, 65 * 32));
    executor.Upload("input", Bytes(std::vector<float>(65 * 32, 1.0f)));
    const double elapsed = executor.MeasureGpuMicroseconds("forward", 4);
    ASSERT_TRUE(std::isfinite(elapsed) && elapsed > 0);
    for (float v : Floats(executor.Readback("output")))
        ASSERT_TRUE(v == 65 * 32);
    ASSERT_THROWS(ArgumentOutOfRangeException, executor.MeasureGpuMicroseconds("forward", 0));
    ASSERT_THROWS(ArgumentOutOfRangeException, executor.MeasureGpuMicroseconds("forward", 1025));
    ASSERT_THROWS(ArgumentException, executor.MeasureGpuMicroseconds("missing", 1));
}

TEST(gpu, SpanUploadExecutesWithoutOwnedSourceArray)
{
    // [[1, 2], [3, 4], [5, 6]] . [2, 3] = [8, 18, 28], as one Q8_0 block per row (d = 1)
    HipVmExecutor executor(MatVecProgram(SI_HIP_Q8_0, 3, 32));
    uint8_t matrix[3 * 34] = {};
    for (int r = 0; r < 3; r++) {
        matrix[34 * r + 1] = 0x3c;
        matrix[34 * r + 2] = static_cast<uint8_t>(2 * r + 1);
        matrix[34 * r + 3] = static_cast<uint8_t>(2 * r + 2);
    }
    float input[32] = {2, 3};
    executor.Upload("weight", matrix, sizeof matrix);
    executor.Upload("input", input, sizeof input);
    executor.Execute("forward");
    ASSERT_TRUE(Floats(executor.Readback("output")) == (std::vector<float>{8, 18, 28}));
}

TEST(gpu, UploadRequiresExactSlotBytesAndKnownNames)
{
    HipVmExecutor executor(MatVecProgram(SI_HIP_Q4_0, 5, 64));
    ASSERT_THROWS(ArgumentException, executor.Upload("weight", std::vector<uint8_t>(5 * 36 - 1)));
    ASSERT_THROWS(ArgumentException, executor.Upload("weight", std::vector<uint8_t>(5 * 36 + 1)));
    ASSERT_THROWS(ArgumentException, executor.Upload("missing", std::vector<uint8_t>(4)));
    ASSERT_THROWS(ArgumentException, executor.Readback("missing"));
    ASSERT_THROWS(ArgumentException, executor.Execute("missing"));
    // slots start zeroed: the product of a zero matrix is zero
    executor.Execute("forward");
    for (float v : Floats(executor.Readback("output")))
        ASSERT_TRUE(v == 0.0f);
}

TEST(gpu, GatherRowDecodesTheIndexedRowExactlyAndNaNOutsideTheTable)
{
    for (int fmt : {SI_HIP_Q8_0, SI_HIP_Q4_0, SI_HIP_Q4_K}) {
        const int64_t rows = 50, columns = 3072;
        HipVmExecutor executor(GatherProgram(fmt, rows, columns));
        const auto table = Quant(fmt, 700 + fmt, rows, columns);
        executor.Upload("table", table);
        for (int32_t index : {0, 17, 49, 50, -1}) {
            std::vector<uint8_t> out(4 * columns);
            executor.ExecuteWithTransfers("forward", "index", Bytes(std::vector<int32_t>{index}), "output", out);
            const auto y = Floats(out);
            if (index < 0 || index >= rows) {
                for (float v : y)
                    ASSERT_TRUE(std::isnan(v));
                continue;
            }
            std::vector<float> expected(columns);
            orc_dequant_row(fmt, table.data() + index * RowBytes(fmt, columns), columns, expected.data());
            ASSERT_TRUE(std::memcmp(y.data(), expected.data(), 4 * columns) == 0);
        }
        std::vector<uint8_t> small(4);
        ASSERT_THROWS(ArgumentException,
                      executor.ExecuteWithTransfers("forward", "index", Bytes(std::vector<int32_t>{0}), "output", small));
    }
}

}  // namespace

int main(int argc, char** argv)
{
    const std::string group = argc > 1 ? argv[1] : "cpu";
    const std::string only = argc > 2 ? argv[2] : "";
    if (group != "cpu" && group != "gpu") {
        std::fprintf(stderr, "usage: %s cpu|gpu [test-name]\n", argv[0]);
        return 2;
    }
    int run = 0, failed = 0;
    for (const auto& t : Registry()) {
        if (t.group != group || (!only.empty() && only != t.name))
            continue;
        std::printf("[ RUN  ] %s\n", t.name);
        std::fflush(stdout);
        run++;
        try {
            t.body();
            std::printf("[  OK  ] %s\n", t.name);
        } catch (const std::exception& e) {
            failed++;
            std::printf("[ FAIL ] %s: %s\n", t.name, e.what());
        }
        std::fflush(stdout);
    }
    std::printf("%d %s tests, %d failed\n", run, group.c_str(), failed);
    return failed || run == 0 ? 1 : 0;
}
