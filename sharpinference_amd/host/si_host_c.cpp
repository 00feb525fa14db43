// C entry points of the host library (si_host_c.h) over HipVmProgram /
// HipVmExecutor and BuildPhi4DecodeProgram.
#include "si_host_c.h"

#include "si_graph.hpp"
#include "si_host.hpp"

#include <algorithm>
#include <memory>
#include <string>
#include <vector>

using namespace sharpinference;

struct sih_program {
    HipVmProgram program;
    std::unique_ptr<HipVmExecutor> executor;
    std::string report;   // graph programs: the lowering report (JSON)
};

namespace {

thread_local std::string g_error;

// Runs f, mapping the host layer's exceptions to library status codes.
template <typename Fn>
int Guard(Fn&& f)
{
    try {
        f();
        return SI_HIP_OK;
    } catch (const InstructionAdaptationException& e) {
        g_error = e.what();
        return SI_HIP_ERR_ADAPTATION;
    } catch (const NotSupportedException& e) {
        g_error = e.what();
        return SI_HIP_ERR_UNSUPPORTED;
    } catch (const InvalidDataException& e) {
        g_error = e.what();
        return SI_HIP_ERR_FORMAT;
    } catch (const OutOfMemoryException& e) {
        g_error = e.what();
        return SI_HIP_ERR_OUT_OF_MEMORY;
    } catch (const InvalidOperationException& e) {
        g_error = e.what();
        return SI_HIP_ERR_STATE;
    } catch (const ArgumentException& e) {
        g_error = e.what();
        return SI_HIP_ERR_ARGUMENT;
    } catch (const std::exception& e) {
        g_error = e.what();
        return SI_HIP_ERR_DEVICE;
    }
}

ModelTensorCatalog Catalog(const sih_model_tensor* tensors, int count, int64_t vocabulary, int64_t embedding,
                           int64_t layers)
{
    if (!tensors || count < 1)
        throw ArgumentException("a catalog needs at least one tensor");
    ModelTensorCatalog c;
    c.vocabulary = vocabulary;
    c.embedding = embedding;
    c.layers = layers;
    for (int i = 0; i < count; i++) {
        const sih_model_tensor& t = tensors[i];
        if (!t.name || t.rank < 1 || t.rank > 4)
            throw ArgumentException("catalog tensor " + std::to_string(i) + ": null name or rank outside 1..4");
        if (!c.tensors.emplace(t.name, ModelTensor{t.type, std::vector<int64_t>(t.dims, t.dims + t.rank)}).second)
            throw ArgumentException(std::string("duplicate catalog tensor '") + t.name + "'");
    }
    return c;
}

HipVmOptimizationOptions Options(const sih_graph_options* o)
{
    HipVmOptimizationOptions opt;
    if (!o)
        return opt;
    opt.reuse_local_storage = o->reuse_local_storage != 0;
    opt.weight_views = o->weight_views != 0;
    opt.native_half_weights = o->native_half_weights != 0;
    opt.threads_per_group = o->threads_per_group;
    if (o->matvec_mode >= 0) {
        if (o->matvec_mode > 3 || o->matvec_mode == static_cast<int>(GpuMatVecMode::Profile))
            throw ArgumentOutOfRangeException("matvec_mode");
        opt.gpu_matvec.emplace(static_cast<GpuMatVecMode>(o->matvec_mode));
    }
    return opt;
}

void CopyOut(const std::string& text, char* buffer, uint64_t capacity, uint64_t* length)
{
    if (length)
        *length = text.size();
    if (buffer) {
        if (capacity < text.size())
            throw ArgumentException("buffer too small");
        std::copy(text.begin(), text.end(), buffer);
    }
}

std::string GraphJson(const LogicalGraph& g)
{
    const auto str = [](const std::string& s) { return JsonString(s); };
    const auto list = [&](const std::vector<std::string>& v) {
        std::string o = "[";
        for (size_t i = 0; i < v.size(); i++)
            o += (i ? "," : "") + str(v[i]);
        return o + "]";
    };
    std::vector<std::string> state;
    for (const auto& e : g.state)
        state.push_back(e.name);
    std::string j = "{\"name\":" + str(g.name) + ",\"architecture\":" + str(g.architecture) +
                    ",\"stateSchema\":" + str(g.state_schema) + ",\"stateAbi\":" + str(g.state_abi) +
                    ",\"inputs\":" + list(g.inputs) + ",\"outputs\":" + list(g.outputs) + ",\"state\":" +
                    list(state) + ",\"resources\":[";
    for (size_t i = 0; i < g.resources.size(); i++) {
        const auto& r = g.resources[i];
        j += (i ? "," : "") + std::string("{\"id\":") + str(r.id) + ",\"key\":" + str(r.binding_key) + ",\"kind\":" +
             std::to_string(static_cast<int>(r.kind)) + ",\"type\":" +
             std::to_string(static_cast<int>(r.tensor.element_type)) + ",\"dims\":[";
        for (size_t k = 0; k < r.tensor.dimensions.size(); k++)
            j += (k ? "," : "") + std::to_string(r.tensor.dimensions[k]);
        j += "]}";
    }
    j += "],\"nodes\":[";
    for (size_t i = 0; i < g.nodes.size(); i++) {
        const auto& n = g.nodes[i];
        j += (i ? "," : "") + std::string("{\"id\":") + str(n.id) + ",\"operation\":" + str(n.operation) +
             ",\"dependencies\":" + list(n.dependencies) + ",\"bindings\":[";
        for (size_t k = 0; k < n.resources.size(); k++)
            j += (k ? "," : "") + std::string("[") + str(n.resources[k].port) + "," + str(n.resources[k].resource) +
                 "," + std::to_string(static_cast<int>(n.resources[k].access)) + "]";
        j += "],\"attributes\":{";
        size_t k = 0;
        for (const auto& [a, v] : n.attributes)
            j += (k++ ? "," : "") + str(a) + ":" + str(v);
        j += "}}";
    }
    j += "]}";
    return j;
}

}  // namespace

extern "C" {

int sih_phi4_program_create(const sih_phi4_shape* s, int device, sih_program** out)
{
    return Guard([&] {
        if (!s || !out)
            throw ArgumentException("sih_phi4_program_create: null argument");
        *out = nullptr;
        Phi4ProgramShape shape;
        shape.layers = s->layers;
        shape.hidden = s->hidden;
        shape.heads = s->heads;
        shape.kv_heads = s->kv_heads;
        shape.head_dim = s->head_dim;
        shape.rotary_dim = s->rotary_dim;
        shape.ffn = s->ffn;
        shape.vocab = s->vocab;
        shape.context = s->context;
        shape.weight_format = s->weight_format;
        shape.embed_format = s->embed_format;
        shape.head_format = s->head_format;
        shape.tied = s->tied != 0;
        shape.cache_type = s->cache_fp16 ? GraphElementType::Float16 : GraphElementType::Float32;
        shape.rms_eps = s->rms_eps;
        shape.rope_base = s->rope_base;
        shape.rope_scale = s->rope_scale;
        shape.prompt_rows = s->prompt_rows;
        auto p = std::make_unique<sih_program>();
        p->program = BuildPhi4DecodeProgram(shape);
        p->executor = std::make_unique<HipVmExecutor>(p->program, device);
        const auto f = Phi4RopeFrequencies(shape);
        p->executor->Upload("rope_frequencies", f.data(), f.size() * sizeof(float));
        *out = p.release();
    });
}

int sih_program_destroy(sih_program* program)
{
    delete program;
    return SI_HIP_OK;
}

int sih_program_slot_bytes(const sih_program* program, const char* slot, uint64_t* bytes)
{
    return Guard([&] {
        if (!program || !slot || !bytes)
            throw ArgumentException("sih_program_slot_bytes: null argument");
        const int i = program->program.SlotIndex(slot);
        if (i < 0)
            throw ArgumentException(std::string("Unknown slot '") + slot + "'.");
        *bytes = program->program.Slots()[i].tensor.ByteLength();
    });
}

int sih_program_upload(sih_program* program, const char* slot, const void* bytes, uint64_t length)
{
    return Guard([&] {
        if (!program || !slot)
            throw ArgumentException("sih_program_upload: null argument");
        program->executor->Upload(slot, bytes, length);
    });
}

int sih_program_readback(sih_program* program, const char* slot, void* bytes, uint64_t length)
{
    return Guard([&] {
        if (!program || !slot || !bytes)
            throw ArgumentException("sih_program_readback: null argument");
        const auto v = program->executor->Readback(slot);
        if (v.size() != length)
            throw ArgumentException("Expected a " + std::to_string(v.size()) + "-byte buffer for slot '" + slot + "'.");
        std::copy(v.begin(), v.end(), static_cast<uint8_t*>(bytes));
    });
}

int sih_program_execute(sih_program* program, const char* entry)
{
    return Guard([&] {
        if (!program || !entry)
            throw ArgumentException("sih_program_execute: null argument");
        program->executor->Execute(entry);
    });
}

int sih_program_measure_us(sih_program* program, const char* entry, int repetitions, double* microseconds)
{
    return Guard([&] {
        if (!program || !entry || !microseconds)
            throw ArgumentException("sih_program_measure_us: null argument");
        *microseconds = program->executor->MeasureGpuMicroseconds(entry, repetitions);
    });
}

int sih_program_set_fusion(sih_program* program, int on)
{
    return Guard([&] {
        if (!program)
            throw ArgumentException("sih_program_set_fusion: null argument");
        program->executor->SetDispatchFusion(on != 0);
    });
}

int sih_program_launch_count(sih_program* program, const char* entry, int* count)
{
    return Guard([&] {
        if (!program || !entry || !count)
            throw ArgumentException("sih_program_launch_count: null argument");
        *count = program->executor->LaunchCount(entry);
    });
}

int sih_program_dispatch_count(const sih_program* program, const char* entry, int* count)
{
    return Guard([&] {
        if (!program || !entry || !count)
            throw ArgumentException("sih_program_dispatch_count: null argument");
        const auto it = program->program.Entries().find(entry);
        if (it == program->program.Entries().end())
            throw ArgumentException(std::string("Unknown entry '") + entry + "'.");
        *count = static_cast<int>(it->second.size());
    });
}

int sih_program_serialize(const sih_program* program, char* buffer, uint64_t capacity, uint64_t* length)
{
    return Guard([&] {
        if (!program || !length)
            throw ArgumentException("sih_program_serialize: null argument");
        const std::string xml = SerializeVmProgram(program->program);
        *length = xml.size();
        if (buffer) {
            if (capacity < xml.size())
                throw ArgumentException("sih_program_serialize: buffer too small");
            std::copy(xml.begin(), xml.end(), buffer);
        }
    });
}

int sih_program_create_from_xml(const char* xml, int device, sih_program** out)
{
    return Guard([&] {
        if (!xml || !out)
            throw ArgumentException("sih_program_create_from_xml: null argument");
        *out = nullptr;
        auto p = std::make_unique<sih_program>();
        p->program = DeserializeVmProgram(xml);
        p->executor = std::make_unique<HipVmExecutor>(p->program, device);
        *out = p.release();
    });
}

int sih_program_export_artifact(const sih_program* program, void* buffer, uint64_t capacity, uint64_t* length)
{
    return Guard([&] {
        if (!program || !length)
            throw ArgumentException("sih_program_export_artifact: null argument");
        const auto a = ExportHipVmArtifact(program->program);
        *length = a.size();
        if (buffer) {
            if (capacity < a.size())
                throw ArgumentException("sih_program_export_artifact: buffer too small");
            std::copy(a.begin(), a.end(), static_cast<uint8_t*>(buffer));
        }
    });
}

int sih_program_import_artifact(const void* bytes, uint64_t length, int device, sih_program** out)
{
    return Guard([&] {
        if (!bytes || !out)
            throw ArgumentException("sih_program_import_artifact: null argument");
        *out = nullptr;
        auto p = std::make_unique<sih_program>();
        const auto* b = static_cast<const uint8_t*>(bytes);
        p->program = ImportHipVmArtifact(std::vector<uint8_t>(b, b + length));
        p->executor = std::make_unique<HipVmExecutor>(p->program, device);
        *out = p.release();
    });
}

const char* sih_last_error(void) { return g_error.c_str(); }


int sih_rwkv7_graph_program_create(const sih_model_tensor* tensors, int count, int64_t vocabulary, int64_t embedding,
                                   int64_t layers, const sih_graph_options* options, int device, sih_program** out)
{
    return Guard([&] {
        if (!out)
            throw ArgumentException("sih_rwkv7_graph_program_create: null argument");
        *out = nullptr;
        HipVmOptimizationResult r =
            OptimizeWithReport(BuildRwkv7Graph(Catalog(tensors, count, vocabulary, embedding, layers)), Options(options));
        auto p = std::make_unique<sih_program>();
        p->report = OptimizationReportJson(r);
        p->program = r.program;
        p->executor = std::make_unique<HipVmExecutor>(std::move(r.program), device);
        *out = p.release();
    });
}

int sih_program_report(const sih_program* program, char* buffer, uint64_t capacity, uint64_t* length)
{
    return Guard([&] {
        if (!program || !length)
            throw ArgumentException("sih_program_report: null argument");
        CopyOut(program->report, buffer, capacity, length);
    });
}

int sih_rwkv7_graph_describe(const sih_model_tensor* tensors, int count, int64_t vocabulary, int64_t embedding,
                             int64_t layers, const sih_graph_options* options, char* graph_json, uint64_t graph_capacity,
                             uint64_t* graph_length, char* report_json, uint64_t report_capacity,
                             uint64_t* report_length, char* xml, uint64_t xml_capacity, uint64_t* xml_length)
{
    return Guard([&] {
        const LogicalGraph g = BuildRwkv7Graph(Catalog(tensors, count, vocabulary, embedding, layers));
        const HipVmOptimizationResult r = OptimizeWithReport(g, Options(options));
        CopyOut(GraphJson(g), graph_json, graph_capacity, graph_length);
        CopyOut(OptimizationReportJson(r), report_json, report_capacity, report_length);
        CopyOut(SerializeVmProgram(r.program), xml, xml_capacity, xml_length);
    });
}

int sih_program_xml_roundtrip(const char* xml, char* buffer, uint64_t capacity, uint64_t* length)
{
    return Guard([&] {
        if (!xml || !length)
            throw ArgumentException("sih_program_xml_roundtrip: null argument");
        CopyOut(SerializeVmProgram(DeserializeVmProgram(xml)), buffer, capacity, length);
    });
}

}  // extern "C"
