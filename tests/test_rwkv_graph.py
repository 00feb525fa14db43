"""The portable RWKV-7 forward-token graph and its lowering to a HIP VM
program, on the CPU (no device): host/si_graph.cpp through
host_program.rwkv7_graph_describe.

Graph tests restate PortableRwkv7GraphProviderTests.cs (:11-128) on the
same catalog (width 8 in 2 heads of 4, vocabulary 32, LoRA ranks 2-4):
identity, state slots, the node chain, the cast count, the WKV update's
matrix algebra and the rejection of a mis-shaped LoRA.  Lowering tests
follow VmGraphOptimizer.cs: FP16 weight casts that only feed matrix
operators become FP16 views, reshapes of weights become views, local
intermediates share slots, one kernel definition per distinct operator,
and the mat-vec selection's diagnostics (GpuMatVecOptimization.cs:34-59).
"""
from types import SimpleNamespace

import numpy as np
import pytest

from sharpinference_amd import host_program, native, rwkv7

PRIMITIVES = {"core.copy", "core.add", "core.subtract", "core.multiply", "core.divide", "core.maximum", "core.exp",
              "core.tanh", "core.sigmoid", "core.rsqrt", "core.square", "core.relu", "core.reduce-sum",
              "core.reduce-mean", "core.mat-vec", "core.gather-row", "core.tensor.fill", "core.tensor.cast-f16-f32",
              "core.tensor.reshape", "core.tensor.slice", "core.tensor.broadcast", "core.tensor.batched-mat-vec",
              "core.tensor.reduce-last-sum", "core.tensor.reduce-last-mean", "core.tensor.head-outer"}

CFG8 = SimpleNamespace(vocab=32, hidden=8, layers=1)


def reference_catalog(layers, fmt, invalid_w2=False):
    """The catalog of PortableRwkv7GraphProviderTests.Catalog (:176-209):
    name -> (type, dims, data) with zero data of the right byte size."""
    cat = {}

    def add(name, *dims):
        n = int(np.prod(dims))
        cat[name] = (fmt, list(dims), np.zeros(n, np.float16 if fmt == native.F16 else np.float32))

    add("emb.weight", 8, 32)
    add("head.weight", 8, 32)
    add("ln_out.weight", 8)
    add("ln_out.bias", 8)
    add("blocks.0.ln0.weight", 8)
    add("blocks.0.ln0.bias", 8)
    for i in range(layers):
        p = f"blocks.{i}."
        for name in ("ln1.weight", "ln1.bias", "ln2.weight", "ln2.bias", "att.w0", "att.a0", "att.k_k", "att.k_a",
                     "att.ln_x.weight", "att.ln_x.bias", "ffn.x_k"):
            add(p + name, 8)
        add(p + "att.x_rwkvag", 8, 6)
        add(p + "att.r_k", 4, 2)
        for name in ("att.receptance.weight", "att.key.weight", "att.value.weight", "att.output.weight"):
            add(p + name, 8, 8)
        for family, rank in (("w", 2 if i == 0 else 3), ("a", 3), ("g", 4)):
            add(p + f"att.{family}1", 8, rank)
            add(p + f"att.{family}2", rank + 1 if family == "w" and invalid_w2 else rank, 8)
        if i > 0:
            add(p + "att.v0", 8)
            add(p + "att.v1", 8, 2)
            add(p + "att.v2", 2, 8)
        add(p + "ffn.key.weight", 8, 16)
        add(p + "ffn.value.weight", 16, 8)
    return cat


def describe(layers, fmt, **options):
    return host_program.rwkv7_graph_describe(SimpleNamespace(vocab=32, hidden=8, layers=layers),
                                             reference_catalog(layers, fmt), **options)


@pytest.mark.parametrize("fmt,layers", [(native.F32, 1), (native.F16, 2)], ids=["f32-1", "f16-2"])
def test_builds_complete_primitive_graph_with_versioned_tensor_contracts(fmt, layers):
    graph, _, _ = describe(layers, fmt)
    assert graph["name"] == "rwkv7.forward-token.portable"
    assert graph["architecture"] == "rwkv-7"
    assert graph["stateSchema"] == "RWKV7_State"
    assert graph["stateAbi"] == "rwkv-7.state.fp32@1"
    assert graph["inputs"] == ["token"] and graph["outputs"] == ["logits"]
    assert graph["state"] == [f"state.{l}.{s}" for l in range(layers) for s in ("ffn-previous", "att-previous", "wkv")]
    res = {r["id"]: r for r in graph["resources"]}
    assert res["state.0.wkv"]["dims"] == [2, 4, 4]
    for r in graph["resources"]:
        if r["kind"] == 2:   # Weight
            assert r["key"] == r["id"][len("weight."):]
    nodes = graph["nodes"]
    assert all(n["operation"] in PRIMITIVES for n in nodes)
    assert not any(n["operation"].startswith(("rwkv7.", "rwkv.")) for n in nodes)
    for i in range(1, len(nodes)):
        assert nodes[i]["dependencies"] == [nodes[i - 1]["id"]]
    assert [n["id"] for n in nodes] == [f"portable.{i:05d}" for i in range(len(nodes))]
    casts = sum(n["operation"] == "core.tensor.cast-f16-f32" for n in nodes)
    assert casts == (len(reference_catalog(layers, fmt)) if fmt == native.F16 else 0)
    stores = [n for n in nodes if n["operation"] == "core.copy" and n["bindings"][-1][1].endswith(".wkv")]
    assert len(stores) == layers
    assert sum(n["operation"] == "core.tensor.slice" for n in nodes) == 6 * layers
    fills = {n["attributes"]["value"] for n in nodes if n["operation"] == "core.tensor.fill"}
    assert "-0.606531" in fills and "0.00064" in fills


def test_wkv_update_is_explicit_matrix_algebra_with_old_state_projection_and_new_state_output():
    graph, _, _ = describe(1, native.F32)
    nodes = graph["nodes"]
    producers = {}
    for n in nodes:
        for port, resource, access in n["bindings"]:
            if access != 0 and not resource.startswith("state."):
                producers[resource] = n
    read = lambda n, port: next(r for p, r, a in n["bindings"] if p == port)
    store = next(n for n in nodes if n["operation"] == "core.copy" and read(n, "output") == "state.0.wkv")
    updated = read(store, "input")
    total = producers[updated]
    assert total["operation"] == "core.add"
    old_terms = producers[read(total, "left")]
    assert old_terms["operation"] == "core.add"
    decay_term = producers[read(old_terms, "left")]
    assert decay_term["operation"] == "core.multiply"
    assert read(decay_term, "left") == "state.0.wkv"
    assert producers[read(decay_term, "right")]["operation"] == "core.tensor.broadcast"
    assert producers[read(old_terms, "right")]["operation"] == "core.tensor.head-outer"
    adaptation_term = producers[read(total, "right")]
    assert adaptation_term["operation"] == "core.tensor.head-outer"
    negative = producers[read(adaptation_term, "left")]
    assert negative["operation"] == "core.subtract"
    projection = producers[read(negative, "right")]
    assert projection["operation"] == "core.tensor.batched-mat-vec"
    assert read(projection, "matrix") == "state.0.wkv"
    assert read(projection, "vector") == read(producers[read(adaptation_term, "right")], "left")
    assert any(n["operation"] == "core.tensor.batched-mat-vec" and read(n, "matrix") == updated for n in nodes)
    assert nodes.index(projection) < nodes.index(store)


def test_rejects_invalid_low_rank_projection_shape():
    with pytest.raises(native.HipError) as e:
        host_program.rwkv7_graph_describe(CFG8, reference_catalog(1, native.F32, invalid_w2=True))
    assert e.value.status == native.ERR_FORMAT


@pytest.mark.parametrize("edit,message", [
    (lambda c: c.pop("blocks.0.att.r_k"), "does not satisfy the RWKV-7 x070 contract"),
    (lambda c: c.__setitem__("blocks.0.att.r_k", (native.F32, [4, 3], np.zeros(12, np.float32))),
     "head dimensions do not match the embedding size"),
    (lambda c: c.__setitem__("blocks.0.att.r_k", (native.F32, [3, 2], np.zeros(6, np.float32))),
     "receptance-key dimensions do not match the head shape"),
    (lambda c: c.__setitem__("blocks.0.att.k_k", (native.F32, [7], np.zeros(7, np.float32))),
     "does not have 8 elements"),
    (lambda c: c.__setitem__("blocks.0.att.key.weight", (native.F32, [4, 16], np.zeros(64, np.float32))),
     "has invalid projection dimensions"),
    (lambda c: c.__setitem__("emb.weight", (native.F32, [8, 31], np.zeros(248, np.float32))),
     "does not match the vocabulary size"),
])
def test_catalog_errors_carry_the_reference_messages(edit, message):
    cat = reference_catalog(1, native.F32)
    edit(cat)
    with pytest.raises(native.HipError) as e:
        host_program.rwkv7_graph_describe(CFG8, cat)
    assert e.value.status == native.ERR_FORMAT and message in str(e.value)


def test_fp16_weights_feed_matrix_operators_as_views():
    """NativeHalfWeights + WeightViews (VmGraphOptimizer.cs:198-299): the
    casts of the FP16 matrices (mat-vec matrices and the embedding table,
    through their reshapes) are gone and those operators read FP16 slots;
    the casts of vectors stay, and their reshapes become views."""
    graph, report, xml = describe(2, native.F16)
    cat = reference_catalog(2, native.F16)
    matrices = [n for n in cat if cat[n][1] != [8] and n not in ("blocks.0.att.x_rwkvag", "blocks.1.att.x_rwkvag",
                                                                 "blocks.0.att.r_k", "blocks.1.att.r_k")]
    ops = [n["operation"] for n in report["nodes"]]
    assert ops.count("core.tensor.cast-f16-f32") == len(cat) - len(matrices)
    assert ops.count("core.mat-vec") == 12 + 14 + 1
    # removed: each matrix's cast and its reshape to [output, input] (none for the 8 x 8 matrices, 4 per
    # layer, whose shape needs no reshape), and per layer the reshapes of the cast r_k and x_rwkvag
    square = sum(cat[n][1] == [8, 8] for n in matrices)
    assert report["removedNodes"] == 2 * len(matrices) - square + 2 * 2
    assert 'elementType="Float16"' in xml
    # the lowered program reads back identically (operators re-adapted on the HIP target)
    assert host_program.xml_roundtrip(xml) == xml


def test_reuse_of_local_storage_and_one_definition_per_operator():
    graph, report, xml = describe(2, native.F32)
    temporaries = sum(r["kind"] == 5 for r in graph["resources"])
    assert 0 < report["localSlots"] < temporaries // 4
    _, unshared, _ = describe(2, native.F32, reuse_local_storage=False)
    assert unshared["localSlots"] == 0
    definitions = {n["definition"] for n in report["nodes"]}
    assert len(definitions) == report["definitions"] < len(report["nodes"])
    assert xml.count('kind="Kernel"') == report["definitions"]
    assert xml.count("<Dispatch ") == len(report["nodes"]) == xml.count("<Barrier")
    # nodes sharing a definition share the operator and its parameter shapes
    by_def = {}
    for n in report["nodes"]:
        by_def.setdefault(n["definition"], set()).add(n["operation"])
    assert all(len(v) == 1 for v in by_def.values())


@pytest.mark.parametrize("mode,cooperative,diagnostic", [
    (None, True, "Default GPU MatVec implementation: cooperative."),
    ("default", True, "Default GPU MatVec implementation: cooperative."),
    ("cooperative", True, "Explicit cooperative MatVec; not a measured selection."),
    ("serial", False, "Explicit serial MatVec."),
])
def test_matvec_selection_report(mode, cooperative, diagnostic):
    _, report, _ = describe(2, native.F32, matvec_mode=mode)
    mv = [n for n in report["nodes"] if n["operation"] == "core.mat-vec"]
    assert report["matvec"]["calls"] == len(mv) == 27
    assert report["matvec"]["cooperativeCalls"] == (27 if cooperative else 0)
    assert report["matvec"]["diagnostics"] == [diagnostic]
    for n in mv:
        assert n["cooperative"] == cooperative and n["diagnostic"] == diagnostic
        assert n["implementation"] == ("si_hip_gemv.dense" if cooperative else "si_hip_gemv.dense.any_shape")
        assert n["threads"] == (256 if cooperative else 64)


def test_quantized_catalog_lowers_to_quantized_operators():
    cfg = rwkv7.Rwkv7Config(layers=2, hidden=128, heads=2, ffn=256, vocab=50, rank_w=32, rank_a=32, rank_v=32,
                            rank_g=32)
    cat = host_program.rwkv7_catalog(cfg, rwkv7.synth_weights(cfg, seed=1))
    graph, report, xml = host_program.rwkv7_graph_describe(cfg, cat)
    ops = [n["operation"] for n in graph["nodes"]]
    assert ops.count("quant.mat-vec") == 12 + 14 + 1 and ops.count("quant.gather-row") == 1
    assert "core.mat-vec" not in ops and "core.tensor.cast-f16-f32" not in ops
    mv = [n for n in graph["nodes"] if n["operation"] == "quant.mat-vec"]
    assert all(n["attributes"]["format"] == "q8_0" for n in mv)
    assert report["removedNodes"] == 2      # the r_k reshapes of the two layers
    assert host_program.xml_roundtrip(xml) == xml


def test_thread_group_bounds():
    for bad in (0, 1025):
        with pytest.raises(native.HipError) as e:
            describe(1, native.F32, threads_per_group=bad)
        assert e.value.status == native.ERR_ARGUMENT
