"""MoEPack install reader (host code, no GPU): the frozen v1/v2 documents
(MoEPackFormatCompatibilityTests.swift), the reference's manifest and layout
acceptance and rejection cases (ManifestReaderTests.swift,
PackedExpertsLayoutTests.swift, MoEPackFormatCodecTests.swift), routed-expert
offsets (ModelExpertIO.swift:56-88) and the directory rules
(MoEPackModelDirectory.swift:21-115)."""
import base64
import copy
import hashlib
import json
import os

import pytest

from tests import moepack_writer as W

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "moepack")
FORMAT, IO, INVALID = 7, 8, 1


@pytest.fixture(scope="module")
def tsg():
    import tsugumi_amd
    return tsugumi_amd


def golden(name: str) -> bytes:
    with open(os.path.join(GOLDEN, name + ".base64"), "rb") as fh:
        return base64.b64decode(fh.read())


def parse(tsg, manifest, layout=None):
    mb = manifest if isinstance(manifest, bytes) else W.dumps(manifest)
    lb = layout if (layout is None or isinstance(layout, bytes)) else W.dumps(layout)
    return tsg.MoEPack.parse(mb, lb)


def rejects(tsg, manifest, layout, status, text):
    with pytest.raises(tsg.TsgError) as e:
        parse(tsg, manifest, layout)
    assert e.value.status == status, str(e.value)
    assert text in str(e.value), str(e.value)


# ------------------------------------------------------------ frozen bytes

def test_frozen_fixture_digests():
    """The digests the reference's compatibility test pins
    (MoEPackFormatCompatibilityTests.swift:65-69)."""
    assert hashlib.sha256(golden("v2_manifest.json")).hexdigest() == \
        "da5f8d7564513546be5aae3321cd7aa4b4222c0e870726a74f14efc846b1aa82"
    assert hashlib.sha256(golden("v1_layout.json")).hexdigest() == \
        "acf57a355128d1d8afb1d09b75dc1aa7fef98687871b1ff9f738dd511cb6e341"
    # v1 differs from v2 in the magic only (MoEPackFormatCompatibilityTests.swift:28-30)
    assert golden("v1_manifest.json").replace(b'"GTURBO"', b'"MOEPACK"') == \
        golden("v2_manifest.json")


def test_frozen_documents_decode(tsg):
    pack = parse(tsg, golden("v2_manifest.json"), golden("v1_layout.json"))
    info = pack.info
    assert (info["num_layers"], info["experts_per_layer"], info["expert_stride"]) == \
        (1, 2, 16384)
    assert (info["hidden_size"], info["moe_intermediate_size"], info["top_k"]) == (64, 32, 1)
    assert info["legacy_magic"] == 0 and info["has_layout"] == 1 and info["is_gemma4"] == 1
    assert (info["affine_group_size"], info["symmetric"]) == (64, 0)
    assert (info["routed_weight_bits"], info["router_weight_bits"]) == (4, 8)
    # layout.expert(layer: 0, expert: 1).offset == expertStride
    assert list(pack.physical_offsets(0)) == [0, 16384]
    assert pack.tensor(0, 1, "gate") == {"offset": 0, "size": 32, "dtype": "U32", "bits": 4,
                                         "shape": [8, 8], "physical_rank": 1}


def test_legacy_magic_still_reads(tsg):
    pack = parse(tsg, golden("v1_manifest.json"), golden("v1_layout.json"))
    assert pack.info["legacy_magic"] == 1


def test_fixture_has_no_routed_roles(tsg):
    """The frozen layout holds a `gate` only: routedExpertOffsets has no
    gate_scales to read (the reference traps; here a format error)."""
    pack = parse(tsg, golden("v2_manifest.json"), golden("v1_layout.json"))
    with pytest.raises(tsg.TsgError) as e:
        pack.routed_offsets(0)
    assert e.value.status == FORMAT and "gate_scales" in str(e.value)


# ------------------------------------------------------------ manifest

def test_toy_manifest_reads(tsg):
    pack = parse(tsg, W.toy_manifest())
    assert pack.info["has_layout"] == 0
    assert pack.info["expert_stride"] == 16384


def test_additive_minor_and_unknown_key_accepted(tsg):
    m = W.toy_manifest(versionMinor=9, somethingNew={"x": [1, 2.5, None, True]})
    assert parse(tsg, m).info["version_minor"] == 9


@pytest.mark.parametrize("key", ["sourceSnapshotHash", "quant", "bitWidthOverridesHonored"])
def test_optional_keys_may_be_absent(tsg, key):
    m = W.toy_manifest(bitWidthOverridesHonored=120)
    del m[key]
    info = parse(tsg, m).info
    assert info["has_quant"] == (0 if key == "quant" else 1)


def test_stride_reads_exactly_above_2_53(tsg):
    stride = 2**62 + 16384  # not representable as a double
    m = W.toy_manifest(stride=stride, layer_files={})
    assert parse(tsg, m).info["expert_stride"] == stride


def test_int8_shared_expert_accepted(tsg):
    m = W.toy_manifest()
    m["quant"]["sharedExpert"]["weightBits"] = 8
    assert parse(tsg, m).info["shared_weight_bits"] == 8


def test_bf16_router_and_sym_scheme(tsg):
    m = W.toy_manifest()
    for k in ("embedding", "attention", "sharedExpert", "routedExpert"):
        m["quant"][k].update(scheme="sym", biasType="none", groupSize=32)
    m["quant"]["router"] = {"weightBits": 16, "scheme": "BF16", "scaleType": "none",
                            "biasType": "None", "groupSize": 32}
    info = parse(tsg, m).info
    assert (info["symmetric"], info["affine_group_size"], info["router_weight_bits"]) == \
        (1, 32, 16)


def test_second_family_may_widen_embedding(tsg):
    """validateQuant gates 8-bit embedding/attention on not being Gemma 4
    (ManifestReader.swift:250-260)."""
    m = W.toy_manifest()
    m["quant"]["embedding"]["weightBits"] = 8
    rejects(tsg, m, None, FORMAT, "unsupported quantization for embedding")
    m["arch"]["family"] = "qwen3_5_moe"
    info = parse(tsg, m).info
    assert info["is_gemma4"] == 0 and info["family"] == "qwen3_5_moe"


def test_linear_attention_section(tsg):
    m = W.toy_manifest(num_layers=2, versionMinor=3)
    m["flags"]["linearAttention"] = True
    m["arch"].update(family="qwen3_5_moe", slidingWindow=0,
                     layerKinds=["linear_attention", "full_attention"],
                     fullAttentionLayerMask=[0, 1],
                     linearAttention={"numKeyHeads": 16, "numValueHeads": 32, "keyHeadDim": 128,
                                      "valueHeadDim": 128, "convKernelDim": 4, "layerCount": 1})
    assert parse(tsg, m).info["num_layers"] == 2
    for mutate, text in [
        (lambda x: x.update(versionMinor=2), "linear attention requires minor >= 3"),
        (lambda x: x["flags"].pop("linearAttention"), "the flag is not set"),
        (lambda x: x["arch"].update(layerKinds=["linear_attention", "sliding_attention"]),
         "disagrees with fullAttentionLayerMask"),
        (lambda x: x["arch"].update(layerKinds=["linear_attention"]), "expected 2 entries"),
        (lambda x: x["arch"].update(layerKinds=["mamba", "full_attention"]),
         "unknown v1 layer kind"),
        (lambda x: x["arch"]["linearAttention"].update(layerCount=2),
         "layerKinds has 1 linear layers, section says 2"),
        (lambda x: x["arch"].pop("layerKinds"), "must say which layers are which"),
        (lambda x: x["arch"].update(family=""), "empty family name"),
        (lambda x: x["arch"].pop("linearAttention"), "invalid architecture values"),
    ]:
        bad = copy.deepcopy(m)
        mutate(bad)
        rejects(tsg, bad, None, FORMAT, text)
    m["arch"].pop("linearAttention")
    m["arch"]["slidingWindow"] = 128
    rejects(tsg, m, None, FORMAT, "flags.linearAttention is set but the section is absent")


def _m(fn):
    m = W.toy_manifest()
    fn(m)
    return m


MANIFEST_REJECTIONS = [
    ("magic", lambda m: m.update(magic="NOT_MOEPACK"), "notAMoEPackDirectory"),
    ("version", lambda m: m.update(versionMajor=2), "unsupportedVersion: major 2"),
    ("negative-minor", lambda m: m.update(versionMinor=-1), "unsupportedVersion"),
    ("flag", lambda m: m["flags"].update(newFangledOption=True), "unknownFlag: newFangledOption"),
    ("flag-typo", lambda m: m["flags"].update(streamingPresnt=True), "unknownFlag"),
    ("turboquant", lambda m: m["flags"].update(turboQuantKV=True), "removed TurboQuant KV"),
    ("stride", lambda m: m.update(expertStride=1024), "expertStrideNotPageAligned"),
    ("shared-3bit", lambda m: m["quant"]["sharedExpert"].update(weightBits=3),
     "unsupported quantization for sharedExpert"),
    ("router-4bit", lambda m: m["quant"]["router"].update(weightBits=4),
     "unsupported quantization for router"),
    ("routed-8bit", lambda m: m["quant"]["routedExpert"].update(weightBits=8),
     "unsupported quantization for routedExpert"),
    ("sym-with-bias", lambda m: m["quant"]["routedExpert"].update(scheme="sym"),
     "unsupported quantization for routedExpert"),
    ("bf16-with-scale", lambda m: m["quant"]["router"].update(weightBits=16, scheme="bf16"),
     "unsupported quantization for router"),
    ("scheme-mix", lambda m: m["quant"]["routedExpert"].update(scheme="sym", biasType="none"),
     "4-bit slots disagree on the affine scheme"),
    ("group-128", lambda m: [s.update(groupSize=128) for s in m["quant"].values()],
     "unsupported affine group size 128"),
    ("group-mix", lambda m: m["quant"]["routedExpert"].update(groupSize=32),
     "routedExpert group size 32 disagrees with the model's 64"),
    ("quant-zero", lambda m: m["quant"]["attention"].update(groupSize=0),
     "manifest.quant.attention: invalid quantization values"),
    ("no-weights", lambda m: m["files"].pop("model_weights.bin"), "missingFile: model_weights.bin"),
    ("no-layout", lambda m: m["files"].pop("packed_experts/layout.json"),
     "missingFile: packed_experts/layout.json"),
    ("sha", lambda m: m["files"]["model_weights.bin"].update(sha256="xyz"),
     "expected 64 hexadecimal characters"),
    ("sha-nonhex", lambda m: m["files"]["model_weights.bin"].update(sha256="g" * 64),
     "expected 64 hexadecimal characters"),
    ("reserved-manifest", lambda m: m["files"].update({"manifest.json": m["files"]["model_weights.bin"]}),
     "reserved artifact filename"),
    ("reserved-receipt", lambda m: m["files"].update(
        {"verified-install.json/x": m["files"]["model_weights.bin"]}),
     "reserved artifact filename"),
    ("reserved-tokenizer", lambda m: m["files"].update({"Tokenizer": m["files"]["model_weights.bin"]}),
     "reserved artifact filename"),
    ("dotdot", lambda m: m["files"].update({"../escape.bin": m["files"]["model_weights.bin"]}),
     "non-canonical path"),
    ("absolute", lambda m: m["files"].update({"/abs.bin": m["files"]["model_weights.bin"]}),
     "unsafe relative path"),
    ("empty-component", lambda m: m["files"].update({"a//b.bin": m["files"]["model_weights.bin"]}),
     "non-canonical path"),
    ("case-duplicate", lambda m: m["files"].update(
        {"MODEL_WEIGHTS.BIN": m["files"]["model_weights.bin"]}),
     "filesystem-equivalent duplicate path"),
    ("dir-prefix", lambda m: m["files"].update({"packed_experts": m["files"]["model_weights.bin"]}),
     "file path collides with a directory prefix"),
    ("arch-experts", lambda m: m["arch"].update(numExperts=3),
     "dimensions disagree with streaming metadata"),
    ("topk", lambda m: m["arch"].update(topKExperts=5), "invalid architecture values"),
    ("rotary", lambda m: m["arch"].update(partialRotaryFactor=1.5), "invalid architecture values"),
    ("mask-len", lambda m: m["arch"].update(fullAttentionLayerMask=[0, 1]),
     "invalid architecture values"),
    ("mask-value", lambda m: m["arch"].update(fullAttentionLayerMask=[2]),
     "invalid architecture values"),
    ("no-window", lambda m: m["arch"].update(slidingWindow=0), "invalid architecture values"),
    ("model-id", lambda m: m.update(modelID=""), "invalid dimensions or stride"),
    ("zero-layers", lambda m: m.update(numLayers=0), "invalid dimensions or stride"),
    ("missing-key", lambda m: m["arch"].pop("hiddenSize"), "arch.hiddenSize: required key is missing"),
    ("type", lambda m: m.update(numLayers="1"), "manifest.numLayers: expected an integer"),
    ("fraction", lambda m: m.update(expertsPerLayer=2.5), "expected an integer"),
    ("negative-stride", lambda m: m.update(expertStride=-16384), "expected a non-negative integer"),
    ("flag-type", lambda m: m["flags"].update(streamingPresent=1), "expected a Bool"),
    ("vision-flag", lambda m: m["flags"].update(visionTower=True),
     "flags.visionTower is set but the vision section is absent"),
    ("draft-section", lambda m: m.update(draft={"weightsPath": "draft/draft_weights.bin",
                                                 "payloadBytes": 1}),
     "draft section present but the flag is not set"),
]


@pytest.mark.parametrize("name,mutate,text", MANIFEST_REJECTIONS,
                         ids=[c[0] for c in MANIFEST_REJECTIONS])
def test_manifest_rejections(tsg, name, mutate, text):
    rejects(tsg, _m(mutate), None, FORMAT, text)


def test_vision_and_draft_files(tsg):
    m = W.toy_manifest(versionMinor=2)
    m["flags"].update(visionTower=True, mtpDraft=True)
    m["vision"] = {"weightsPath": "vision/vision_weights.bin", "payloadBytes": 100}
    m["draft"] = {"weightsPath": "draft/draft_weights.bin", "payloadBytes": 100}
    m["files"]["vision/vision_weights.bin"] = {"size": 16484, "sha256": W.ZERO_SHA}
    m["files"]["draft/draft_weights.bin"] = {"size": 16484, "sha256": W.ZERO_SHA}
    parse(tsg, m)
    bad = copy.deepcopy(m)
    bad["files"].pop("vision/vision_weights.bin")
    rejects(tsg, bad, None, FORMAT, "is not declared in manifest.files")
    bad = copy.deepcopy(m)
    bad["draft"]["payloadBytes"] = 16484
    rejects(tsg, bad, None, FORMAT, "does not fit in 16484 bytes")
    bad = copy.deepcopy(m)
    bad["versionMinor"] = 0
    rejects(tsg, bad, None, FORMAT, "vision requires minor >= 1")


def test_layer_filenames_are_left_to_the_layout(tsg):
    """defersPackedLayerFilenamesToLayoutValidation (ManifestReaderTests.swift:367-378)."""
    m = W.toy_manifest(num_layers=2, experts=2, layer_files={
        "packed_experts/experts_a.bin": 16384, "packed_experts/experts_b.bin": 16384})
    assert parse(tsg, m).info["num_layers"] == 2


# ------------------------------------------------------------ JSON reader

@pytest.mark.parametrize("doc,text", [
    (b'{"magic": "MOEPACK", "magic": "GTURBO"}', "duplicate key"),
    (b'{"magic": "MOEPACK"} x', "trailing characters"),
    (b'{"magic": "MO\xffEPACK"}', "not valid UTF-8"),
    (b'{"magic": "MOEPACK",}', "expected a member name"),
    (b'[' * 100 + b']' * 100, "nesting too deep"),
    (b'{"a": 01}', "expected ',' or '}'"),
    (b'{"a": "\\ud800"}', "lone surrogate"),
    (b'', "unexpected end of input"),
])
def test_json_reader_rejects(tsg, doc, text):
    rejects(tsg, doc, None, FORMAT, text)


def test_json_escapes_decode(tsg):
    """\\u escapes decode before the names are compared: a layer file spelled
    with escapes matches the manifest entry."""
    m = W.toy_manifest()
    lb = W.dumps(W.toy_layout()).replace(b'"layer_00.bin"', b'"layer_\\u0030\\u0030.bin"')
    assert b"\\u0030" in lb
    assert parse(tsg, m, lb).info["has_layout"] == 1


# ------------------------------------------------------------ layout

TOY_TENSORS = {"gate": {"offset": 0, "size": 4096, "dtype": "U32", "shape": [64, 64], "bits": 4},
               "gate_scales": {"offset": 4096, "size": 256, "dtype": "BF16", "shape": [64, 1]}}


def test_toy_layout_decodes(tsg):
    """decodesToyLayout (PackedExpertsLayoutTests.swift:87-104)."""
    pack = parse(tsg, W.toy_manifest(), W.toy_layout(tensors=TOY_TENSORS, physical=[[0, 1]]))
    assert list(pack.physical_offsets(0)) == [0, 16384]
    assert pack.tensor(0, 0, "gate")["offset"] == 0
    assert pack.tensor(0, 0, "gate_scales")["offset"] == 4096
    assert pack.tensor(0, 0, "gate_scales")["bits"] is None


def test_positional_ids_accepted(tsg):
    pack = parse(tsg, W.toy_manifest(), W.toy_layout(explicit_ids=False))
    assert list(pack.physical_offsets(0)) == [0, 16384]


def test_physical_ranks_permute_offsets(tsg):
    perm = [[2, 0, 3, 1]]
    pack = parse(tsg, W.toy_manifest(experts=4), W.toy_layout(experts=4, physical=perm))
    assert list(pack.physical_offsets(0)) == [r * 16384 for r in perm[0]]
    assert [pack.tensor(0, e, "gate")["physical_rank"] for e in range(4)] == perm[0]


def test_experts_listed_out_of_order_sort_by_logical_id(tsg):
    lay = W.toy_layout(experts=4, physical=[[1, 2, 3, 0]])
    lay["layers"][0]["experts"].reverse()
    pack = parse(tsg, W.toy_manifest(experts=4), lay)
    assert list(pack.physical_offsets(0)) == [16384, 32768, 49152, 0]


def nine_tensors(symmetric):
    t, cur = {}, 0
    for role in ("gate", "up", "down"):
        for comp, size, dtype in (("", 1024, "U32"), ("_scales", 64, "BF16"),
                                  ("_biases", 64, "BF16")):
            if symmetric and comp == "_biases":
                continue
            t[role + comp] = {"offset": cur, "size": size, "dtype": dtype,
                              "shape": [16, 128] if dtype == "U32" else [16, 2]}
            cur += size
    return t


@pytest.mark.parametrize("symmetric", [False, True])
def test_routed_offsets(tsg, symmetric):
    """routedExpertOffsets: nine offsets; under `sym` the bias aliases the scales."""
    pack = parse(tsg, W.toy_manifest(), W.toy_layout(tensors=nine_tensors(symmetric)))
    o = pack.routed_offsets(0)
    got = [o.gate_w, o.gate_s, o.gate_b, o.up_w, o.up_s, o.up_b, o.down_w, o.down_s, o.down_b]
    if symmetric:
        assert got == [0, 1024, 1024, 1088, 2112, 2112, 2176, 3200, 3200]
    else:
        assert got == [0, 1024, 1088, 1152, 2176, 2240, 2304, 3328, 3392]


def _l(fn, **kw):
    lay = W.toy_layout(**kw)
    fn(lay)
    return lay


def _ex(lay, i=0):
    return lay["layers"][0]["experts"][i]


LAYOUT_REJECTIONS = [
    ("dup-layer", dict(num_layers=2), lambda l: l["layers"][1].update(layer=0),
     "duplicate or invalid layer"),
    ("layer-range", {}, lambda l: l["layers"][0].update(layer=1), "duplicate or invalid layer"),
    ("slash", {}, lambda l: l["layers"][0].update(file="sub/layer_00.bin"), "expected basename"),
    ("dotdot", {}, lambda l: l["layers"][0].update(file=".."), "non-canonical path"),
    ("reserved", {}, lambda l: l["layers"][0].update(file="Layout.JSON"),
     "reserved packed-expert filename"),
    ("dup-file", dict(num_layers=2), lambda l: l["layers"][1].update(file="LAYER_00.BIN"),
     "duplicate layer filename"),
    ("count", {}, lambda l: l["layers"][0]["experts"].pop(), "wrong expert count"),
    ("mixed-ids", {}, lambda l: _ex(l, 1).pop("expert"),
     "expert ids must be either all explicit or all positional"),
    ("dup-logical", {}, lambda l: _ex(l, 1).update(expert=0),
     "duplicate or invalid expert mapping"),
    ("dup-physical", dict(physical=[[0, 1]]), lambda l: _ex(l, 1).update(physicalRank=0),
     "duplicate or invalid expert mapping"),
    ("rank-range", dict(physical=[[0, 1]]), lambda l: _ex(l, 1).update(physicalRank=2),
     "duplicate or invalid expert mapping"),
    ("offset", {}, lambda l: _ex(l, 1).update(offset=32768),
     "offset or size does not match physical rank"),
    ("size", {}, lambda l: _ex(l, 1).update(size=8192),
     "offset or size does not match physical rank"),
    ("dtype", {}, lambda l: _ex(l)["tensors"]["gate"].update(dtype="F16"),
     "invalid dtype or shape"),
    ("shape-empty", {}, lambda l: _ex(l)["tensors"]["gate"].update(shape=[]),
     "invalid dtype or shape"),
    ("shape-zero", {}, lambda l: _ex(l)["tensors"]["gate"].update(shape=[0, 8]),
     "invalid dtype or shape"),
    ("bits-zero", {}, lambda l: _ex(l)["tensors"]["gate"].update(bits=0),
     "invalid dtype or shape"),
    ("bits-33", {}, lambda l: _ex(l)["tensors"]["gate"].update(bits=33),
     "invalid dtype or shape"),
    ("size-zero", {}, lambda l: _ex(l)["tensors"]["gate"].update(size=0),
     "invalid dtype or shape"),
    ("outside", {}, lambda l: _ex(l)["tensors"]["gate"].update(offset=16380),
     "range exceeds expert blob"),
    ("overflow", {}, lambda l: _ex(l)["tensors"]["gate"].update(offset=2**64 - 16),
     "arithmetic overflow"),
    ("overlap", {}, lambda l: _ex(l)["tensors"].update(
        gate_scales={"offset": 16, "size": 32, "dtype": "BF16", "shape": [8, 1]}),
     "overlapping ranges gate and gate_scales"),
    ("stride", {}, lambda l: l.update(expertStride=8192), "invalid dimensions or stride"),
]


@pytest.mark.parametrize("name,kw,mutate,text", LAYOUT_REJECTIONS,
                         ids=[c[0] for c in LAYOUT_REJECTIONS])
def test_layout_rejections(tsg, name, kw, mutate, text):
    n = kw.get("num_layers", 1)
    rejects(tsg, W.toy_manifest(num_layers=n), _l(mutate, **kw), FORMAT, text)


def test_cross_validation(tsg):
    """crossValidationRequiresExactLayerManifestEntry (MoEPackFormatCodecTests.swift:515)."""
    m = W.toy_manifest()
    m["files"]["packed_experts/layer_00.bin"]["size"] = 16384
    rejects(tsg, m, W.toy_layout(), FORMAT, "missing or wrong layer size")
    m = W.toy_manifest(layer_files={"packed_experts/layer_01.bin": 32768})
    rejects(tsg, m, W.toy_layout(), FORMAT, "missing or wrong layer size")
    m = W.toy_manifest(stride=32768)
    rejects(tsg, m, W.toy_layout(), FORMAT, "dimension mismatch")


def test_layer_size_overflow(tsg):
    stride = 2**62 + 16384
    m = W.toy_manifest(experts=4, stride=stride, layer_files={})
    lay = W.toy_layout(experts=4, stride=stride)
    rejects(tsg, m, lay, FORMAT, "layout.layerSize: arithmetic overflow")


def test_query_errors(tsg):
    pack = parse(tsg, W.toy_manifest(), W.toy_layout())
    with pytest.raises(tsg.TsgError) as e:
        pack.routed_offsets(1)
    assert e.value.status == INVALID
    with pytest.raises(tsg.TsgError) as e:
        pack.tensor(0, 2, "gate")
    assert e.value.status == INVALID
    with pytest.raises(tsg.TsgError) as e:
        pack.tensor(0, 0, "up")
    assert e.value.status == INVALID
    no_layout = parse(tsg, W.toy_manifest())
    with pytest.raises(tsg.TsgError) as e:
        no_layout.physical_offsets(0)
    assert e.value.status == INVALID and "without packed_experts/layout.json" in str(e.value)


# ------------------------------------------------------------ directory

def write_toy_install(root, manifest=None, layout=None):
    os.makedirs(os.path.join(root, "packed_experts"), exist_ok=True)
    with open(os.path.join(root, "manifest.json"), "wb") as fh:
        fh.write(W.dumps(manifest or W.toy_manifest()))
    with open(os.path.join(root, "packed_experts", "layout.json"), "wb") as fh:
        fh.write(W.dumps(layout or W.toy_layout()))
    with open(os.path.join(root, "packed_experts", "layer_00.bin"), "wb") as fh:
        fh.write(bytes(32768))


def test_open_directory(tsg, tmp_path):
    write_toy_install(tmp_path)
    pack = tsg.MoEPack.open(tmp_path)
    assert pack.info["has_layout"] == 1 and list(pack.physical_offsets(0)) == [0, 16384]


def open_fails(tsg, path, status, text, **kw):
    with pytest.raises(tsg.TsgError) as e:
        tsg.MoEPack.open(path, **kw)
    assert e.value.status == status, str(e.value)
    assert text in str(e.value), str(e.value)


def test_missing_manifest_is_partial_install(tsg, tmp_path):
    open_fails(tsg, tmp_path, IO, "partialInstall")


def test_missing_layout(tsg, tmp_path):
    write_toy_install(tmp_path)
    os.remove(tmp_path / "packed_experts" / "layout.json")
    open_fails(tsg, tmp_path, IO, "missingFile: packed_experts/layout.json")


def test_missing_directory(tsg, tmp_path):
    open_fails(tsg, tmp_path / "nope", IO, "posixFailed")


@pytest.mark.parametrize("which", ["manifest.json", "packed_experts/layout.json"])
def test_oversized_metadata_rejected_before_decode(tsg, tmp_path, which):
    """oversizedManifestRejectsBeforeDecode / oversizedLayoutRejectsBeforeDecode."""
    write_toy_install(tmp_path)
    with open(tmp_path / which, "wb") as fh:
        fh.write(b" " * 64)
    kw = {"manifest_max_bytes" if which == "manifest.json" else "layout_max_bytes": 16}
    open_fails(tsg, tmp_path, FORMAT, "exceeds metadata cap 16", **kw)


@pytest.mark.timeout(30)
def test_fifo_layout_does_not_block(tsg, tmp_path):
    """rejectsLayoutFIFOWithoutBlocking (PackedExpertsLayoutTests.swift:8-18)."""
    write_toy_install(tmp_path)
    os.remove(tmp_path / "packed_experts" / "layout.json")
    os.mkfifo(tmp_path / "packed_experts" / "layout.json", 0o600)
    open_fails(tsg, tmp_path, IO, "not a regular file")


def test_symlinks_are_not_followed(tsg, tmp_path):
    real = tmp_path / "real"
    write_toy_install(real)
    link = tmp_path / "linked"
    os.mkdir(link)
    os.symlink(real / "manifest.json", link / "manifest.json")
    open_fails(tsg, link, IO, "posixFailed")
    os.remove(link / "manifest.json")
    with open(link / "manifest.json", "wb") as fh:
        fh.write(W.dumps(W.toy_manifest()))
    os.symlink(real / "packed_experts", link / "packed_experts")
    open_fails(tsg, link, IO, "posixFailed")


def test_writer_install_reads(tsg, tmp_path):
    """The install written for the GPU tests passes every check, with real
    file digests and a permuted physical order."""
    import numpy as np
    rng = np.random.default_rng(5)
    d, f, ne, group = 128, 64, 8, 32
    parts = [[(rng.integers(0, 256, (r, k // 2), np.uint8),
               rng.integers(0, 2**15, (r, k // group), np.uint16),
               rng.integers(0, 2**15, (r, k // group), np.uint16))
              for (r, k) in ((f, d), (f, d), (d, f))] for _ in range(ne)]
    perm = [list(rng.permutation(ne))]
    stride, offs, images = W.write_pack(tmp_path, [parts], d=d, f=f, group=group,
                                       symmetric=False, physical=perm)
    pack = tsg.MoEPack.open(tmp_path)
    assert pack.expert_stride == stride and stride % 16384 == 0
    o = pack.routed_offsets(0)
    assert [o.gate_w, o.gate_s, o.gate_b, o.up_w, o.up_s, o.up_b, o.down_w, o.down_s,
            o.down_b] == [int(v) for v in offs]
    assert list(pack.physical_offsets(0)) == [int(p) * stride for p in perm[0]]
    m = json.loads((tmp_path / "manifest.json").read_bytes())
    layer_file = (tmp_path / "packed_experts" / "layer_00.bin").read_bytes()
    assert m["files"]["packed_experts/layer_00.bin"]["sha256"] == \
        hashlib.sha256(layer_file).hexdigest()
