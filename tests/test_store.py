"""Weight-store host logic (no GPU): safetensors parsing, key rules, scale
siblings, LoRA files and merge bookkeeping through include/ltxw_store.h.

Cases restate the reference's own integration tests
(crates/ltx-weights/tests/integration.rs) where they exercise host-side
behaviour; the numerical `read` results of those tests are GPU tests
(test_gpu_store.py). Files are written with tests/st_io.py, the
`safetensors` package, or the synthetic checkpoint writer.
"""
import json
import struct

import numpy as np
import pytest

import ltx_weights as lw
import oracle_lib as O
import st_io
from ltx_weights import synth
from ltx_weights.store import KeyMap, LoraFile, WeightStore


def f32(*v):
    return np.array(v, dtype=np.float32)


@pytest.fixture
def tmp(tmp_path):
    class W:
        n = 0

        def __call__(self, tensors, metadata=None):
            W.n += 1
            p = tmp_path / f"f{W.n}.safetensors"
            st_io.write(p, tensors, metadata)
            return p

    return W()


# ---------------------------------------------------------------------------
# open / keys / rules (integration.rs:148-209, 439-455, 792-801, 878-909)
# ---------------------------------------------------------------------------
def test_transformer_key_map_strips_prefix(tmp):
    p = tmp([("model.diffusion_model.transformer_blocks.0.attn.to_q.weight", "F32", [2, 1], f32(1, 2)),
             ("unrelated_key", "F32", [2], f32(1, 2))])
    s = WeightStore.open([p], KeyMap.transformer())
    assert s.contains("transformer_blocks.0.attn.to_q.weight")
    assert not s.contains("unrelated_key")
    assert not s.contains("model.diffusion_model.transformer_blocks.0.attn.to_q.weight")
    assert s.keys() == ["transformer_blocks.0.attn.to_q.weight"]


def test_video_encoder_key_map(tmp):
    p = tmp([("vae.encoder.blocks.0.conv.weight", "F32", [3, 1], f32(1, 2, 3)),
             ("encoder.blocks.1.weight", "F32", [3], f32(1, 2, 3))])
    s = WeightStore.open([p], KeyMap.video_encoder())
    assert s.contains("blocks.0.conv.weight") and s.contains("blocks.1.weight")


def test_rename_exact_drop_prefix_drop_suffix(tmp):
    p = tmp([("t_embedder.mlp.0.weight", "F32", [1], f32(1)),
             ("coarse_head.weight", "F32", [1], f32(1)),
             ("x.tmp", "F32", [1], f32(1)),
             ("mid.t_embedder.mlp.0.bias", "F32", [1], f32(1))])
    km = KeyMap([(KeyMap.RENAME_EXACT, ["t_embedder.mlp.0.", "t_embedder.timestep_embedder.linear_1."]),
                 (KeyMap.DROP_PREFIX, ["coarse_"]),
                 (KeyMap.DROP_SUFFIX, [".tmp"])])
    s = WeightStore.open([p], km)
    # RenameExact only rewrites a leading match (key_map.rs:250-253).
    assert s.keys() == ["mid.t_embedder.mlp.0.bias", "t_embedder.timestep_embedder.linear_1.weight"]


def test_replace_rewrites_every_occurrence(tmp):
    p = tmp([("a.b.a.b", "F32", [1], f32(1))])
    s = WeightStore.open([p], KeyMap([(KeyMap.REPLACE, ["a.", "x."])]))
    assert s.keys() == ["x.b.x.b"]
    # An empty pattern matches around every character, as Rust's str::replace.
    s = WeightStore.open([p], KeyMap([(KeyMap.REPLACE, ["", "-"])]))
    assert s.keys() == ["-a-.-b-.-a-.-b-"]


def test_empty_require_any_prefix_passes_all(tmp):
    p = tmp([("k", "F32", [1], f32(1))])
    assert WeightStore.open([p], KeyMap([(KeyMap.REQUIRE_ANY_PREFIX, [])])).keys() == ["k"]


# ---------------------------------------------------------------------------
# Video-decoder map: renames and open-time value transforms
# (integration.rs:195-398, 831-848; the values are GPU tests)
# ---------------------------------------------------------------------------
def test_video_decoder_renames_and_drops(tmp):
    p = tmp([("vae.decoder.conv_in.weight", "F32", [2, 1], f32(0.5, 1.0)),
             ("vae.decoder.t_embedder.mlp.0.weight", "F32", [2, 1], f32(1, 2)),
             ("vae.decoder.t_embedder.mlp.2.bias", "F32", [2], f32(1, 2)),
             ("vae.decoder.coarse_up.weight", "F32", [1], f32(1)),
             ("vae.per_channel_statistics.mean", "F32", [2], f32(1, 2)),
             ("other.weight", "F32", [1], f32(1))])
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert s.keys() == ["conv_in.weight", "per_channel_statistics.mean",
                        "t_embedder.timestep_embedder.linear_1.weight",
                        "t_embedder.timestep_embedder.linear_2.bias", "type_emb"]
    # conv_in.weight [2, 1] -> a zero type_emb of 1 channel (store.rs:398-419).
    assert s.shape("type_emb") == [1] and s.dtype("type_emb") == "F32"


def test_type_emb_kept_when_present_or_no_conv_in(tmp):
    p = tmp([("decoder.conv_in.weight", "F32", [1, 3], f32(1, 2, 3)), ("decoder.type_emb", "BF16", [2],
                                                                         np.zeros(2, np.uint16))])
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert s.shape("type_emb") == [2] and s.dtype("type_emb") == "BF16"
    s = WeightStore.open([tmp([("decoder.x", "F32", [1], f32(1))])], KeyMap.video_decoder())
    assert not s.contains("type_emb")


def test_qkv_split_keys_shapes_and_scale_sibling(tmp):
    p = tmp([("vae.decoder.blocks.0.attn.qkv.weight", "F8_E4M3", [3, 1], np.array([0x38, 0x40, 0x44], np.uint8)),
             ("vae.decoder.blocks.0.attn.qkv.weight_scale", "F32", [1], f32(4.0)),
             ("vae.decoder.blocks.0.attn.qkv.bias", "F32", [6], np.arange(6, dtype=np.float32))])
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert not s.contains("blocks.0.attn.qkv.weight") and not s.contains("blocks.0.attn.qkv.weight_scale")
    for part in ("to_q", "to_k", "to_v"):
        assert s.shape(f"blocks.0.attn.{part}.weight") == [1, 1]
        assert s.dtype(f"blocks.0.attn.{part}.weight") == "F32"
        assert s.shape(f"blocks.0.attn.{part}.bias") == [2]
    with pytest.raises(lw.MissingKey):
        s.shape("blocks.0.attn.qkv.weight_scale")


def test_qkv_split_bad_dim_and_duplicates(tmp):
    p = tmp([("decoder.blocks.0.attn.qkv.weight", "F32", [5, 4], np.zeros(20, np.float32))])
    with pytest.raises(lw.QkvSplitDim, match="leading dim 5"):
        WeightStore.open([p], KeyMap.video_decoder())
    p = tmp([("decoder.a.qkv.weight", "F32", [3, 1], f32(1, 2, 3)), ("decoder.a.to_k.weight", "F32", [1, 1], f32(9))])
    with pytest.raises(lw.DuplicateKey):
        WeightStore.open([p], KeyMap.video_decoder())


def test_gate_fold_keys_and_errors(tmp):
    p = tmp([("vae.decoder.blocks.0.gate_msa", "F32", [1], f32(2.0)),
             ("vae.decoder.blocks.0.attn.proj.weight", "F8_E4M3", [1], np.array([0x38], np.uint8)),
             ("vae.decoder.blocks.0.attn.proj.weight_scale", "F32", [1], f32(4.0)),
             ("vae.decoder.blocks.0.attn.proj.bias", "F32", [2], f32(0.5, 1.5)),
             ("vae.decoder.blocks.0.gate_mlp", "F32", [], f32(3.0))])  # no target: just removed
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert s.keys() == ["blocks.0.attn.proj.bias", "blocks.0.attn.proj.weight"]
    assert s.dtype("blocks.0.attn.proj.weight") == "F32" and s.dtype("blocks.0.attn.proj.bias") == "F32"
    with pytest.raises(lw.MissingKey):
        s.shape("blocks.0.attn.proj.weight_scale")
    p = tmp([("decoder.b.gate_ctx", "F32", [2], f32(1, 2)), ("decoder.b.context_proj.weight", "F32", [1], f32(1))])
    with pytest.raises(lw.GateNotScalar):
        WeightStore.open([p], KeyMap.video_decoder())
    p = tmp([("decoder.b.gate_msa", "I32", [1], np.array([2], np.int32)), ("decoder.b.attn.proj.bias", "F32", [1], f32(1))])
    with pytest.raises(lw.UnsupportedDtype):
        WeightStore.open([p], KeyMap.video_decoder())


def test_value_transforms_run_only_when_asked(tmp):
    p = tmp([("a.qkv.weight", "F32", [3, 1], f32(1, 2, 3)), ("a.gate_msa", "F32", [1], f32(2))])
    assert WeightStore.open([p]).keys() == ["a.gate_msa", "a.qkv.weight"]
    assert WeightStore.open([p], KeyMap([(KeyMap.SPLIT_QKV, [])])).keys() == [
        "a.gate_msa", "a.to_k.weight", "a.to_q.weight", "a.to_v.weight"]
    assert WeightStore.open([p], KeyMap([(KeyMap.FOLD_GATES, [])])).keys() == ["a.qkv.weight"]


def test_fp8_scale_key_is_internal(tmp):
    p = tmp([("w", "F8_E4M3", [1], np.array([0x38], np.uint8)), ("w_scale", "F32", [1], f32(3.0))])
    s = WeightStore.open([p])
    assert not s.contains("w_scale") and s.keys() == ["w"]
    assert s.shape("w_scale") == [1]  # still addressable by shape (store.rs:462-467)


def test_non_fp8_scale_sibling_is_visible(tmp):
    p = tmp([("w", "F32", [1], f32(2.0)), ("w_scale", "F32", [1], f32(100.0))])
    s = WeightStore.open([p])
    assert s.contains("w_scale") and s.keys() == ["w", "w_scale"]


def test_duplicate_keys_across_files(tmp):
    a = tmp([("x", "F32", [1], f32(1))])
    b = tmp([("x", "F32", [1], f32(1))])
    with pytest.raises(lw.DuplicateKey):
        WeightStore.open([a, b])
    # A rename that makes two keys collide is a duplicate too.
    c = tmp([("p.x", "F32", [1], f32(1)), ("q.x", "F32", [1], f32(1))])
    with pytest.raises(lw.DuplicateKey):
        WeightStore.open([c], KeyMap([(KeyMap.REPLACE, ["p.", ""]), (KeyMap.REPLACE, ["q.", ""])]))


def test_multiple_files_merged_metadata_first_wins(tmp):
    a = tmp([("a.weight", "F32", [1], f32(1))], {"model_version": "2.5", "x": "first"})
    b = tmp([("b.weight", "F32", [1], f32(1))], {"x": "second", "y": "only-b"})
    s = WeightStore.open([a, b])
    assert s.contains("a.weight") and s.contains("b.weight")
    assert s.metadata("model_version") == "2.5"
    assert s.metadata("x") == "first" and s.metadata("y") == "only-b"
    assert s.metadata("absent") is None


def test_shape_and_dtype(tmp):
    p = tmp([("w", "F32", [2, 3], np.zeros(6, np.float32)), ("s", "BF16", [], np.zeros(1, np.uint16))])
    s = WeightStore.open([p])
    assert s.shape("w") == [2, 3] and s.dtype("w") == "F32"
    assert s.shape("s") == [] and s.dtype("s") == "BF16"
    with pytest.raises(lw.MissingKey):
        s.shape("nope")


def test_missing_file_is_io_error(tmp_path):
    with pytest.raises(lw.IoError):
        WeightStore.open([tmp_path / "absent.safetensors"])


def test_scope_contains(tmp):
    p = tmp([("transformer_blocks.0.attn.weight", "F32", [2], f32(1, 2)), ("other.weight", "F32", [2], f32(1, 2))])
    s = WeightStore.open([p])
    blk = s.scope("transformer_blocks.0")
    assert blk.contains("attn.weight") and not blk.contains("other.weight")
    assert blk.scope("attn").contains("weight")
    assert blk.scope("attn").full_key("weight") == "transformer_blocks.0.attn.weight"


# ---------------------------------------------------------------------------
# safetensors container rules
# ---------------------------------------------------------------------------
def raw_file(tmp_path, header_bytes, data=b"", hlen=None, name="raw.safetensors"):
    p = tmp_path / name
    n = len(header_bytes) if hlen is None else hlen
    p.write_bytes(struct.pack("<Q", n) + header_bytes + data)
    return p


def hdr(obj):
    return json.dumps(obj).encode()


@pytest.mark.parametrize("case", [
    "too_small", "too_large", "length_past_end", "not_utf8", "not_object_start", "bad_json", "not_object",
    "gap", "overlap", "size_mismatch", "incomplete_buffer", "trailing_data", "unknown_dtype",
    "bad_shape", "bad_offsets", "metadata_not_string", "duplicate_name", "float_shape",
])
def test_format_errors(tmp_path, case):
    t = {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}
    data = b"\0" * 8
    if case == "too_small":
        p = tmp_path / "x.safetensors"
        p.write_bytes(b"\1\0\0")
    elif case == "too_large":
        p = raw_file(tmp_path, b"{}", hlen=100_000_001)
    elif case == "length_past_end":
        p = raw_file(tmp_path, b"{}", hlen=64)
    elif case == "not_utf8":
        p = raw_file(tmp_path, b'{"\xff":1}')
    elif case == "not_object_start":
        p = raw_file(tmp_path, b' {"a":1}')
    elif case == "bad_json":
        p = raw_file(tmp_path, b'{"a":')
    elif case == "not_object":
        p = raw_file(tmp_path, b"{}")  # valid; replaced below
        p = raw_file(tmp_path, b"{ }x")
    elif case == "gap":
        p = raw_file(tmp_path, hdr({"a": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}), b"\0" * 12)
    elif case == "overlap":
        p = raw_file(tmp_path, hdr({"a": t, "b": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}),
                     b"\0" * 12)
    elif case == "size_mismatch":
        p = raw_file(tmp_path, hdr({"a": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]}}), data)
    elif case == "incomplete_buffer":
        p = raw_file(tmp_path, hdr({"a": t}), b"\0" * 4)
    elif case == "trailing_data":
        p = raw_file(tmp_path, hdr({"a": t}), b"\0" * 9)
    elif case == "unknown_dtype":
        p = raw_file(tmp_path, hdr({"a": {"dtype": "F7", "shape": [2], "data_offsets": [0, 8]}}), data)
    elif case == "bad_shape":
        p = raw_file(tmp_path, hdr({"a": {"dtype": "F32", "shape": [-2], "data_offsets": [0, 8]}}), data)
    elif case == "bad_offsets":
        p = raw_file(tmp_path, hdr({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0]}}), data)
    elif case == "metadata_not_string":
        p = raw_file(tmp_path, hdr({"__metadata__": {"k": 1}, "a": t}), data)
    elif case == "duplicate_name":
        p = raw_file(tmp_path, b'{"a":' + hdr(t) + b',"a":' + hdr(t) + b"}", data)
    elif case == "float_shape":
        p = raw_file(tmp_path, hdr({"a": {"dtype": "F32", "shape": [2.0], "data_offsets": [0, 8]}}), data)
    with pytest.raises(lw.InvalidTensorData):
        WeightStore.open([p])


def test_header_padding_escapes_and_empty_tensors(tmp_path):
    # Trailing spaces pad the header (the format allows it); names with JSON
    # escapes decode to their UTF-8 text; zero-element tensors take no bytes.
    h = ('{"__metadata__":{"note":"a\\"b\\u00e9"},"w\\u00e9\\n":{"dtype":"F32","shape":[2],'
         '"data_offsets":[0,8]},"e":{"dtype":"BF16","shape":[0,4],"data_offsets":[8,8]}}').encode() + b"    "
    p = raw_file(tmp_path, h, f32(1, 2).tobytes())
    s = WeightStore.open([p])
    assert s.keys() == ["e", "wé\n"]
    assert s.metadata("note") == 'a"bé'
    assert s.shape("e") == [0, 4]


def test_files_from_the_safetensors_package(tmp_path):
    """Files written by the `safetensors` package parse to the same names,
    dtypes, shapes and metadata."""
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file

    rng = np.random.default_rng(3)
    tensors = {
        "a.f32": torch.from_numpy(rng.standard_normal((3, 5)).astype(np.float32)),
        "b.bf16": torch.from_numpy(rng.standard_normal((7,)).astype(np.float32)).to(torch.bfloat16),
        "c.f16": torch.from_numpy(rng.standard_normal((2, 2, 2)).astype(np.float16)),
        "d.fp8": torch.from_numpy(rng.integers(0, 126, (4, 4), dtype=np.uint8)).view(torch.float8_e4m3fn),
        "e.fp8": torch.from_numpy(rng.integers(0, 120, (4, 8), dtype=np.uint8)).view(torch.float8_e5m2),
        "f.i64": torch.arange(3),
        "g.scalar": torch.tensor(1.5),
    }
    p = tmp_path / "pkg.safetensors"
    save_file(tensors, str(p), metadata={"format": "pt", "k": "v"})
    s = WeightStore.open([p])
    names = {"F32": torch.float32, "BF16": torch.bfloat16, "F16": torch.float16, "F8_E4M3": torch.float8_e4m3fn,
             "F8_E5M2": torch.float8_e5m2, "I64": torch.int64}
    assert s.keys() == sorted(tensors)
    for k, t in tensors.items():
        assert s.shape(k) == list(t.shape)
        assert names[s.dtype(k)] == t.dtype
    assert s.metadata("k") == "v"


# ---------------------------------------------------------------------------
# LoRA files and merge_lora (integration.rs:460-700, 804-829)
# ---------------------------------------------------------------------------
def base_2x2(tmp, key="layer.weight"):
    return tmp([(key, "F32", [2, 2], f32(1, 0, 0, 1))])


def test_lora_merge_basic_report(tmp):
    store = WeightStore.open([base_2x2(tmp)])
    lf = LoraFile.open(tmp([("layer.lora_A.weight", "F32", [1, 2], f32(1, 2)),
                            ("layer.lora_B.weight", "F32", [2, 1], f32(3, 4))]))
    rep = store.merge_lora(lf, 1.0)
    assert rep.matched_keys == ["layer.weight"] and rep.unmatched_lora_keys == []
    assert store.deltas("layer.weight") == [(1, 1.0)]


def test_lora_merge_with_alpha(tmp):
    store = WeightStore.open([base_2x2(tmp, "w.weight")])
    lf = LoraFile.open(tmp([("w.lora_A.weight", "F32", [1, 2], f32(1, 2)),
                            ("w.lora_B.weight", "F32", [2, 1], f32(3, 4)),
                            ("w.alpha", "F32", [1], f32(2.0))]))
    store.merge_lora(lf, 1.0)
    assert store.deltas("w.weight") == [(1, 2.0)]


@pytest.mark.parametrize("strength,alpha,alpha_dtype,rank", [
    (0.75, 4.0, "F32", 2), (1.0, None, None, 64), (0.5, None, None, 128), (0.3, 7.0, "BF16", 3),
    (-1.25, 3.0, "F16", 5), (0.0, 2.0, "F32", 2), (-0.0, None, None, 1), (1e-3, 0.1, "F32", 7),
])
def test_lora_coefficient_matches_oracle(tmp, strength, alpha, alpha_dtype, rank):
    """coeff = strength.mul_add(alpha / rank, 0) with alpha's exact widening
    (store.rs:605-615), bit for bit against the oracle."""
    store = WeightStore.open([tmp([("w.weight", "F32", [2, 3], np.zeros(6, np.float32))])])
    ts = [("w.lora_A.weight", "F32", [rank, 3], np.zeros(rank * 3, np.float32)),
          ("w.lora_B.weight", "F32", [2, rank], np.zeros(2 * rank, np.float32))]
    widened = None
    if alpha is not None:
        if alpha_dtype == "F32":
            raw = f32(alpha)
        else:
            raw = synth.bf16_from_f64([alpha]) if alpha_dtype == "BF16" else np.array([alpha], np.float16).view(np.uint16)
        ts.append(("w.alpha", alpha_dtype, [1], raw))
        widened = float(O.decode(raw, O.DTYPE_CODES[alpha_dtype])[0])
    store.merge_lora(LoraFile.open(tmp(ts)), strength)
    (r, c), = store.deltas("w.weight")
    want = np.float32(O.lora_coeff(strength, widened, rank))
    assert r == rank
    assert np.float32(c).view(np.uint32) == want.view(np.uint32)


def test_empty_alpha_defaults_to_rank(tmp):
    store = WeightStore.open([tmp([("w.weight", "F32", [2, 3], np.zeros(6, np.float32))])])
    lf = LoraFile.open(tmp([("w.lora_A.weight", "F32", [4, 3], np.zeros(12, np.float32)),
                            ("w.lora_B.weight", "F32", [2, 4], np.zeros(8, np.float32)),
                            ("w.alpha", "F32", [0], np.zeros(0, np.float32))]))
    store.merge_lora(lf, 0.5)
    assert store.deltas("w.weight") == [(4, 0.5)]


def test_lora_merges_stack_in_call_order(tmp):
    store = WeightStore.open([base_2x2(tmp, "w.weight")])
    first = LoraFile.open(tmp([("w.lora_A.weight", "F32", [1, 2], f32(1, 2)),
                               ("w.lora_B.weight", "F32", [2, 1], f32(3, 4))]))
    second = LoraFile.open(tmp([("w.lora_A.weight", "F32", [2, 2], f32(1, 0, 0, 1)),
                                ("w.lora_B.weight", "F32", [2, 2], f32(2, 0, 0, -2))]))
    store.merge_lora(first, 1.0)
    store.merge_lora(second, 0.5)
    # The store keeps the files mapped: closing them does not drop the deltas.
    first.close()
    second.close()
    assert store.deltas("w.weight") == [(1, 1.0), (2, 0.5)]


def test_lora_unmatched_keys_reported(tmp):
    store = WeightStore.open([tmp([("present.weight", "F32", [1], f32(1))])])
    lf = LoraFile.open(tmp([(f"{k}.lora_{x}.weight", "F32", [1, 1], f32(1)) for k in ("present", "absent")
                            for x in "AB"]))
    rep = store.merge_lora(lf, 1.0)
    assert rep.matched_keys == ["present.weight"]
    assert rep.unmatched_lora_keys == ["absent.lora_A.weight"]


def test_lora_missing_b_is_unmatched(tmp):
    store = WeightStore.open([tmp([("a.weight", "F32", [1, 1], f32(1)), ("b.weight", "F32", [1, 1], f32(1))])])
    lf = LoraFile.open(tmp([("a.lora_A.weight", "F32", [1, 1], f32(1)), ("a.lora_B.weight", "F32", [1, 1], f32(1)),
                            ("b.lora_A.weight", "F32", [1, 1], f32(1))]))
    rep = store.merge_lora(lf, 1.0)
    assert rep.matched_keys == ["a.weight"] and rep.unmatched_lora_keys == ["b.lora_A.weight"]


def test_lora_all_unmatched_errors_and_leaves_store_unchanged(tmp):
    store = WeightStore.open([tmp([("present.weight", "F32", [1], f32(1))])])
    lf = LoraFile.open(tmp([("absent.lora_A.weight", "F32", [1, 1], f32(1)),
                            ("absent.lora_B.weight", "F32", [1, 1], f32(1))]))
    with pytest.raises(lw.NoLoraMatches):
        store.merge_lora(lf, 1.0)
    # A file with no lora_A keys matches nothing and is not an error.
    rep = store.merge_lora(LoraFile.open(tmp([("x", "F32", [1], f32(1))])), 1.0)
    assert rep.matched_keys == [] and rep.unmatched_lora_keys == []


def test_lora_decode_error_is_not_reported_as_unmatched(tmp):
    store = WeightStore.open([tmp([("layer.weight", "F32", [1, 1], f32(0))])])
    lf = LoraFile.open(tmp([("layer.lora_A.weight", "I32", [1, 1], np.array([7], np.int32)),
                            ("layer.lora_B.weight", "F32", [1, 1], f32(1))]))
    with pytest.raises(lw.UnsupportedDtype, match="layer.lora_A.weight"):
        store.merge_lora(lf, 1.0)


def test_lora_shape_mismatch(tmp):
    store = WeightStore.open([tmp([("layer.weight", "F32", [2, 3], np.zeros(6, np.float32))])])
    lf = LoraFile.open(tmp([("layer.lora_A.weight", "F32", [1, 3], f32(1, 2, 3)),
                            ("layer.lora_B.weight", "F32", [4, 1], np.zeros(4, np.float32))]))
    with pytest.raises(lw.LoraShapeMismatch):
        store.merge_lora(lf, 1.0)
    assert store.deltas("layer.weight") == []


@pytest.mark.parametrize("a_shape,b_shape,err", [
    ([2, 3], [2, 3], lw.LoraRankMismatch), ([0, 3], [2, 0], lw.LoraRankMismatch),
    # rank_a = A.shape[0] = 3 = B.shape[1]; the missing A.shape[1] then fails the
    # shape check (store.rs:593-603).
    ([3], [2, 3], lw.LoraShapeMismatch),
])
def test_lora_rank_mismatch(tmp, a_shape, b_shape, err):
    store = WeightStore.open([tmp([("layer.weight", "F32", [2, 3], np.zeros(6, np.float32))])])
    na, nb = int(np.prod(a_shape)), int(np.prod(b_shape))
    lf = LoraFile.open(tmp([("layer.lora_A.weight", "F32", a_shape, np.zeros(na, np.float32)),
                            ("layer.lora_B.weight", "F32", b_shape, np.zeros(nb, np.float32))]))
    with pytest.raises(err):
        store.merge_lora(lf, 1.0)


def test_one_dimensional_base_takes_in_features_one(tmp):
    # store.rs:593-599: a 1-D base has in_features = 1.
    store = WeightStore.open([tmp([("b.weight", "F32", [3], f32(1, 2, 3))])])
    lf = LoraFile.open(tmp([("b.lora_A.weight", "F32", [1, 1], f32(2)), ("b.lora_B.weight", "F32", [3, 1], f32(1, 1, 1))]))
    assert store.merge_lora(lf, 1.0).matched_keys == ["b.weight"]


def test_ic_layout(tmp):
    lf = LoraFile.open(tmp([("d.lora_A.weight", "F32", [1, 1], f32(1))],
                           {"reference_downscale_factor": "2", "reference_temporal_scale_factor": " +4 "}))
    assert lf.ic_layout() == (2, 4)
    assert LoraFile.open(tmp([("d.lora_A.weight", "F32", [1, 1], f32(1))])).ic_layout() == (1, 1)
    # Unparsable values fall back to 1; a stored zero is rejected.
    assert LoraFile.open(tmp([("d", "F32", [1], f32(1))], {"reference_downscale_factor": "x2"})).ic_layout() == (1, 1)
    with pytest.raises(lw.InvalidArgument):
        LoraFile.open(tmp([("d", "F32", [1], f32(1))], {"reference_temporal_scale_factor": "0"})).ic_layout()


def test_lora_file_accessors_and_read_f32(tmp):
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 1 << 16, 64, dtype=np.uint16)
    bits[:4] = [0x7C00, 0xFC01, 0x7E55, 0x0001]  # f16 Inf, NaN (payload), qNaN, subnormal
    fp8 = np.arange(256, dtype=np.uint8)
    ts = [("z.f32", "F32", [2, 3], rng.standard_normal(6).astype(np.float32)),
          ("y.bf16", "BF16", [64], bits), ("x.f16", "F16", [8, 8], bits),
          ("w.e4m3", "F8_E4M3", [256], fp8), ("v.e5m2", "F8_E5M2", [16, 16], fp8),
          ("u.i32", "I32", [1], np.array([1], np.int32))]
    lf = LoraFile.open(tmp(ts, {"m": "1"}))
    assert lf.tensor_names() == sorted(n for n, *_ in ts)
    assert lf.tensor_info("x.f16") == ("F16", (8, 8)) and lf.tensor_info("nope") is None
    assert lf.metadata("m") == "1" and lf.metadata("q") is None
    assert lf.read_f32("nope") is None
    for name, dt, shape, raw in ts[:-1]:
        shp, got = lf.read_f32(name)
        want = O.decode(raw, O.DTYPE_CODES[dt])
        assert shp == shape
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
    with pytest.raises(lw.UnsupportedDtype):
        lf.read_f32("u.i32")


# ---------------------------------------------------------------------------
# Synthetic checkpoints (the whole-model workload's input files)
# ---------------------------------------------------------------------------
def test_synthetic_model_and_lora_files(tmp_path):
    m, l = tmp_path / "m.safetensors", tmp_path / "l.safetensors"
    synth.write_model(m, 77, 1, variant=1, threads=4)
    synth.write_lora(l, 78, 1, 32, variant=1, threads=4)
    layout = synth.model_layout(1, 1)
    s = WeightStore.open([m], KeyMap.transformer())
    assert s.keys() == sorted(k for k, *_ in layout)
    assert s.metadata("seed") == "77"
    for key, fmt, sm, r, c in layout:
        assert s.shape(key) == [r, c]
        assert s.dtype(key) == ("F8_E4M3" if fmt == synth.E4M3FN else "F8_E5M2")
        assert s.shape(key + "_scale") == ([r] if sm == synth.SCALE_ROW else [])
        assert not s.contains(key + "_scale")
    rep = s.merge_lora(LoraFile.open(l), 1.0)
    assert rep.matched_keys == sorted(k for k, *_ in layout) and rep.unmatched_lora_keys == []
    # The file bytes are the generator's (checked with an independent reader).
    tensors, meta = st_io.read(m)
    key, fmt, sm, r, c = layout[8]  # FFN up, e5m2, row scales
    rows = np.array([0, 1, r - 1])
    w, sc = synth.model_rows(77, key, fmt, sm, rows, c, r)
    raw = tensors[synth.CKPT_PREFIX + key][2].reshape(r, c)
    assert np.array_equal(raw[rows], w)
    assert np.array_equal(tensors[synth.CKPT_PREFIX + key + "_scale"][2], sc)
    lt, _ = st_io.read(l)
    b, a = synth.lora_factors_rows(78, key, 32, rows, r, c)
    assert np.array_equal(lt[key[:-7] + ".lora_A.weight"][2].reshape(32, c), a)
    assert np.array_equal(lt[key[:-7] + ".lora_B.weight"][2].reshape(r, 32)[rows], b)
