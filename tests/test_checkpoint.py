"""consumer_int8.checkpoint and the group32 encoding (CPU).

Mirrors tests/test_quantization.py:27-63 of the reference (group32 round trip with K
tails, non-finite rejection, the tensor-name classes) and checks `encode` end to end on
a synthetic snapshot with the reference's geometry in its config and small tensors:
codes and scales against the oracle, the tensor inventory, shard ownership, report,
index, copied files, the published config, every refusal of
src/consumer_int8/checkpoint.py:59-130, and the debiasing loader.
"""

import hashlib
import json

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from oracle import oracle as O


# ------------------------------------------------------------------ group32

@pytest.mark.parametrize("k", [32, 72, 128, 4304])
def test_group32_roundtrip_keeps_unaligned_vision_tail(k):
    """tests/test_quantization.py:27-36."""
    from consumer_int8.quantization import dequantize_group32, quantize_group32

    weight = torch.randn(7, k, generator=torch.Generator().manual_seed(4))
    weight[0] = 0
    codes, scale = quantize_group32(weight)
    restored = dequantize_group32(codes, scale)
    assert codes.shape == weight.shape and codes.dtype == torch.int8
    assert scale.shape == (7, (k + 31) // 32) and scale.dtype == torch.float32
    bound = scale.repeat_interleave(32, dim=1)[:, :k] / 2 + 1e-6
    assert ((restored - weight).abs() <= bound).all()
    assert (scale[0] == 1).all() and not codes[0].any()


@pytest.mark.parametrize("name", ["quantize_channel", "quantize_group32"])
def test_nonfinite_weights_are_rejected(name):
    """tests/test_quantization.py:39-42."""
    from consumer_int8 import quantization

    with pytest.raises(ValueError, match="non-finite"):
        getattr(quantization, name)(torch.tensor([[float("nan")]]))


@pytest.mark.parametrize("k", [1, 31, 33, 4304])
def test_group32_matches_oracle(k):
    from consumer_int8.quantization import quantize_group32

    rng = np.random.default_rng(k)
    w = (rng.standard_normal((9, k)) * 0.05).astype(np.float32)
    w[2] = 0
    w[4, : min(k, 40)] = np.float32(3e-39)  # subnormal block maxima
    codes, scale = quantize_group32(torch.from_numpy(w))
    ocodes, oscale = O.quantize_group32(w)
    assert np.array_equal(codes.numpy(), ocodes)
    assert np.array_equal(scale.numpy(), oscale)


def test_group32_oracle_known_answer_and_exact_rounding():
    """A block with maximum 127 has scale 1, so codes are rne of the values (63.5 -> 64,
    -2.5 -> -2); a zero block has scale 1; the tail block is scaled by its own maximum."""
    from fractions import Fraction

    from tests import exact as E

    w = np.zeros((2, 40), np.float32)
    w[0, :4] = [127.0, 63.5, -2.5, 0.49]
    w[0, 32:35] = [0.5, -0.25, 0.125]
    codes, scale = O.quantize_group32(w)
    assert scale.tolist() == [[1.0, np.float32(0.5 / 127)], [1.0, 1.0]]
    assert codes[0, :4].tolist() == [127, 64, -2, 0]
    for t, v in zip(range(32, 35), (0.5, -0.25, 0.125)):
        s = E.f32(Fraction(0.5) / 127)
        assert codes[0, t] == E.rne_int(E.f32(Fraction(v) / s))
    assert not codes[1].any()


# ------------------------------------------------------------------ names

@pytest.mark.parametrize(
    "name,expected",
    [
        ("model.language_model.layers.0.linear_attn.in_proj_qkv.weight", "channel_uint8"),
        ("model.language_model.layers.0.linear_attn.in_proj_a.weight", "passthrough"),
        ("model.language_model.layers.0.linear_attn.conv1d.weight", "passthrough"),
        ("model.language_model.embed_tokens.weight", "passthrough"),
        ("lm_head.weight", "passthrough"),
        ("mtp.fc.weight", "channel_uint8"),
        ("mtp.layers.0.mlp.gate_proj.weight", "channel_uint8"),
        ("model.visual.blocks.0.mlp.linear_fc2.weight", "group32_int8"),
        ("model.visual.patch_embed.proj.weight", "passthrough"),
        # beyond the reference's table
        ("model.language_model.layers.63.mlp.down_proj.weight", "channel_uint8"),
        ("model.language_model.layers.7.self_attn.o_proj.weight", "channel_uint8"),
        ("model.language_model.layers.7.self_attn.o_proj.bias", "passthrough"),
        ("model.language_model.layers.7.self_attn.q_norm.weight", "passthrough"),
        ("model.language_model.layers.x.mlp.up_proj.weight", "passthrough"),
        ("xmodel.language_model.layers.0.mlp.up_proj.weight", "passthrough"),
        ("model.visual.blocks.3.attn.qkv.weight", "group32_int8"),
        ("model.visual.merger.linear_fc1.weight", "group32_int8"),
        ("model.visual.merger.linear_fc3.weight", "passthrough"),
        ("mtp.fc.weight_scale_inv", "passthrough"),
    ],
)
def test_encoding_preserves_gates_embeddings_and_convolutions(name, expected):
    """tests/test_quantization.py:45-63, plus near misses."""
    from consumer_int8.checkpoint import encoding_for

    assert encoding_for(name) == expected


# ------------------------------------------------------------------ encode

LAYOUT = {
    "model-00001-of-00002.safetensors": {
        "model.language_model.embed_tokens.weight": (64, 32),
        "model.language_model.layers.0.mlp.down_proj.weight": (48, 96),
        "model.language_model.layers.0.mlp.gate_proj.weight": (96, 48),
        "model.language_model.layers.0.linear_attn.conv1d.weight": (8, 1, 4),
        "model.language_model.layers.0.linear_attn.in_proj_qkv.weight": (80, 48),
        "model.language_model.norm.weight": (48,),
    },
    "model-00002-of-00002.safetensors": {
        "mtp.fc.weight": (48, 96),
        "mtp.layers.0.self_attn.k_proj.weight": (32, 48),
        "model.visual.blocks.0.attn.qkv.weight": (72, 40),
        "model.visual.patch_embed.proj.weight": (16, 3, 2, 2),
        "lm_head.weight": (64, 48),
    },
}


def make_snapshot(root, layout=LAYOUT, config=None, dtype=torch.bfloat16, seed=0):
    root.mkdir(parents=True, exist_ok=True)
    gen = torch.Generator().manual_seed(seed)
    weight_map = {}
    tensors = {}
    for shard, entries in layout.items():
        out = {}
        for name, shape in entries.items():
            out[name] = (torch.randn(shape, generator=gen) * 0.02).to(dtype)
            weight_map[name] = shard
        save_file(out, root / shard, metadata={"format": "pt"})
        tensors.update(out)
    cfg = config or {"model_type": "qwen3_5",
                     "text_config": {"hidden_size": 5120, "num_hidden_layers": 64}}
    (root / "config.json").write_text(json.dumps(cfg))
    (root / "model.safetensors.index.json").write_text(
        json.dumps({"metadata": {"total_size": 0}, "weight_map": weight_map}))
    (root / "tokenizer.json").write_text("{}")
    (root / "chat_template.jinja").write_text("{{ messages }}")
    (root / "crc32.txt").write_text("0")
    (root / "LICENSE").write_text("license")
    (root / "notes.md").write_text("not copied")
    return tensors


def read_all(directory):
    index = json.loads((directory / "model.safetensors.index.json").read_text())
    out = {}
    for name, shard in index["weight_map"].items():
        with safe_open(directory / shard, framework="pt", device="cpu") as handle:
            out[name] = handle.get_tensor(name)
    return index, out


def bf16_bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def test_encode_end_to_end(tmp_path):
    from consumer_int8 import __version__
    from consumer_int8.checkpoint import SOURCE_REPO, encode, encoding_for

    src, dst = tmp_path / "src", tmp_path / "dst"
    tensors = make_snapshot(src)
    report = encode(src, dst, source_revision="rev123")
    index, out = read_all(dst)

    expected_names = set()
    for name, tensor in tensors.items():
        enc = encoding_for(name)
        assert report["tensors"][name]["encoding"] == enc
        assert report["tensors"][name]["shape"] == list(tensor.shape)
        if enc == "passthrough":
            assert torch.equal(out[name], tensor)
            assert report["tensors"][name]["stored_dtype"] == "torch.bfloat16"
            expected_names.add(name)
            continue
        w = tensor.float().numpy()
        stem = name.removesuffix(".weight")
        if enc == "channel_uint8":
            codes, scale = O.quantize_channel(w)
            assert np.array_equal(out[name].numpy(), codes)
            assert np.array_equal(bf16_bits(out[stem + ".weight_scale_inv"]), scale)
            restored = O.dequantize_channel(codes, scale)
            expected_names |= {name, stem + ".weight_scale_inv"}
        else:
            codes, scale = O.quantize_group32(w)
            assert np.array_equal(out[name].numpy(), codes)
            assert np.array_equal(out[stem + ".weight_scale"].numpy(), scale)
            restored = O.dequantize_group32(codes, scale)
            expected_names |= {name, stem + ".weight_scale"}
        err = restored.astype(np.float64) - w
        rec = report["tensors"][name]
        assert rec["rmse"] == pytest.approx(np.sqrt(np.mean(err**2)), rel=1e-5)
        assert rec["max_abs_error"] == pytest.approx(np.abs(err).max(), rel=1e-6)
    assert set(out) == expected_names

    # shard ownership follows the source, scales beside their weights
    src_index = json.loads((src / "model.safetensors.index.json").read_text())
    for name, shard in index["weight_map"].items():
        base = name.replace(".weight_scale_inv", ".weight").replace(".weight_scale", ".weight")
        assert shard == src_index["weight_map"][base]
    total = sum(t.numel() * t.element_size() for t in out.values())
    assert index["metadata"]["total_size"] == total == report["total_tensor_bytes"]
    for shard, rec in report["shards"].items():
        assert rec["sha256"] == hashlib.sha256((dst / shard).read_bytes()).hexdigest()
        assert rec["tensor_count"] == sum(1 for s in index["weight_map"].values() if s == shard)

    assert report["status"] == "encoded_unvalidated"
    assert report["format_version"] == 1 and report["encoder_version"] == __version__
    assert report["source_repo"] == SOURCE_REPO and report["source_revision"] == "rev123"
    assert json.loads((dst / "encoding_report.json").read_text()) == report

    config = json.loads((dst / "config.json").read_text())
    qc = config["quantization_config"]
    assert qc["quant_method"] == "qwen_int8" and qc["format_version"] == 1
    assert qc["weight_strategy"] == "channel_uint8"
    assert qc["vision_weight_strategy"] == "group32_int8"
    assert qc["source_revision"] == "rev123"
    assert qc["quantized_modules"] == {
        n.removesuffix(".weight"): encoding_for(n) for n in tensors
        if encoding_for(n) != "passthrough"}

    copied = {p.name for p in dst.iterdir()}
    assert {"tokenizer.json", "chat_template.jinja", "LICENSE"} <= copied
    assert "crc32.txt" not in copied and "notes.md" not in copied
    assert not [p for p in dst.iterdir() if p.name.endswith(".tmp")]


def test_encode_refusals(tmp_path):
    from consumer_int8.checkpoint import encode

    src = tmp_path / "src"
    make_snapshot(src)
    with pytest.raises(ValueError, match="Source and destination must differ"):
        encode(src, src, source_revision="r")
    busy = tmp_path / "busy"
    busy.mkdir()
    (busy / "x").write_text("x")
    with pytest.raises(ValueError, match="Destination must be empty"):
        encode(src, busy, source_revision="r")

    def variant(name, config=None, layout=LAYOUT):
        root = tmp_path / name
        make_snapshot(root, layout=layout, config=config)
        return root

    quantized = {"model_type": "qwen3_5", "quantization_config": {"x": 1},
                 "text_config": {"hidden_size": 5120, "num_hidden_layers": 64}}
    for cfg in ({"model_type": "llama", "text_config": {"hidden_size": 5120, "num_hidden_layers": 64}},
                quantized):
        with pytest.raises(ValueError, match="Expected an unquantized Qwen3.5"):
            encode(variant(f"c{len(str(cfg))}", cfg), tmp_path / "o1", source_revision="r")
    small = {"model_type": "qwen3_5", "text_config": {"hidden_size": 4096, "num_hidden_layers": 64}}
    with pytest.raises(ValueError, match="Qwen3.8-27B geometry"):
        encode(variant("small", small), tmp_path / "o2", source_revision="r")
    no_mtp = {s: {n: v for n, v in e.items() if not n.startswith("mtp.")} for s, e in LAYOUT.items()}
    with pytest.raises(ValueError, match="must contain MTP weights"):
        encode(variant("nomtp", layout=no_mtp), tmp_path / "o3", source_revision="r")
    no_vis = {s: {n: v for n, v in e.items() if not n.startswith("model.visual.")}
              for s, e in LAYOUT.items()}
    with pytest.raises(ValueError, match="must contain vision weights"):
        encode(variant("novis", layout=no_vis), tmp_path / "o4", source_revision="r")

    # index and shard disagree
    bad = variant("bad")
    index = json.loads((bad / "model.safetensors.index.json").read_text())
    index["weight_map"]["lm_head.weight"] = "model-00001-of-00002.safetensors"
    (bad / "model.safetensors.index.json").write_text(json.dumps(index))
    with pytest.raises(ValueError, match="Index and shard disagree"):
        encode(bad, tmp_path / "o5", source_revision="r")
    # layout refusals come before anything is written
    assert not (tmp_path / "o5").exists()
    # a shard name with a directory part
    sub = variant("sub")
    index = json.loads((sub / "model.safetensors.index.json").read_text())
    index["weight_map"] = {n: ("../" + s if s.endswith("1-of-00002.safetensors") else s)
                           for n, s in index["weight_map"].items()}
    (sub / "model.safetensors.index.json").write_text(json.dumps(index))
    with pytest.raises(ValueError, match="Invalid shard filename"):
        encode(sub, tmp_path / "o6", source_revision="r")
    # a scale tensor already present in the source
    clash_layout = {s: dict(e) for s, e in LAYOUT.items()}
    clash_layout["model-00002-of-00002.safetensors"]["mtp.fc.weight_scale_inv"] = (48,)
    with pytest.raises(ValueError, match="Scale name already exists: mtp.fc.weight_scale_inv"):
        encode(variant("clash", layout=clash_layout), tmp_path / "o7", source_revision="r")
    assert not (tmp_path / "o7").exists()
    # non-finite weights are refused by the encoders
    nan = variant("nan")
    shard = "model-00002-of-00002.safetensors"
    with safe_open(nan / shard, framework="pt", device="cpu") as h:
        tensors = {n: h.get_tensor(n) for n in h.keys()}
    tensors["mtp.fc.weight"][0, 0] = float("inf")
    save_file(tensors, nan / shard, metadata={"format": "pt"})
    with pytest.raises(ValueError, match="non-finite"):
        encode(nan, tmp_path / "o8", source_revision="r")
    assert not (tmp_path / "o8" / "config.json").exists()


def test_load_channel_linear_debiases(tmp_path):
    from consumer_int8.checkpoint import encode, load_channel_linear

    src, dst = tmp_path / "src", tmp_path / "dst"
    tensors = make_snapshot(src)
    encode(src, dst, source_revision="r")
    module = "model.language_model.layers.0.mlp.down_proj"
    codes, scale = O.quantize_channel(tensors[module + ".weight"].float().numpy())
    w, s = load_channel_linear(dst, module, device="cpu")
    assert w.dtype == torch.int8
    assert np.array_equal(w.numpy(), (codes.astype(np.int16) - 128).astype(np.int8))
    assert np.array_equal(bf16_bits(s), scale)
    wb, _ = load_channel_linear(dst, module, device="cpu", signed=False)
    assert wb.dtype == torch.uint8 and np.array_equal(wb.numpy(), codes)
    with pytest.raises(ValueError, match="Not a channel_uint8 module"):
        load_channel_linear(dst, "model.visual.blocks.0.attn.qkv", device="cpu")


def test_command_line(tmp_path):
    from consumer_int8.checkpoint import main

    src, dst = tmp_path / "src", tmp_path / "dst"
    make_snapshot(src)
    main([str(src), str(dst), "--source-revision", "cli", "--threads", "2"])
    assert json.loads((dst / "config.json").read_text())["quantization_config"]["source_revision"] == "cli"
