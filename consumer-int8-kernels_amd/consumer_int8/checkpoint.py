"""Channel-UINT8 checkpoint encoding and loading for the INT8 linear layers.

`encode` converts an unquantized Qwen3.8-27B safetensors snapshot into the reference's
published encoding (src/consumer_int8/checkpoint.py:58-171): the language-model and MTP
linear weights become biased UINT8 codes plus BF16 `*.weight_scale_inv` channel scales,
the vision tower's linear weights become signed INT8 plus FP32 `*.weight_scale` group
scales, and every other tensor passes through. Shard ownership, the tensor inventory,
the per-tensor error report, the index and the `quantization_config` are those of the
reference, and the same inputs are refused with the same messages. `device` selects
where the quantization arithmetic runs: "cuda" encodes on the MI355X with results
bit-identical to the host's (the codes and scales are IEEE FP32 operations with one
correct rounding each); the report's error statistics are reductions and may differ in
their last bits.

`load_channel_linear` is the loading side, for the ops of this package: it reads one
channel-UINT8 layer back onto a device, debiased to signed INT8 for fused_channel_mm
(`signed=True`) or left biased for channel_mm.

Command line: `python -m consumer_int8.checkpoint SOURCE DESTINATION
[--source-revision REV] [--threads N] [--device cpu|cuda]`, the reference's
`consumer-int8-encode` (pyproject.toml:23-24).
"""

from __future__ import annotations

import argparse
import hashlib
import json
import re
import shutil
from pathlib import Path

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from . import __version__
from .quantization import (
    dequantize_channel,
    dequantize_group32,
    quantize_channel,
    quantize_group32,
)

SOURCE_REPO = "Qwen/Qwen3.8-27B"
SOURCE_REVISION = "1d4bf0f2ff6012fd82039f2fa52739d0dd7c60c0"

# Tensor-name classes (src/consumer_int8/checkpoint.py:26-33, 36-41): the linear layers
# of the language model and the MTP head, and the vision tower's attention, MLP and
# merger projections.
_LAYER_PREFIX = r"(?:model\.language_model|mtp)\.layers\.\d+\."
_CHANNEL_MODULES = (
    "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj",
    "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
    "linear_attn.in_proj_qkv", "linear_attn.in_proj_z", "linear_attn.out_proj",
)
_CHANNEL_NAME = re.compile(
    _LAYER_PREFIX + "(?:" + "|".join(re.escape(m) for m in _CHANNEL_MODULES) + r")\.weight"
)
_VISION_NAME = re.compile(
    r"model\.visual\.(?:blocks\.\d+\.(?:attn\.qkv|attn\.proj|mlp\.linear_fc1|mlp\.linear_fc2)"
    r"|merger\.linear_fc1|merger\.linear_fc2)\.weight"
)

_COPIED_SUFFIXES = {".json", ".txt", ".jinja"}
_NOT_COPIED = {"config.json", "model.safetensors.index.json", "crc32.txt"}


def encoding_for(name: str) -> str:
    """"channel_uint8", "group32_int8" or "passthrough" for a checkpoint tensor name
    (src/consumer_int8/checkpoint.py:36-41)."""
    if name == "mtp.fc.weight" or _CHANNEL_NAME.fullmatch(name):
        return "channel_uint8"
    if _VISION_NAME.fullmatch(name):
        return "group32_int8"
    return "passthrough"


def scale_name_for(name: str, encoding: str) -> str:
    """Name of the scale tensor stored beside an encoded weight (:105, :109)."""
    stem = name.removesuffix(".weight")
    return stem + (".weight_scale_inv" if encoding == "channel_uint8" else ".weight_scale")


def _sha256(path: Path) -> str:
    digest = hashlib.sha256()
    with path.open("rb") as stream:
        while block := stream.read(8 << 20):
            digest.update(block)
    return digest.hexdigest()


def _publish_json(path: Path, value: dict) -> None:
    """Write through a temporary file and rename, so readers never see half a file."""
    pending = path.with_name(path.name + ".tmp")
    pending.write_text(json.dumps(value, indent=2) + "\n")
    pending.replace(path)


def _check_source(source: Path, destination: Path) -> tuple[dict, dict]:
    # src/consumer_int8/checkpoint.py:59-76
    if source.resolve() == destination.resolve():
        raise ValueError("Source and destination must differ")
    if destination.exists() and any(destination.iterdir()):
        raise ValueError("Destination must be empty; partial conversions are not models")
    config = json.loads((source / "config.json").read_text())
    if config.get("model_type") != "qwen3_5" or config.get("quantization_config"):
        raise ValueError("Expected an unquantized Qwen3.5 architecture checkpoint")
    text = config["text_config"]
    if (text["hidden_size"], text["num_hidden_layers"]) != (5120, 64):
        raise ValueError("This encoding manifest targets Qwen3.8-27B geometry")
    weight_map = json.loads((source / "model.safetensors.index.json").read_text())["weight_map"]
    if not any(name.startswith("mtp.") for name in weight_map):
        raise ValueError("The full checkpoint must contain MTP weights")
    if not any(name.startswith("model.visual.") for name in weight_map):
        raise ValueError("The full checkpoint must contain vision weights")
    return config, weight_map


def _encode_tensor(name: str, weight: torch.Tensor, device: str, source_names) -> tuple[dict, dict]:
    """Encoded tensors of one source tensor and its report record (:97-118)."""
    encoding = encoding_for(name)
    record = {"shape": list(weight.shape), "encoding": encoding}
    if encoding == "passthrough":
        tensors = {name: weight}
    else:
        on_device = weight.to(device)
        if encoding == "channel_uint8":
            codes, scales = quantize_channel(on_device)
            restored = dequantize_channel(codes, scales)
        else:
            codes, scales = quantize_group32(on_device)
            restored = dequantize_group32(codes, scales)
        scale_name = scale_name_for(name, encoding)
        if scale_name in source_names:
            raise ValueError(f"Scale name already exists: {scale_name}")
        error = restored - on_device.float()
        record["rmse"] = error.square().mean().sqrt().item()
        record["max_abs_error"] = error.abs().max().item()
        tensors = {name: codes.cpu(), scale_name: scales.cpu()}
    record["stored_dtype"] = str(tensors[name].dtype)
    return tensors, record


def encode(source: Path, destination: Path, *, source_revision: str, device: str = "cpu") -> dict:
    """Encode the checkpoint at `source` into the empty directory `destination`; returns
    the encoding report (also written as encoding_report.json). The config is published
    last, so an interrupted conversion never looks loadable (:164-166)."""
    source, destination = Path(source), Path(destination)
    config, source_map = _check_source(source, destination)
    destination.mkdir(parents=True, exist_ok=True)
    report = {
        "format_version": 1,
        "encoder_version": __version__,
        "source_repo": SOURCE_REPO,
        "source_revision": source_revision,
        "status": "encoding",
        "tensors": {},
        "shards": {},
    }
    weight_map: dict[str, str] = {}
    total_size = 0
    for shard in sorted(set(source_map.values())):
        if Path(shard).name != shard:
            raise ValueError(f"Invalid shard filename: {shard}")
        owned = {name for name, owner in source_map.items() if owner == shard}
        output: dict[str, torch.Tensor] = {}
        with safe_open(source / shard, framework="pt", device="cpu") as handle:
            if set(handle.keys()) != owned:
                raise ValueError(f"Index and shard disagree: {shard}")
            for name in sorted(owned):
                tensors, record = _encode_tensor(name, handle.get_tensor(name), device, source_map)
                output.update(tensors)
                report["tensors"][name] = record
        pending = destination / (shard + ".tmp")
        save_file(output, pending, metadata={"format": "pt"})
        pending.replace(destination / shard)
        for name, tensor in output.items():
            weight_map[name] = shard
            total_size += tensor.numel() * tensor.element_size()
        report["shards"][shard] = {"sha256": _sha256(destination / shard),
                                   "tensor_count": len(output)}
        del output
        _publish_json(destination / "encoding_report.json", report)
        print(f"Encoded {shard}", flush=True)
    if set(report["tensors"]) != set(source_map):
        raise RuntimeError("Conversion did not preserve the source tensor inventory")
    for path in source.iterdir():
        if path.is_file() and path.suffix in _COPIED_SUFFIXES and path.name not in _NOT_COPIED:
            shutil.copy2(path, destination / path.name)
        elif path.name == "LICENSE":
            shutil.copy2(path, destination / path.name)
    config["quantization_config"] = {
        "quant_method": "qwen_int8",
        "format_version": 1,
        "weight_strategy": "channel_uint8",
        "vision_weight_strategy": "group32_int8",
        "source_repo": SOURCE_REPO,
        "source_revision": source_revision,
        "quantized_modules": {
            name.removesuffix(".weight"): record["encoding"]
            for name, record in report["tensors"].items()
            if record["encoding"] != "passthrough"
        },
    }
    _publish_json(destination / "model.safetensors.index.json",
                  {"metadata": {"total_size": total_size}, "weight_map": weight_map})
    report["status"] = "encoded_unvalidated"
    report["total_tensor_bytes"] = total_size
    _publish_json(destination / "encoding_report.json", report)
    _publish_json(destination / "config.json", config)
    return report


def load_channel_linear(checkpoint: Path, module: str, device="cuda", signed: bool = True):
    """One channel-UINT8 linear layer of an encoded checkpoint, on `device`.

    `module` is the layer name without ".weight". Returns (weight [N, K], scale BF16 [N]):
    signed INT8 codes (byte ^ 0x80, the debias of channel_mm's load path) for
    fused_channel_mm when `signed`, else the stored biased UINT8 for channel_mm.
    """
    checkpoint = Path(checkpoint)
    config = json.loads((checkpoint / "config.json").read_text())
    modules = config.get("quantization_config", {}).get("quantized_modules", {})
    if modules.get(module) != "channel_uint8":
        raise ValueError(f"Not a channel_uint8 module of this checkpoint: {module}")
    weight_map = json.loads((checkpoint / "model.safetensors.index.json").read_text())["weight_map"]
    name = module + ".weight"
    scale_name = scale_name_for(name, "channel_uint8")
    tensors = {}
    for key in (name, scale_name):
        with safe_open(checkpoint / weight_map[key], framework="pt", device="cpu") as handle:
            tensors[key] = handle.get_tensor(key)
    codes = tensors[name].to(device)
    if codes.dtype != torch.uint8 or codes.ndim != 2:
        raise ValueError(f"Expected UINT8 [N, K] codes for {module}")
    scale = tensors[scale_name].to(device)
    if signed:
        codes = codes.bitwise_xor(0x80).view(torch.int8)
    return codes, scale


def main(argv=None) -> None:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("source", type=Path)
    parser.add_argument("destination", type=Path)
    parser.add_argument("--source-revision", default=SOURCE_REVISION)
    parser.add_argument("--threads", type=int, default=4)
    parser.add_argument("--device", default="cpu", help="where to run the quantization (cpu or cuda)")
    args = parser.parse_args(argv)
    torch.set_num_threads(args.threads)
    encode(args.source, args.destination, source_revision=args.source_revision, device=args.device)


if __name__ == "__main__":
    main()
