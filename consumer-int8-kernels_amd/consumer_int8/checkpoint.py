"""Channel-UINT8 checkpoint encoding and loading for the INT8 linear layers.

`encode` converts an unquantized Qwen3.8-27B safetensors snapshot into the reference's
published encoding (the format written by src/consumer_int8/checkpoint.py:58-171): the
language-model and MTP linear weights become biased UINT8 codes plus BF16
`*.weight_scale_inv` channel scales, the vision tower's linear weights become signed
INT8 plus FP32 `*.weight_scale` group scales, and every other tensor passes through.
The files, tensor names, shard ownership, report fields, index and `quantization_config`
are that format, and the same inputs are refused with the same messages. The encoder
itself is organised differently: it plans and checks the whole snapshot before writing
anything (a snapshot refused for its layout leaves the destination empty; only
non-finite weights are found while encoding), then encodes shard by shard.

`device` selects where the quantization arithmetic runs: "cuda" encodes on the MI355X
with results bit-identical to the host's (the codes and scales are IEEE FP32 operations
with one correct rounding each); the report's error statistics are reductions and may
differ in their last bits.

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

# Files of the snapshot published next to the shards: small text sidecars (tokenizer,
# chat template, generation config, ...) and the licence, but not the files the encoder
# rewrites itself or the source's checksum list.
_SIDECAR_SUFFIXES = (".json", ".txt", ".jinja")
_REWRITTEN = ("config.json", "model.safetensors.index.json", "crc32.txt")


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


def _file_sha256(path: Path) -> str:
    digest = hashlib.sha256()
    with path.open("rb") as stream:
        while chunk := stream.read(1 << 23):
            digest.update(chunk)
    return digest.hexdigest()


def _atomic_json(path: Path, value: dict) -> None:
    """Publish `value` at `path` by writing a sibling and renaming it over the target, so
    a reader sees either the old file or the whole new one."""
    staged = path.parent / f"{path.name}.tmp"
    staged.write_text(json.dumps(value, indent=2) + "\n")
    staged.replace(path)


class _Job:
    """One source tensor: how it is stored and under which extra name its scales go."""

    __slots__ = ("name", "encoding", "scale_name")

    def __init__(self, name: str):
        self.name = name
        self.encoding = encoding_for(name)
        self.scale_name = (None if self.encoding == "passthrough"
                           else scale_name_for(name, self.encoding))


def _plan(source: Path, destination: Path) -> tuple[dict, dict[str, list[_Job]]]:
    """Everything that can refuse a snapshot without encoding it, done before the first
    byte is written: the directories, the architecture and geometry of the config (the
    manifest targets Qwen3.8-27B only), the MTP and vision parts of the index, shard file
    names, the tensors each shard actually holds, and scale names that would collide with
    source tensors. The refusals carry the reference's messages
    (src/consumer_int8/checkpoint.py:59-76, :86-90, :110-111). Returns the config and,
    per shard in sorted order, the jobs of its tensors in sorted name order."""
    if source.resolve() == destination.resolve():
        raise ValueError("Source and destination must differ")
    if destination.exists() and next(destination.iterdir(), None) is not None:
        raise ValueError("Destination must be empty; partial conversions are not models")
    config = json.loads((source / "config.json").read_text())
    if config.get("model_type") != "qwen3_5" or config.get("quantization_config"):
        raise ValueError("Expected an unquantized Qwen3.5 architecture checkpoint")
    geometry = config["text_config"]
    if geometry["hidden_size"] != 5120 or geometry["num_hidden_layers"] != 64:
        raise ValueError("This encoding manifest targets Qwen3.8-27B geometry")
    owner = json.loads((source / "model.safetensors.index.json").read_text())["weight_map"]
    for part, prefix in (("MTP", "mtp."), ("vision", "model.visual.")):
        if not any(name.startswith(prefix) for name in owner):
            raise ValueError(f"The full checkpoint must contain {part} weights")

    by_shard: dict[str, list[str]] = {}
    for name, shard in owner.items():
        by_shard.setdefault(shard, []).append(name)
    shards: dict[str, list[_Job]] = {}
    for shard in sorted(by_shard):
        if Path(shard).name != shard:
            raise ValueError(f"Invalid shard filename: {shard}")
        with safe_open(source / shard, framework="pt", device="cpu") as handle:
            held = set(handle.keys())
        if held != set(by_shard[shard]):
            raise ValueError(f"Index and shard disagree: {shard}")
        jobs = [_Job(name) for name in sorted(held)]
        for job in jobs:
            if job.scale_name is not None and job.scale_name in owner:
                raise ValueError(f"Scale name already exists: {job.scale_name}")
        shards[shard] = jobs
    return config, shards


def _quantize(job: _Job, weight: torch.Tensor, device: str):
    """Codes, scales and the report's error statistics of one quantized tensor (the
    reference's arithmetic, src/consumer_int8/checkpoint.py:100-118)."""
    on_device = weight.to(device)
    if job.encoding == "channel_uint8":
        codes, scales = quantize_channel(on_device)
        error = dequantize_channel(codes, scales) - on_device.float()
    else:
        codes, scales = quantize_group32(on_device)
        error = dequantize_group32(codes, scales) - on_device.float()
    stats = {"rmse": error.square().mean().sqrt().item(),
             "max_abs_error": error.abs().max().item()}
    return codes.cpu(), scales.cpu(), stats


def encode(source: Path, destination: Path, *, source_revision: str, device: str = "cpu") -> dict:
    """Encode the checkpoint at `source` into the empty directory `destination`; returns
    the encoding report (also written as encoding_report.json).

    The snapshot is planned and checked in full first (`_plan`), then encoded one shard
    at a time: each shard's tensors go to a staged file renamed into place once complete,
    and the report is republished after every shard, so progress is visible and every
    published shard is whole. The index, the final report and, last of all, the config
    (which is what makes a directory loadable) follow the shards."""
    source, destination = Path(source), Path(destination)
    config, shards = _plan(source, destination)
    destination.mkdir(parents=True, exist_ok=True)

    records: dict[str, dict] = {}
    shard_records: dict[str, dict] = {}
    stored_in: dict[str, str] = {}
    stored_bytes = 0

    def report(status: str) -> dict:
        return {"format_version": 1, "encoder_version": __version__,
                "source_repo": SOURCE_REPO, "source_revision": source_revision,
                "status": status, "tensors": records, "shards": shard_records}

    for shard, jobs in shards.items():
        tensors: dict[str, torch.Tensor] = {}
        with safe_open(source / shard, framework="pt", device="cpu") as handle:
            for job in jobs:
                weight = handle.get_tensor(job.name)
                record = {"shape": list(weight.shape), "encoding": job.encoding}
                if job.scale_name is None:
                    tensors[job.name] = weight
                else:
                    codes, scales, stats = _quantize(job, weight, device)
                    tensors[job.name], tensors[job.scale_name] = codes, scales
                    record.update(stats)
                record["stored_dtype"] = str(tensors[job.name].dtype)
                records[job.name] = record
        staged = destination / f"{shard}.tmp"
        save_file(tensors, staged, metadata={"format": "pt"})
        staged.replace(destination / shard)
        stored_in.update(dict.fromkeys(tensors, shard))
        stored_bytes += sum(t.numel() * t.element_size() for t in tensors.values())
        shard_records[shard] = {"sha256": _file_sha256(destination / shard),
                                "tensor_count": len(tensors)}
        tensors.clear()
        _atomic_json(destination / "encoding_report.json", report("encoding"))
        print(f"Encoded {shard}", flush=True)

    planned = {job.name for jobs in shards.values() for job in jobs}
    if set(records) != planned:
        raise RuntimeError("Conversion did not preserve the source tensor inventory")

    for path in source.iterdir():
        sidecar = (path.is_file() and path.suffix in _SIDECAR_SUFFIXES
                   and path.name not in _REWRITTEN)
        if sidecar or path.name == "LICENSE":
            shutil.copy2(path, destination / path.name)

    quantized = {name.removesuffix(".weight"): rec["encoding"]
                 for name, rec in records.items() if rec["encoding"] != "passthrough"}
    config["quantization_config"] = {
        "quant_method": "qwen_int8",
        "format_version": 1,
        "weight_strategy": "channel_uint8",
        "vision_weight_strategy": "group32_int8",
        "source_repo": SOURCE_REPO,
        "source_revision": source_revision,
        "quantized_modules": quantized,
    }
    _atomic_json(destination / "model.safetensors.index.json",
                 {"metadata": {"total_size": stored_bytes}, "weight_map": stored_in})
    final = report("encoded_unvalidated")
    final["total_tensor_bytes"] = stored_bytes
    _atomic_json(destination / "encoding_report.json", final)
    _atomic_json(destination / "config.json", config)
    return final


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
