"""Compressed checkpoints: a converted model saved without its BF16 originals, loaded back, or exported to a plain
BF16 Transformers checkpoint.

The directory layout is the reference's on-disk format (parda21/NWC nwc/checkpoint.py:1-16, :47-58), so a
checkpoint written by either library loads in the other:

    config.json, generation_config.json, tokenizer files    Hugging Face files, as usual
    nwc_config.json    {"nwc_checkpoint": 1, "library_version": 9 | 10 | 11, "base_model", "weights": [...],
                        "modules": [...], "bytes_nwc", "bytes_bf16"}
    model.safetensors  every uncompressed parameter, per compressed matrix "nwc/<id>/{data,bases,hdr,lut,low[,scale]}",
                       and the bias of a fused group under "nwc/fused/<parent path>.bias"

A "weights" entry is {id, out, in, block, bytes, elem: "bf16" | "fp8", layout}; a "modules" entry names the module
path and the weight id it uses, with kind "linear" (+ bias key), "embedding" (+ padding_idx) or "fused" (path of
the parent, + names, sizes and bias key of the fused projections).
"""
import json
import os
import shutil

import torch
import torch.nn as nn
from safetensors.torch import load_file, save_file

from .nwc_torch import VERSION, NWCEmbedding, NWCLinear, NWCWeight, _FusedGroup, _FusedSlice

FORMAT = 1
COMPATIBLE = frozenset({9, 10, VERSION})   # v9 (layout 0) and v10 (layouts 0/1) checkpoints load into v11
TENSOR_NAMES = ("data", "bases", "hdr", "lut", "low")
CONFIG_FILE, WEIGHTS_FILE = "nwc_config.json", "model.safetensors"


def _key(wid, name):
    return f"nwc/{wid}/{name}"


def _parent_path(path):
    return path.rpartition(".")[0]


class _Manifest:
    """The "weights" and "modules" lists of nwc_config.json, built while walking a converted model; each
    compressed matrix is listed once however many modules share it (tied embedding and output projection)."""

    def __init__(self):
        self.weights, self.modules, self.matrices = [], [], []
        self._ids = {}

    def weight_id(self, w: NWCWeight):
        if id(w) not in self._ids:
            self._ids[id(w)] = len(self.matrices)
            self.matrices.append(w)
            self.weights.append({"id": self._ids[id(w)], "out": w.out_features, "in": w.in_features,
                                 "block": w.block, "bytes": w.bytes, "elem": "fp8" if w.elem else "bf16",
                                 "layout": w.layout})
        return self._ids[id(w)]

    def walk(self, model):
        groups, biases = set(), {}
        for path, m in model.named_modules():
            if isinstance(m, NWCLinear):
                self.modules.append({"path": path, "kind": "linear", "weight": self.weight_id(m.w),
                                     "bias": None if m.bias is None else f"{path}.bias"})
            elif isinstance(m, NWCEmbedding):
                self.modules.append({"path": path, "kind": "embedding", "weight": self.weight_id(m.w),
                                     "padding_idx": m.padding_idx})
            elif isinstance(m, _FusedSlice) and id(m.group) not in groups:
                groups.add(id(m.group))
                parent, lin = _parent_path(path), m.group.lin
                bias_key = None if lin.bias is None else f"nwc/fused/{parent}.bias"
                if bias_key:
                    biases[bias_key] = lin.bias.detach()
                self.modules.append({"path": parent, "kind": "fused", "weight": self.weight_id(lin.w),
                                     "names": list(m.group.names), "sizes": list(m.group.sizes), "bias": bias_key})
        return biases


def save_pretrained(model: nn.Module, path: str, tokenizer=None, base_model: str = None):
    """Write a converted model (after fuse/convert) as an NWC checkpoint directory.  Returns the nwc_config dict."""
    os.makedirs(path, exist_ok=True)
    manifest = _Manifest()
    fused_biases = manifest.walk(model)
    tensors = {name: t.detach().cpu().contiguous() for name, t in model.state_dict().items()}
    tensors.update({k: t.cpu().contiguous() for k, t in fused_biases.items()})
    for wid, w in enumerate(manifest.matrices):
        tensors.update({_key(wid, name): t.cpu().contiguous() for name, t in w.tensors().items()})
    save_file(tensors, os.path.join(path, WEIGHTS_FILE), metadata={"format": "pt", "nwc": str(FORMAT)})
    config = {"nwc_checkpoint": FORMAT, "library_version": VERSION, "base_model": base_model,
              "weights": manifest.weights, "modules": manifest.modules,
              "bytes_nwc": sum(e["bytes"] for e in manifest.weights),
              "bytes_bf16": sum(2 * e["out"] * e["in"] for e in manifest.weights)}
    with open(os.path.join(path, CONFIG_FILE), "w", encoding="utf-8") as f:
        json.dump(config, f, indent=1)
    model.config.save_pretrained(path)
    if getattr(model, "generation_config", None) is not None:
        model.generation_config.save_pretrained(path)
    if tokenizer is not None:
        tokenizer.save_pretrained(path)
    return config


def resolve(path: str) -> str:
    """A checkpoint directory.  A path that is not a directory is treated as a Hugging Face repo id and fetched
    with huggingface_hub.snapshot_download when that is importable (it needs the network)."""
    if os.path.isdir(path):
        return path
    if os.path.exists(path):
        raise FileNotFoundError(f"{path} is a file; an NWC checkpoint is a directory")
    try:
        from huggingface_hub import snapshot_download
    except ImportError:
        raise FileNotFoundError(f"{path} is not a directory and huggingface_hub is not installed to fetch it")
    return snapshot_download(path)


def _read_manifest(path):
    cfg_path = os.path.join(path, CONFIG_FILE)
    if not os.path.exists(cfg_path):
        raise FileNotFoundError(f"{path} has no {CONFIG_FILE}: not an NWC checkpoint (compress a plain model with "
                                "nwc_amd.convert)")
    with open(cfg_path, encoding="utf-8") as f:
        config = json.load(f)
    if config["library_version"] not in COMPATIBLE:
        raise RuntimeError(f"checkpoint format version {config['library_version']} cannot be read by this library "
                           f"(version {VERSION}; readable: {sorted(COMPATIBLE)})")
    return config


def _weights_from(config, tensors, device):
    """NWCWeight per "weights" entry; its tensors are removed from `tensors`."""
    out = {}
    for e in config["weights"]:
        parts = {name: tensors.pop(_key(e["id"], name)) for name in TENSOR_NAMES}
        out[e["id"]] = NWCWeight.from_tensors(e["out"], e["in"], e["block"], device=device, elem=e.get("elem", "bf16"),
                                              scale=tensors.pop(_key(e["id"], "scale"), None),
                                              layout=e.get("layout", 0), **parts)
    return out


def _install(model, path, module):
    parent, _, name = path.rpartition(".")
    setattr(model.get_submodule(parent) if parent else model, name, module)


def load_pretrained(path: str, device="cuda", verbose=True):
    """Load an NWC checkpoint: the model on `device` with its NWC modules in place; the BF16 originals are never
    materialised."""
    from accelerate import init_empty_weights
    from accelerate.utils import set_module_tensor_to_device
    from transformers import AutoConfig, AutoModelForCausalLM
    path = resolve(path)
    config = _read_manifest(path)
    hf_config = AutoConfig.from_pretrained(path)
    with init_empty_weights():
        try:
            model = AutoModelForCausalLM.from_config(hf_config, dtype=torch.bfloat16)
        except TypeError:                                       # transformers before the dtype keyword
            model = AutoModelForCausalLM.from_config(hf_config, torch_dtype=torch.bfloat16)
    tensors = load_file(os.path.join(path, WEIGHTS_FILE))
    matrices = _weights_from(config, tensors, device)
    for m in config["modules"]:
        w = matrices[m["weight"]]
        if m["kind"] == "embedding":
            _install(model, m["path"], NWCEmbedding(w=w, padding_idx=m["padding_idx"]))
            continue
        bias = tensors.pop(m["bias"], None) if m.get("bias") else None
        lin = NWCLinear(w=w, bias=bias, device=device)
        if m["kind"] == "linear":
            _install(model, m["path"], lin)
        else:
            group = _FusedGroup(lin, m["names"], m["sizes"])
            for index, name in enumerate(m["names"]):
                _install(model, f"{m['path']}.{name}" if m["path"] else name, _FusedSlice(group, index))
    for name, t in tensors.items():
        set_module_tensor_to_device(model, name, device, value=t)
    missing = [n for n, p in model.named_parameters() if p.device.type == "meta"]
    if missing:
        raise RuntimeError(f"parameter {missing[0]} missing in the checkpoint")
    model.to(device).eval()
    if verbose:
        print(f"nwc_amd: loaded {path}: {config['bytes_bf16'] / 1e9:.2f} GB of BF16 weights held in "
              f"{config['bytes_nwc'] / 1e9:.2f} GB")
    return model


def _bf16_of(w: NWCWeight):
    """The matrix as stored in a BF16 checkpoint: decoded weights, fp8 codes times their row scale rounded to
    BF16."""
    full = w.dequant()
    if w.scale is not None:
        full = (full.float() * w.scale.unsqueeze(1)).to(torch.bfloat16)
    return full.contiguous().cpu()


def _export_entries(module, full, tensors, tied_output):
    """(state-dict key, tensor) pairs a module contributes to a BF16 checkpoint."""
    kind, path = module["kind"], module["path"]
    if kind == "embedding":
        return [(f"{path}.weight", full)]
    bias = tensors.pop(module["bias"]) if module.get("bias") else None
    if kind == "linear":
        out = [] if tied_output else [(f"{path}.weight", full)]  # a tied projection is stored as the embedding
        return out + ([(f"{path}.bias", bias)] if bias is not None else [])
    out, start = [], 0
    for name, size in zip(module["names"], module["sizes"]):
        key = f"{path}.{name}" if path else name
        out.append((f"{key}.weight", full[start:start + size].clone()))
        if bias is not None:
            out.append((f"{key}.bias", bias[start:start + size].clone()))
        start += size
    return out


def export_bf16(path: str, out: str, device="cuda", verbose=True):
    """Write the NWC checkpoint at `path` as a plain BF16 Transformers checkpoint at `out` (weights bit-identical
    to the originals).  Returns the number of BF16 bytes written for the compressed matrices."""
    path = resolve(path)
    config = _read_manifest(path)
    with open(os.path.join(path, "config.json"), encoding="utf-8") as f:
        tied = bool(json.load(f).get("tie_word_embeddings", False))
    tensors = load_file(os.path.join(path, WEIGHTS_FILE))
    tables = {m["weight"] for m in config["modules"] if m["kind"] == "embedding"}
    result, written = {}, 0
    for entry in config["weights"]:
        full = _bf16_of(_weights_from({"weights": [entry]}, tensors, device)[entry["id"]])
        written += 2 * full.numel()
        for m in config["modules"]:
            if m["weight"] == entry["id"]:
                result.update(_export_entries(m, full, tensors, tied and entry["id"] in tables))
    result.update(tensors)
    os.makedirs(out, exist_ok=True)
    save_file(result, os.path.join(out, WEIGHTS_FILE), metadata={"format": "pt"})
    for name in os.listdir(path):
        src = os.path.join(path, name)
        if name not in (WEIGHTS_FILE, CONFIG_FILE) and os.path.isfile(src):
            shutil.copyfile(src, os.path.join(out, name))
    if verbose:
        print(f"nwc_amd: {written / 1e9:.2f} GB of BF16 weights exported to {out}")
    return written
