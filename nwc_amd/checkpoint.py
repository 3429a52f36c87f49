"""Compressed checkpoints: save a converted model without the BF16 originals and load it back.

The on-disk format is the reference's (parda21/NWC nwc/checkpoint.py:1-16), so checkpoints written by either
library load in the other:
  config.json, generation_config.json, tokenizer files   (Hugging Face format)
  nwc_config.json      {nwc_checkpoint: 1, library_version, base_model, weights: [...], modules: [...], bytes_*}
  model.safetensors    the remaining parameters + per matrix "nwc/<id>/{data,bases,hdr,lut,low[,scale]}"
                       + biases of fused groups under "nwc/fused/<parent>.bias"
Loading builds the model on the meta device from the config, inserts the NWC modules and fills the rest.
"""
import json
import os

import torch
import torch.nn as nn
from safetensors.torch import load_file, save_file

from .nwc_torch import VERSION, NWCEmbedding, NWCLinear, NWCWeight, _FusedHead

FORMAT = 1
COMPATIBLE = {9, 10, VERSION}      # v9 (layout 0) and v10 (layouts 0/1) checkpoints load into the v11 library
TENSOR_NAMES = ("data", "bases", "hdr", "lut", "low")


def _parent(path):
    return path.rsplit(".", 1)[0] if "." in path else ""


def _collect(model):
    """All NWCWeight objects (each once) and the modules that use them (checkpoint.py:19-40)."""
    ids, weights, modules = {}, [], []

    def key(w):
        if id(w) not in ids:
            ids[id(w)] = len(weights)
            weights.append({"id": len(weights), "out": w.out_features, "in": w.in_features, "block": w.block,
                            "bytes": w.bytes, "elem": "fp8" if w.elem else "bf16", "layout": w.layout, "w": w})
        return ids[id(w)]

    groups = set()
    for path, m in model.named_modules():
        if isinstance(m, NWCLinear):
            modules.append({"path": path, "kind": "linear", "weight": key(m.w),
                            "bias": f"{path}.bias" if m.bias is not None else None})
        elif isinstance(m, NWCEmbedding):
            modules.append({"path": path, "kind": "embedding", "weight": key(m.w), "padding_idx": m.padding_idx})
        elif isinstance(m, _FusedHead) and id(m.g) not in groups:
            groups.add(id(m.g))
            lin = m.g["lin"]
            parent = _parent(path)
            modules.append({"path": parent, "kind": "fused", "weight": key(lin.w), "names": m.g["names"],
                            "sizes": m.g["sizes"], "bias": f"nwc/fused/{parent}.bias" if lin.bias is not None else None})
    return weights, modules


def save_pretrained(model: nn.Module, path: str, tokenizer=None, base_model: str = None):
    """Write a converted model (after convert/fuse) as an NWC checkpoint.  Returns the nwc_config dict."""
    os.makedirs(path, exist_ok=True)
    weights, modules = _collect(model)
    tensors = {k: v.detach().cpu().contiguous() for k, v in model.state_dict().items()}
    for e in weights:
        for name, t in e["w"].tensors().items():
            tensors[f"nwc/{e['id']}/{name}"] = t.cpu().contiguous()
    for m in modules:
        if m["kind"] == "fused" and m["bias"]:
            for p, mod in model.named_modules():
                if isinstance(mod, _FusedHead) and _parent(p) == m["path"]:
                    tensors[m["bias"]] = mod.g["lin"].bias.detach().cpu().contiguous()
                    break
    save_file(tensors, os.path.join(path, "model.safetensors"), metadata={"format": "pt", "nwc": str(FORMAT)})
    config = {"nwc_checkpoint": FORMAT, "library_version": VERSION, "base_model": base_model,
              "weights": [{k: v for k, v in e.items() if k != "w"} for e in weights], "modules": modules,
              "bytes_nwc": sum(e["bytes"] for e in weights), "bytes_bf16": sum(2 * e["out"] * e["in"] for e in weights)}
    with open(os.path.join(path, "nwc_config.json"), "w", encoding="utf-8") as f:
        json.dump(config, f, indent=1)
    model.config.save_pretrained(path)
    gc = getattr(model, "generation_config", None)
    if gc is not None:
        gc.save_pretrained(path)
    if tokenizer is not None:
        tokenizer.save_pretrained(path)
    return config


def _set(model, path, module):
    parent, _, name = path.rpartition(".")
    setattr(model.get_submodule(parent) if parent else model, name, module)


def resolve(path: str) -> str:
    """A local checkpoint directory.  (The reference also resolves Hugging Face repo ids through snapshot_download;
    that needs the network and is tried only when huggingface_hub is importable.)"""
    if os.path.isdir(path):
        return path
    if os.path.exists(path):
        raise FileNotFoundError(f"{path} is a file, an NWC checkpoint is a directory")
    try:
        from huggingface_hub import snapshot_download
    except ImportError:
        raise FileNotFoundError(f"{path} is not a directory, and huggingface_hub (for repo ids) is not installed")
    return snapshot_download(path)


def _load_weight(e, tensors, device):
    t = {n: tensors.pop(f"nwc/{e['id']}/{n}") for n in TENSOR_NAMES}
    return NWCWeight.from_tensors(e["out"], e["in"], e["block"], t["data"], t["bases"], t["hdr"], t["lut"], t["low"], device,
                                  elem=e.get("elem", "bf16"), scale=tensors.pop(f"nwc/{e['id']}/scale", None),
                                  layout=e.get("layout", 0))


def _read_config(path):
    with open(os.path.join(path, "nwc_config.json"), encoding="utf-8") as f:
        config = json.load(f)
    if config["library_version"] not in COMPATIBLE:
        raise RuntimeError(f"checkpoint is format version {config['library_version']}, library is {VERSION}")
    return config


def load_pretrained(path: str, device="cuda", verbose=True):
    """Load an NWC checkpoint: returns the model on `device` with NWC modules in place, no BF16 originals in RAM
    (checkpoint.py:83-128)."""
    from accelerate import init_empty_weights
    from accelerate.utils import set_module_tensor_to_device
    from transformers import AutoConfig, AutoModelForCausalLM
    path = resolve(path)
    if not os.path.exists(os.path.join(path, "nwc_config.json")):
        raise FileNotFoundError(f"{path} is not an NWC checkpoint (no nwc_config.json); a plain HF model is compressed with "
                                "nwc_amd.convert")
    config = _read_config(path)
    hf_config = AutoConfig.from_pretrained(path)
    with init_empty_weights():
        try:
            model = AutoModelForCausalLM.from_config(hf_config, dtype=torch.bfloat16)
        except TypeError:
            model = AutoModelForCausalLM.from_config(hf_config, torch_dtype=torch.bfloat16)
    tensors = load_file(os.path.join(path, "model.safetensors"))
    weights = {e["id"]: _load_weight(e, tensors, device) for e in config["weights"]}
    for m in config["modules"]:
        w = weights[m["weight"]]
        if m["kind"] == "linear":
            bias = tensors.pop(m["bias"], None) if m["bias"] else None
            _set(model, m["path"], NWCLinear(w=w, bias=bias, device=device))
        elif m["kind"] == "embedding":
            _set(model, m["path"], NWCEmbedding(w=w, padding_idx=m["padding_idx"]))
        else:
            bias = tensors.pop(m["bias"], None) if m["bias"] else None
            lin = NWCLinear(w=w, bias=bias, device=device)
            shared = {"lin": lin, "y": None, "x_id": None, "names": m["names"], "sizes": m["sizes"]}
            a = 0
            for i, (name, size) in enumerate(zip(m["names"], m["sizes"])):
                _set(model, f"{m['path']}.{name}" if m["path"] else name, _FusedHead(shared, i, a, a + size))
                a += size
    for k, v in tensors.items():
        set_module_tensor_to_device(model, k, device, value=v)
    for n, p in model.named_parameters():
        if p.device.type == "meta":
            raise RuntimeError(f"parameter {n} missing in the checkpoint")
    model.to(device).eval()
    if verbose:
        print(f"NWC: checkpoint loaded, {config['bytes_bf16']/1e9:.2f} GB BF16 -> {config['bytes_nwc']/1e9:.2f} GB "
              f"(ratio {config['bytes_nwc']/max(config['bytes_bf16'],1):.4f})")
    return model


def export_bf16(path: str, out: str, device="cuda", verbose=True):
    """Turn an NWC checkpoint back into a plain BF16 Transformers checkpoint (bit-identical weights) at `out`.
    Returns the BF16 byte count (checkpoint.py:131-173)."""
    import shutil
    path = resolve(path)
    config = _read_config(path)
    with open(os.path.join(path, "config.json"), encoding="utf-8") as f:
        tied = json.load(f).get("tie_word_embeddings", False)
    tensors = load_file(os.path.join(path, "model.safetensors"))
    embedding_ids = {m["weight"] for m in config["modules"] if m["kind"] == "embedding"}
    result, total = {}, 0
    for e in config["weights"]:
        w = _load_weight(e, tensors, device)
        full = w.dequant()
        if w.scale is not None:
            full = (full.float() * w.scale[:, None]).to(torch.bfloat16)    # fp8 x scale, rounded to BF16
        full = full.contiguous().cpu()
        del w
        total += full.numel() * 2
        for m in config["modules"]:
            if m["weight"] != e["id"]:
                continue
            if m["kind"] == "embedding":
                result[f"{m['path']}.weight"] = full
            elif m["kind"] == "linear":
                if not (tied and e["id"] in embedding_ids):
                    result[f"{m['path']}.weight"] = full
                if m["bias"]:
                    result[f"{m['path']}.bias"] = tensors.pop(m["bias"])
            else:
                bias = tensors.pop(m["bias"]) if m["bias"] else None
                a = 0
                for name, size in zip(m["names"], m["sizes"]):
                    key = f"{m['path']}.{name}" if m["path"] else name
                    result[f"{key}.weight"] = full[a:a + size].clone()
                    if bias is not None:
                        result[f"{key}.bias"] = bias[a:a + size].clone()
                    a += size
    result.update(tensors)
    os.makedirs(out, exist_ok=True)
    save_file(result, os.path.join(out, "model.safetensors"), metadata={"format": "pt"})
    for name in os.listdir(path):
        if name not in ("model.safetensors", "nwc_config.json") and os.path.isfile(os.path.join(path, name)):
            shutil.copyfile(os.path.join(path, name), os.path.join(out, name))
    if verbose:
        print(f"NWC: exported {total/1e9:.2f} GB of BF16 weights to {out}")
    return total
