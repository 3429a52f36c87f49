"""nwc_amd -- NWC lossless weight compression with a fused decode-matvec for AMD Instinct MI355X (gfx950).

    from nwc_amd import convert, fuse, save_pretrained, load_pretrained, export_bf16
    fuse(model); convert(model)              # nn.Linear -> NWCLinear, model to the GPU (lossless BF16)
    fuse(model, elem="fp8"); convert(model, elem="fp8")   # or weight-only fp8, the fp8 values stored lossless
    save_pretrained(model, "Qwen3-4B-NWC")   # write a compressed checkpoint (format v9/v10/v11)
    model = load_pretrained("Qwen3-4B-NWC")  # load without the BF16 originals
    export_bf16("Qwen3-4B-NWC", "Qwen3-4B")  # back to a plain BF16 checkpoint, bit-identical

The public API mirrors the reference package `nwc` (parda21/NWC nwc/__init__.py:10-16); `import nwc_amd as nwc`
is the drop-in.
"""
__version__ = "0.10.1"

__all__ = ["NWCWeight", "NWCLinear", "NWCEmbedding", "convert", "fuse", "fits", "choose_block",
           "quantize_fp8", "save_pretrained", "load_pretrained", "export_bf16", "__version__"]

_FROM = {**{n: "nwc_torch" for n in ("NWCWeight", "NWCLinear", "NWCEmbedding", "convert", "fuse", "fits", "choose_block",
                                      "quantize_fp8")},
         **{n: "checkpoint" for n in ("save_pretrained", "load_pretrained", "export_bf16")}}


def __getattr__(name):
    """The public names load the HIP library on first use (ImportError when it is not built), so that
    `python -m nwc_amd.build` works before the library exists."""
    if name in _FROM:
        import importlib
        value = getattr(importlib.import_module(f".{_FROM[name]}", __name__), name)
        globals()[name] = value
        return value
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
