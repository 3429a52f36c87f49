"""Command line: an NWC checkpoint back to a plain BF16 Transformers checkpoint (bit-identical weights).

    python -m nwc_amd.export CHECKPOINT OUT_DIR [--device cuda]

The counterpart of the reference's `python -m nwc.export` (parda21/NWC nwc/export.py); the work is done by
nwc_amd.checkpoint.export_bf16.
"""
import argparse
import sys


def main(argv=None):
    parser = argparse.ArgumentParser(prog="python -m nwc_amd.export",
                                     description="write an NWC checkpoint as a plain BF16 checkpoint")
    parser.add_argument("checkpoint", help="NWC checkpoint directory")
    parser.add_argument("out", help="output directory (model.safetensors, config and tokenizer files)")
    parser.add_argument("--device", default="cuda", help="GPU that decodes the matrices (default: cuda)")
    args = parser.parse_args(argv)
    from .checkpoint import export_bf16
    export_bf16(args.checkpoint, args.out, device=args.device)
    return 0


if __name__ == "__main__":
    sys.exit(main())
