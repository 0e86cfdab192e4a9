"""Command line of the gfx950 lrrt bundle tool.

Mirrors the reference's ``sparsewave-bundle`` options
(tools/sparsewave-bundle/sparsewave-bundle.py:287-322): an optional
fixed-shape SparseWave IR input, --output, --chip, --operation, --mapping,
--block-size, --tile-size, --wavefront-size, and --verify.  Shapes may also
be given directly (--rows/--rhs-columns for SpMM; --rows/--key-value-rows/
--head-dimension/--value-columns for sparse attention) since this build has
no MLIR front end.  Exit status 1 on a rejected request or bundle.
"""
import argparse
import json
import sys
from pathlib import Path

from . import (BundleError, DEFAULT_TILE_SIZE, SUPPORTED_BLOCK_SIZE,
               SUPPORTED_MAPPING, SUPPORTED_TARGET, SUPPORTED_WAVEFRONT_SIZE,
               build_attention_bundle, build_spmm_bundle,
               parse_spmm_signature, verify_bundle)


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m sparsewavecomp_amd.bundle")
    ap.add_argument("input", nargs="?", type=Path,
                    help="fixed-shape IR holding sparsewave.spmm")
    ap.add_argument("--output", type=Path)
    ap.add_argument("--verify", type=Path, help="verify an existing bundle")
    ap.add_argument("--chip", default=SUPPORTED_TARGET)
    ap.add_argument("--operation", default="auto",
                    choices=["auto", "spmm", "sparse-attention",
                             "sparse_attention"])
    ap.add_argument("--mapping", default=SUPPORTED_MAPPING)
    ap.add_argument("--block-size", type=int, default=SUPPORTED_BLOCK_SIZE)
    ap.add_argument("--tile-size", type=int, default=DEFAULT_TILE_SIZE)
    ap.add_argument("--wavefront-size", type=int,
                    default=SUPPORTED_WAVEFRONT_SIZE)
    ap.add_argument("--rows", type=int)
    ap.add_argument("--rhs-columns", type=int)
    ap.add_argument("--key-value-rows", type=int)
    ap.add_argument("--head-dimension", type=int)
    ap.add_argument("--value-columns", type=int)
    ap.add_argument("--alpha", type=float)
    ap.add_argument("--beta", type=float, default=0.0)
    args = ap.parse_args(argv)
    try:
        if args.verify:
            manifest = verify_bundle(args.verify)
            print(f"verified {args.verify}: {len(manifest['kernels'])} "
                  "kernel(s)")
            return 0
        if args.output is None:
            raise BundleError("--output is required")
        op = args.operation.replace("_", "-")
        if op == "auto":
            op = ("sparse-attention" if args.key_value_rows is not None
                  else "spmm")
        if op == "spmm":
            if args.input is not None:
                shapes = parse_spmm_signature(args.input.read_text())
                rows, k = shapes["rows"], shapes["rhs_columns"]
            else:
                if args.rows is None:
                    raise BundleError("SpMM bundle needs an input or --rows")
                rows = args.rows
                k = args.rhs_columns if args.rhs_columns else args.tile_size
            manifest = build_spmm_bundle(
                args.output, rows, k, tile_size=args.tile_size,
                mapping=args.mapping, block_size=args.block_size,
                wavefront_size=args.wavefront_size, chip=args.chip)
        else:
            for name in ("rows", "key_value_rows", "head_dimension",
                         "value_columns"):
                if getattr(args, name) is None:
                    raise BundleError(f"sparse-attention bundle needs "
                                      f"--{name.replace('_', '-')}")
            manifest = build_attention_bundle(
                args.output, args.rows, args.key_value_rows,
                args.head_dimension, args.value_columns, alpha=args.alpha,
                beta=args.beta, block_size=args.block_size,
                wavefront_size=args.wavefront_size, chip=args.chip)
        verify_bundle(args.output)
        print(json.dumps({"bundle": str(args.output),
                          "kernels": [k["name"] for k in
                                      manifest["kernels"]]}))
        return 0
    except BundleError as e:
        print(f"error: {e}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    sys.exit(main())
