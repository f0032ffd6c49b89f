"""Single-shot command line over the .krunch container (the role of
krunch/cli.py:1-158): compress or decompress stdin -> stdout, or --in/--out
files.

    python -m krunch_amd.cli compress   [--in PATH] [--out PATH] [--weights PATH]
                                        [--tokenizer PATH] [--w8a8]
    python -m krunch_amd.cli decompress [--in PATH] [--out PATH] [--weights PATH]
                                        [--tokenizer PATH]

`--in`/`--out` default to stdin/stdout ("-" also means them), as in the
reference (cli.py:121-134). The model is an RWKV-4 checkpoint (`--weights`
or $KRUNCH_WEIGHTS; `.pth` / `.safetensors`, read with safe loaders), else the
synthetic RWKV-4-169M-shaped model (seed 0). The tokenizer is a `tokenizers`
JSON (`--tokenizer` or $KRUNCH_TOKENIZER), else the byte tokenizer. Compress
writes header + entries for all chunks in one batched call (cli.py:49-70);
decompress picks the fp16 or int8 codec from the blob's model_id and checks
codec, CRC32 and length as the reference does (cli.py:73-118). Errors go to
stderr with exit status 1; logs go to stderr so stdout carries only data.
"""
from __future__ import annotations

import argparse
import logging
import os
import sys
from typing import Callable, Optional, Sequence

from krunch_amd.inference import MODEL_ID_W8A8, InferenceEngine, decode_header

logger = logging.getLogger("krunch_amd.cli")

# (weights, tokenizer, w8a8) -> loaded engine: one load per codec in a process
_ENGINES: dict = {}


def _load_engine(weights: Optional[str], tokenizer: Optional[str], w8a8: bool) -> InferenceEngine:
    key = (weights, tokenizer, w8a8)
    if key not in _ENGINES:
        _ENGINES[key] = InferenceEngine().load(weights, tokenizer_path=tokenizer, w8a8=w8a8)
    return _ENGINES[key]


def _read_input(path: Optional[str]) -> bytes:
    if path and path != "-":
        with open(path, "rb") as f:
            return f.read()
    return sys.stdin.buffer.read()


def _write_output(path: Optional[str], data: bytes) -> None:
    if path and path != "-":
        with open(path, "wb") as f:
            f.write(data)
    else:
        sys.stdout.buffer.write(data)
        sys.stdout.buffer.flush()


def _model_paths(args) -> tuple:
    weights = args.weights or os.environ.get("KRUNCH_WEIGHTS") or None
    tokenizer = args.tokenizer or os.environ.get("KRUNCH_TOKENIZER") or None
    return weights, tokenizer


def cmd_compress(args, load: Callable = _load_engine) -> None:
    raw = _read_input(args.input)
    weights, tokenizer = _model_paths(args)
    blob = load(weights, tokenizer, bool(args.w8a8)).compress(raw)
    _write_output(args.output, blob)
    ratio = len(blob) / len(raw) if raw else 0.0
    logger.info("compress %d -> %d bytes (ratio=%.4f)", len(raw), len(blob), ratio)


def cmd_decompress(args, load: Callable = _load_engine) -> None:
    blob = _read_input(args.input)
    hdr = decode_header(blob)            # ValueError on a short or foreign blob
    weights, tokenizer = _model_paths(args)
    raw = load(weights, tokenizer, hdr["model_id"] == MODEL_ID_W8A8).decompress(blob)
    _write_output(args.output, raw)
    logger.info("decompress %d -> %d bytes", len(blob), len(raw))


def build_parser() -> argparse.ArgumentParser:
    ap = argparse.ArgumentParser(prog="krunch", description="Krunch neural compression (MI355X)")
    sub = ap.add_subparsers(dest="cmd", required=True)
    for name, hlp in (("compress", "Compress bytes"), ("decompress", "Decompress a .krunch blob")):
        p = sub.add_parser(name, help=hlp)
        p.add_argument("--in", dest="input", help="input file (default: stdin)")
        p.add_argument("--out", dest="output", help="output file (default: stdout)")
        p.add_argument("--weights", help="RWKV-4 checkpoint (.pth / .safetensors); "
                                         "default $KRUNCH_WEIGHTS, else the synthetic model")
        p.add_argument("--tokenizer", help="tokenizers JSON; default $KRUNCH_TOKENIZER, "
                                           "else the byte tokenizer")
        if name == "compress":
            p.add_argument("--w8a8", action="store_true",
                           help="int8 codec (model_id 2); decompress detects it from the blob")
    return ap


def main(argv: Optional[Sequence[str]] = None, load: Callable = _load_engine) -> int:
    logging.basicConfig(level=logging.INFO, format="%(asctime)s %(levelname)s %(message)s",
                        stream=sys.stderr)
    args = build_parser().parse_args(argv)
    try:
        if args.cmd == "compress":
            cmd_compress(args, load)
        else:
            cmd_decompress(args, load)
    except (ValueError, OSError) as e:
        print(f"krunch: {e}", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
