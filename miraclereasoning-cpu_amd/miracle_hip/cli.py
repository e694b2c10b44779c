"""Command line: ``python -m miracle_hip {devices,inspect,export,generate}``.

The reference's commands and flags (cli.py:30-95) over the HIP engine:
``devices`` lists the visible gfx950 GPUs, ``inspect`` reads a bundle's
config without touching a GPU, ``export`` writes a standalone bundle, and
``generate`` runs a prompt (token ids, or text through a SentencePiece /
tokenizers file) on one MI355X and prints the generated ids as JSON.  Errors
are printed to stderr and give exit status 2.
"""
from __future__ import annotations

import argparse
import json
import math
import sys
from pathlib import Path

from .config import FAMILIES, ModelConfig
from .hip import HIPBackend, HIPError, list_devices

_ERRORS = (ValueError, OSError, KeyError, ImportError, HIPError, FloatingPointError)


def load_tokenizer(path):
    """SentencePiece ``.model`` or a tokenizers ``.json``, as encode/decode."""
    path = Path(path)
    if path.suffix == ".model":
        import sentencepiece
        return sentencepiece.SentencePieceProcessor(model_file=str(path))
    from tokenizers import Tokenizer
    tok = Tokenizer.from_file(str(path))

    class _Ids:
        @staticmethod
        def encode(text):
            return tok.encode(text, add_special_tokens=False).ids

        @staticmethod
        def decode(ids):
            return tok.decode(ids)
    return _Ids()


def _parser():
    ap = argparse.ArgumentParser(prog="miracle_hip", description="Miracle per-token inference on MI355X (HIP)")
    sub = ap.add_subparsers(dest="command", required=True)
    sub.add_parser("devices", help="list HIP GPUs and their memory")
    p = sub.add_parser("inspect", help="summarise a bundle's configuration (no GPU needed)")
    p.add_argument("model_dir", type=Path)
    p.add_argument("--family", choices=FAMILIES)
    p = sub.add_parser("export", help="convert a checkpoint into a standalone safetensors bundle")
    p.add_argument("--checkpoint", required=True, type=Path)
    p.add_argument("--config", required=True, type=Path)
    p.add_argument("--output", required=True, type=Path)
    p.add_argument("--family", choices=FAMILIES)
    p.add_argument("--fp32", action="store_true", help="write FP32 tensors (the reference's bundle format)")
    p = sub.add_parser("generate", help="generate tokens on one MI355X")
    p.add_argument("model_dir", type=Path)
    src = p.add_mutually_exclusive_group(required=True)
    src.add_argument("--ids", help="token ids separated by commas or spaces")
    src.add_argument("--prompt")
    p.add_argument("--tokenizer", type=Path)
    p.add_argument("--family", choices=FAMILIES)
    p.add_argument("--context-length", type=int, help="default: min(2048, model context limit)")
    p.add_argument("--weight-cache-mib", type=int, default=256)
    p.add_argument("--platform-index", type=int, help="accepted for compatibility; HIP has one platform (0)")
    p.add_argument("--device-index", type=int)
    p.add_argument("--max-new-tokens", type=int, default=32)
    p.add_argument("--temperature", type=float, default=0.0)
    p.add_argument("--top-k", type=int, default=0)
    p.add_argument("--top-p", type=float, default=1.0)
    p.add_argument("--seed", type=int, default=17)
    p.add_argument("--prefill-mode", choices=("exact", "batched"), default="exact")
    return ap


def _inspect(args):
    from .weights import expected_shapes
    config = ModelConfig.from_dict(json.loads((args.model_dir / "config.json").read_text(encoding="utf-8")),
                                   args.family)
    params = sum(math.prod(shape) for shape in expected_shapes(config).values())
    return {"family": config.family, "layers": config.layers, "hidden_size": config.hidden_size,
            "max_positions": config.max_positions, "inference_parameters": params, "fp32_weight_bytes": params * 4}


def _generate(args):
    from .model import MiracleModel
    tokenizer = None
    if args.prompt is not None:
        if args.tokenizer is None:
            raise ValueError("--prompt requires --tokenizer (SentencePiece .model or tokenizers .json)")
        tokenizer = load_tokenizer(args.tokenizer)
        ids = list(tokenizer.encode(args.prompt))
    else:
        ids = [int(t) for t in args.ids.replace(",", " ").split()]
    backend = HIPBackend(platform_index=args.platform_index, device_index=args.device_index)
    try:
        model = MiracleModel.from_pretrained(args.model_dir, family=args.family, backend=backend,
                                             context_length=args.context_length,
                                             weight_cache_bytes=args.weight_cache_mib * 1024 * 1024,
                                             prefill_mode=args.prefill_mode)
        tokens = model.generate(ids, max_new_tokens=args.max_new_tokens, temperature=args.temperature,
                                top_k=args.top_k, top_p=args.top_p, seed=args.seed)
        model.close()
        out = {"device": backend.device.to_dict(), "token_ids": tokens}
        if tokenizer is not None:
            out["text"] = tokenizer.decode(tokens)
        return out
    finally:
        backend.close()


def main(argv=None):
    args = _parser().parse_args(argv)
    try:
        if args.command == "devices":
            print(json.dumps([d.to_dict() for d in list_devices()], indent=2, ensure_ascii=False))
        elif args.command == "inspect":
            print(json.dumps(_inspect(args), indent=2))
        elif args.command == "export":
            from .export import export_checkpoint
            config = export_checkpoint(args.checkpoint, args.config, args.output, family=args.family,
                                       widen=args.fp32)
            print(json.dumps({"output": str(args.output.resolve()), "family": config.family}))
        else:
            print(json.dumps(_generate(args), ensure_ascii=False))
        return 0
    except _ERRORS as exc:
        print(f"error: {exc}", file=sys.stderr)
        return 2


if __name__ == "__main__":
    sys.exit(main())
