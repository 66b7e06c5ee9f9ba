"""Serve a synthetic decoder over stdin/stdout with the reference's serve
protocol (bench/dsv2_decode_bench.c:2749-2897): prints "ready", then answers
each request line "id,id,...[|max_new]" with one line "ids: id,id,...";
EOF ends.  Timing goes to stderr.

    python -m thvm_amd.serve --config C4 [--layers N] [--max-seq S]
        [--temperature T --seed K] [--eos ID] [--max-new N]

The weights are the seeded random-init weights of the configuration (there
is no network for checkpoints); thvm_amd.weights loads real ones into the
same decoder when files are local."""
from __future__ import annotations

import argparse
import sys

import thvm_amd
from thvm_amd.configs import DECODERS


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--config", default="C4", choices=sorted(DECODERS))
    ap.add_argument("--layers", type=int, default=0, help="override n_layers (0: the config's)")
    ap.add_argument("--max-seq", type=int, default=4096)
    ap.add_argument("--temperature", type=float, default=0.0)
    ap.add_argument("--seed", type=int, default=0, help="sampling seed")
    ap.add_argument("--weight-seed", type=int, default=1234)
    ap.add_argument("--eos", type=int, default=-1)
    ap.add_argument("--max-new", type=int, default=256)
    a = ap.parse_args(argv)
    cfg = dict(DECODERS[a.config], batch=1, max_seq=a.max_seq, temperature=a.temperature,
               sample_seed_lo=a.seed & 0xFFFFFFFF, sample_seed_hi=(a.seed >> 32) & 0xFFFFFFFF)
    if a.layers:
        cfg["n_layers"] = a.layers
    thvm_amd.init()
    dec = thvm_amd.Decoder(seed=a.weight_seed, **cfg)
    print(f"[serve] {a.config} {cfg['n_layers']} layers, max_seq {a.max_seq}, "
          f"temperature {a.temperature}", file=sys.stderr, flush=True)
    try:
        dec.serve(sys.stdin.fileno(), sys.stdout.fileno(), a.eos, a.max_new)
    finally:
        dec.close()
        thvm_amd.shutdown()
    return 0


if __name__ == "__main__":
    sys.exit(main())
