"""Write (or check) a golden cache directory with this repository's CPU oracle.

Same command line and output lines as the reference's cache tool
(scripts/generate_full_bwd_golden.py:22-35, 296-317): the inputs are the
reference's deterministic pattern tensors, the outputs the oracle's fp32
forward / backward, the directory layout that of flash-attention3_amd/
golden_cache.py.  Test infrastructure: it runs the oracle.

    python tests/golden/make_golden_cache.py --root /tmp/golden --heads 2 --seqlen 256
"""
import argparse
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "flash-attention3_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import fa3_oracle as O  # noqa: E402
import golden_cache as GC  # noqa: E402


def oracle_arrays(batch, heads_q, heads_kv, seqlen, head_dim, causal, scale):
    g = O.golden(batch, heads_q, heads_kv, seqlen, head_dim, bool(causal), scale=scale,
                 kind="pattern")
    return {"q.f16": g["q"], "k.f16": g["k"], "v.f16": g["v"], "o.f16": g["out"],
            "dout.f16": g["dout"], "scores_max.f32": g["scores_max"],
            "scores_sum.f32": g["scores_sum"], "delta.f32": g["delta"], "dq.f32": g["dq"],
            "dk.f32": g["dk"], "dv.f32": g["dv"]}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--root", required=True)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--heads", type=int, default=1)
    ap.add_argument("--heads-kv", type=int)
    ap.add_argument("--seqlen", type=int, default=128)
    ap.add_argument("--dim", type=int, default=128)
    ap.add_argument("--causal", type=int, choices=(0, 1), default=1)
    ap.add_argument("--softmax-scale", type=float, default=GC.DEFAULT_SCALE)
    ap.add_argument("--regenerate", action="store_true")
    a = ap.parse_args(argv)
    hkv = a.heads if a.heads_kv is None else a.heads_kv
    if min(a.batch, a.heads, hkv, a.seqlen, a.dim) <= 0:
        raise SystemExit("all shape dimensions must be positive")
    if a.heads % hkv:
        raise SystemExit("heads must be divisible by heads-kv")
    dims = dict(batch=a.batch, heads_q=a.heads, heads_kv=hkv, seqlen=a.seqlen, head_dim=a.dim)
    path = os.path.join(os.path.abspath(a.root),
                        GC.cache_key(causal=a.causal, scale=a.softmax_scale, **dims))
    hit = os.path.isdir(path) and not a.regenerate
    arrays = None if hit else oracle_arrays(causal=a.causal, scale=a.softmax_scale, **dims)
    if hit:
        GC.validate(path, causal=a.causal, scale=a.softmax_scale, **dims)
    else:
        GC.write(a.root, arrays, causal=a.causal, scale=a.softmax_scale,
                 regenerate=a.regenerate, **dims)
    manifest = GC.validate(path, causal=a.causal, scale=a.softmax_scale, **dims)
    print(f"golden_cache_status={'HIT' if hit else 'MISS'}")
    print(f"golden_cache_path={path}")
    print(f"golden_payload_sha256={manifest['payload_sha256']}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
