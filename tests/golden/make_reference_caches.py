"""Write the golden caches of the reference's own cache tool as fixtures.

Runs the reference's cache tool, scripts/generate_full_bwd_golden.py (numpy
only; its CPU golden is :135-219, its cache writer :222-290), as a separate
process in the build container, for two small shapes, and leaves the cache
directories it writes under tests/golden/reference_caches/.  Those committed
directories are data -- the tool's deterministic-pattern inputs, its fp32
outputs and its manifest -- which tests/test_golden_cache.py and
tests/test_gpu_golden_cache.py read through flash-attention3_amd/
golden_cache.py.  The reference tree exists only in the build container; the
tests never run the tool.

    python tests/golden/make_reference_caches.py [--reference /root/reference]
"""
import argparse
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "reference_caches")

# (batch, heads, heads_kv, seqlen, dim, causal), at the tool's default scale
# 1 / sqrt(128): the reference's plumbing shape and its GQA gate shape
# (reference docs/full_bwd_correctness.md, docs/fused5_gqa_kv_owned_reduce_20260820.md:117)
SHAPES = [(1, 1, 1, 128, 128, 1), (1, 4, 2, 128, 128, 1)]


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args(argv)
    tool = os.path.join(args.reference, "scripts", "generate_full_bwd_golden.py")
    if not os.path.isfile(tool):
        raise SystemExit(f"reference cache tool not found: {tool}")
    shutil.rmtree(OUT, ignore_errors=True)
    os.makedirs(OUT)
    for b, h, hkv, s, d, causal in SHAPES:
        cmd = [sys.executable, tool, "--root", OUT, "--batch", str(b), "--heads", str(h),
               "--heads-kv", str(hkv), "--seqlen", str(s), "--dim", str(d),
               "--causal", str(causal)]
        print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
