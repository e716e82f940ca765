"""Fixed-seed sweep of v2 over mixed shapes and options, through the C ABI.

Each case draws one combination of the options the parity tests cover one at
a time -- fp16 / bf16, BHSD / BSHD, GQA ratio 1, 2 or 4, causal or full, head
dim 64 or 128, batch 1 or 2, S = 128 .. 1024, deterministic flag -- checks it
against the CPU oracle to the north-star bar and checks that a second call
gives bitwise the same dQ, dK, dV.
"""
import random

import numpy as np
import pytest
import torch

import fa3_oracle as O
import shaobo_fa3 as F
from gpu_util import check, log, run_v2

pytestmark = pytest.mark.gpu


def _cases(seed=7, n=24):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        D = rng.choice([64, 128])
        causal = rng.random() < 0.6
        Hkv = rng.choice([1, 1, 2, 3])
        G = rng.choice([1, 1, 2, 4])
        B = rng.choice([1, 1, 2])
        S = 128 * rng.choice([1, 2, 3, 4, 5, 6, 8])
        dtype = rng.choice(["fp16", "fp16", "bf16"])
        bshd = rng.random() < 0.3
        det = rng.random() < 0.5
        out.append((i, B, Hkv * G, Hkv, S, D, causal, dtype, bshd, det))
    return out


@pytest.mark.parametrize("i,B,Hq,Hkv,S,D,causal,dtype,bshd,det", _cases())
def test_v2_sweep(i, B, Hq, Hkv, S, D, causal, dtype, bshd, det):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    log(f"[case] sweep {i}: B={B} Hq={Hq} Hkv={Hkv} S={S} D={D} causal={causal} {dtype} "
        f"bshd={bshd} deterministic={det}")
    g = O.golden(B, Hq, Hkv, S, D, causal, dtype=dtype, seed_offset=1000 + i)
    res = run_v2(g, torch, bshd=bshd, deterministic=det)
    assert res["status"] == F.SUCCESS, F.status_name(res["status"])
    check(res, g)
    again = run_v2(g, torch, bshd=bshd, deterministic=det)
    for n in ("dq", "dk", "dv"):
        assert np.array_equal(res[n], again[n]), f"{n} differs between two calls"
