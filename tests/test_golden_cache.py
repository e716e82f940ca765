"""Golden-cache format (reference scripts/generate_full_bwd_golden.py:15-18,
60-132, 222-290): round trip through flash-attention3_amd/golden_cache.py,
the manifest and directory-name contract, and fail-closed validation of
tampered caches.  CPU only."""
import hashlib
import json
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

import golden_cache as GC

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden_cache as MK  # noqa: E402

MHA = dict(batch=1, heads_q=1, heads_kv=1, seqlen=128, head_dim=128)
GQA = dict(batch=1, heads_q=4, heads_kv=2, seqlen=128, head_dim=64)


def make(tmp_path, dims, causal=1, scale=GC.DEFAULT_SCALE):
    arrays = MK.oracle_arrays(causal=causal, scale=scale, **dims)
    return GC.write(tmp_path, arrays, causal=causal, scale=scale, **dims), arrays


def test_round_trip_and_manifest(tmp_path):
    path, arrays = make(tmp_path, MHA)
    # directory name and manifest contract of the reference tool
    assert path.name == "v1_b1_h1_s128_d128_c1_scale" + struct.pack(
        "<f", np.float32(GC.DEFAULT_SCALE)).hex()
    m = json.loads((path / "manifest.json").read_text())
    assert m["schema"] == "shaobo-fa3-bwd-golden-v1"
    assert m["formula_version"] == "deterministic-bhsd-fp16-v1"
    assert m["shape"] == {"batch": 1, "heads": 1, "seqlen_q": 128, "seqlen_k": 128,
                          "head_dim_qk": 128, "head_dim_v": 128}
    assert m["layout"] == "BHSD-contiguous" and m["causal"] == 1
    assert m["softmax_scale_f32_bits"] == "f304b53d"  # fp32(1/sqrt(128)) little-endian
    assert sorted(m["files"]) == sorted(GC.file_specs(**MHA))
    # per-file hash is the SHA-256 of the raw bytes; payload digest over sorted records
    h = hashlib.sha256((path / "dq.f32").read_bytes()).hexdigest()
    assert m["files"]["dq.f32"]["sha256"] == h
    rec = b"".join(n.encode() + b"\0" + m["files"][n]["sha256"].encode() + b"\n"
                   for n in sorted(m["files"]))
    assert m["payload_sha256"] == hashlib.sha256(rec).hexdigest()
    # raw little-endian BHSD arrays
    assert (path / "q.f16").stat().st_size == 128 * 128 * 2
    back = GC.read(path, causal=1, **MHA)
    for name in arrays:
        np.testing.assert_array_equal(back[name], arrays[name].reshape(back[name].shape))
    # packed sidecar = [max * scale * log2 e, 1 / sum, delta]
    pk = back["packed_sidecar.f32"]
    sl2 = np.float32(np.float32(GC.DEFAULT_SCALE) * np.float32(1.4426950408889634))
    np.testing.assert_array_equal(pk[..., 0], back["scores_max.f32"] * sl2)
    np.testing.assert_array_equal(pk[..., 1], np.float32(1) / back["scores_sum.f32"])
    np.testing.assert_array_equal(pk[..., 2], back["delta.f32"])


def test_gqa_schema_and_key(tmp_path):
    path, _ = make(tmp_path, GQA, causal=0, scale=0.125)
    assert path.name == "v2_b1_hq4_hkv2_s128_d64_c0_scale0000003e"
    m = GC.validate(path, causal=0, scale=0.125, **GQA)
    assert m["schema"] == "shaobo-fa3-bwd-golden-v2-gqa"
    assert m["formula_version"] == "deterministic-bhsd-fp16-gqa-v1"
    assert m["shape"]["heads_q"] == 4 and m["shape"]["heads_kv"] == 2
    assert m["files"]["dk.f32"]["shape"] == [1, 2, 128, 64]


def test_existing_cache_is_kept(tmp_path):
    path, arrays = make(tmp_path, MHA)
    t0 = (path / "manifest.json").stat().st_mtime_ns
    assert GC.write(tmp_path, arrays, causal=1, **MHA) == path
    assert (path / "manifest.json").stat().st_mtime_ns == t0
    assert GC.write(tmp_path, arrays, causal=1, regenerate=True, **MHA) == path
    assert not [p for p in os.listdir(tmp_path) if p.startswith(".")]  # no temp dirs left


@pytest.mark.parametrize("damage", ["flip_byte", "truncate", "remove", "contract", "extra_file",
                                    "digest"])
def test_tampered_cache_fails_closed(tmp_path, damage):
    path, _ = make(tmp_path, MHA)
    mpath = path / "manifest.json"
    m = json.loads(mpath.read_text())
    if damage == "flip_byte":
        raw = bytearray((path / "dk.f32").read_bytes())
        raw[100] ^= 1
        (path / "dk.f32").write_bytes(bytes(raw))
    elif damage == "truncate":
        raw = (path / "v.f16").read_bytes()
        (path / "v.f16").write_bytes(raw[:-2])
    elif damage == "remove":
        os.remove(path / "delta.f32")
    elif damage == "contract":
        m["causal"] = 0
        mpath.write_text(json.dumps(m))
    elif damage == "extra_file":
        m["files"]["extra.f32"] = m["files"]["delta.f32"]
        mpath.write_text(json.dumps(m))
    elif damage == "digest":
        m["payload_sha256"] = "0" * 64
        mpath.write_text(json.dumps(m))
    with pytest.raises(GC.GoldenCacheError):
        GC.validate(path, causal=1, **MHA)


def test_wrong_problem_is_rejected(tmp_path):
    path, _ = make(tmp_path, MHA)
    with pytest.raises(GC.GoldenCacheError):
        GC.validate(path, causal=1, scale=0.1, **MHA)


def test_command_line_tool(tmp_path):
    tool = os.path.join(HERE, "golden", "make_golden_cache.py")
    args = [sys.executable, tool, "--root", str(tmp_path), "--heads", "2", "--seqlen", "128"]
    out1 = subprocess.run(args, check=True, capture_output=True, text=True).stdout
    out2 = subprocess.run(args, check=True, capture_output=True, text=True).stdout
    assert "golden_cache_status=MISS" in out1 and "golden_cache_status=HIT" in out2
    digest = [line for line in out1.splitlines() if line.startswith("golden_payload_sha256=")]
    assert digest and digest[0] in out2


# ---- caches written by the reference's own tool ----------------------------
# Fixtures made by tests/golden/make_reference_caches.py, which runs the
# reference's scripts/generate_full_bwd_golden.py (build container only).
REF_CACHES = os.path.join(HERE, "golden", "reference_caches")
REF_SHAPES = [dict(batch=1, heads_q=1, heads_kv=1, seqlen=128, head_dim=128),
              dict(batch=1, heads_q=4, heads_kv=2, seqlen=128, head_dim=128)]


def ref_cache(dims, causal=1):
    return os.path.join(REF_CACHES, GC.cache_key(causal=causal, **dims))


@pytest.mark.parametrize("dims", REF_SHAPES, ids=["mha", "gqa"])
def test_reference_tool_cache_is_read(dims):
    """The reference tool's cache sits under the directory name cache_key
    computes, and validate / read accept it unchanged (manifest contract,
    file set, dtypes, shapes, per-file and payload SHA-256)."""
    path = ref_cache(dims)
    assert os.path.isdir(path), path
    GC.validate(path, causal=1, **dims)
    a = GC.read(path, causal=1, **dims)
    assert set(a) == set(GC.file_specs(**dims))
    # its packed sidecar is the one golden_cache derives from the row stats
    want = GC.packed_sidecar(a["scores_max.f32"], a["scores_sum.f32"], a["delta.f32"],
                             GC.DEFAULT_SCALE)
    np.testing.assert_array_equal(a["packed_sidecar.f32"], want)


@pytest.mark.parametrize("dims", REF_SHAPES, ids=["mha", "gqa"])
def test_our_writer_reproduces_reference_cache(tmp_path, dims):
    """golden_cache.write, given the reference cache's arrays, writes the same
    bytes: identical per-file SHA-256, payload digest and manifest."""
    a = GC.read(ref_cache(dims), causal=1, **dims)
    ours = GC.write(tmp_path, a, causal=1, **dims)
    theirs = json.loads(open(os.path.join(ref_cache(dims), "manifest.json")).read())
    mine = json.loads((ours / "manifest.json").read_text())
    assert mine == theirs


@pytest.mark.parametrize("dims", REF_SHAPES, ids=["mha", "gqa"])
def test_oracle_against_reference_cache(dims):
    """The oracle on the reference's deterministic pattern: its inputs equal
    the cache's .f16 files bit for bit, and its outputs meet the reference's
    own gates (src/full_bwd_correctness.cpp:471-500) and the north-star bar
    against the tool's fp32 results; O differs by at most one fp16 ulp and the
    row statistics agree to fp32 rounding (numpy sums in another order)."""
    import fa3_oracle as O
    a = GC.read(ref_cache(dims), causal=1, **dims)
    B, Hq, Hkv, S, D = (dims[k] for k in ("batch", "heads_q", "heads_kv", "seqlen", "head_dim"))
    g = O.golden(B, Hq, Hkv, S, D, True, scale=GC.DEFAULT_SCALE, kind="pattern")
    for ours, theirs in (("q", "q.f16"), ("k", "k.f16"), ("v", "v.f16"), ("dout", "dout.f16")):
        np.testing.assert_array_equal(g[ours].view(np.uint16), a[theirs].view(np.uint16))
    ulp = np.abs(g["out"].view(np.int16).astype(np.int32) - a["o.f16"].view(np.int16).astype(np.int32))
    assert ulp.max() <= 1
    np.testing.assert_allclose(g["scores_max"], a["scores_max.f32"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(g["scores_sum"], a["scores_sum.f32"], rtol=1e-5)
    for n in ("delta", "dq", "dk", "dv"):
        m = O.metrics(g[n], a[n + ".f32"])
        ok, ref_ok = O.gates(n, m)
        assert ok and ref_ok, (n, m)
