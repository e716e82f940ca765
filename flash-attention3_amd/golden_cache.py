"""Reader / writer of the reference's golden-cache directory format.

A cache directory holds one backward problem as raw little-endian arrays plus
a ``manifest.json`` (reference scripts/generate_full_bwd_golden.py:15-18,
60-132, 222-290; read by the reference harness src/full_bwd_correctness.cpp:
82-100, 200-224):

* arrays (BHSD, C order): ``q.f16 k.f16 v.f16 o.f16 dout.f16`` (fp16),
  ``scores_max.f32 scores_sum.f32 delta.f32`` ([B, Hq, S]),
  ``packed_sidecar.f32`` ([B, Hq, S, 3] = [max * scale * log2 e, 1 / sum,
  delta]), ``dq.f32 dk.f32 dv.f32`` (fp32 gradients);
* manifest: the problem contract (schema ``shaobo-fa3-bwd-golden-v1`` when
  Hq == Hkv, ``...-v2-gqa`` otherwise; shape, causal flag, layout, dtypes,
  the fp32 bits of the softmax scale), and per file its dtype, shape, byte
  count and SHA-256, plus ``payload_sha256`` = SHA-256 over the sorted
  ``name NUL sha256 LF`` records.

Directory names follow the reference's cache key, so a cache written here is
found by the reference's tooling and vice versa.  Writing is atomic (a
temporary directory renamed into place); validation fails closed on any
mismatch.  The format is kept identical on purpose: it is an interchange
format between the two implementations.
"""
import hashlib
import json
import os
import shutil
import struct
import tempfile
from pathlib import Path

import numpy as np

SCHEMA_MHA = "shaobo-fa3-bwd-golden-v1"
FORMULA_MHA = "deterministic-bhsd-fp16-v1"
SCHEMA_GQA = "shaobo-fa3-bwd-golden-v2-gqa"
FORMULA_GQA = "deterministic-bhsd-fp16-gqa-v1"
DEFAULT_SCALE = 0.08838834764831845  # 1 / sqrt(128), the reference tool's default


class GoldenCacheError(RuntimeError):
    """A cache directory that does not match its contract."""


def _scale_bits(scale):
    return struct.pack("<f", np.float32(scale)).hex()


def _sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            h.update(block)
    return h.hexdigest()


def payload_sha256(files):
    """Digest over the per-file hashes, in file-name order."""
    h = hashlib.sha256()
    for name in sorted(files):
        h.update(name.encode("utf-8") + b"\0" + str(files[name]["sha256"]).encode("ascii") + b"\n")
    return h.hexdigest()


def contract(batch, heads_q, heads_kv, seqlen, head_dim, causal, scale=DEFAULT_SCALE):
    """The manifest's problem description (everything but the file table)."""
    shape = {"batch": batch}
    if heads_q == heads_kv:
        shape["heads"] = heads_q
    else:
        shape["heads_q"] = heads_q
        shape["heads_kv"] = heads_kv
    shape.update(seqlen_q=seqlen, seqlen_k=seqlen, head_dim_qk=head_dim, head_dim_v=head_dim)
    mha = heads_q == heads_kv
    return {
        "schema": SCHEMA_MHA if mha else SCHEMA_GQA,
        "formula_version": FORMULA_MHA if mha else FORMULA_GQA,
        "shape": shape,
        "causal": int(bool(causal)),
        "layout": "BHSD-contiguous",
        "input_dtype": "float16",
        "output_dtype": "float32",
        "softmax_scale_f32_bits": _scale_bits(scale),
    }


def cache_key(batch, heads_q, heads_kv, seqlen, head_dim, causal, scale=DEFAULT_SCALE):
    """Directory name of a problem inside a cache root."""
    c, sb = int(bool(causal)), _scale_bits(scale)
    if heads_q == heads_kv:
        return f"v1_b{batch}_h{heads_q}_s{seqlen}_d{head_dim}_c{c}_scale{sb}"
    return f"v2_b{batch}_hq{heads_q}_hkv{heads_kv}_s{seqlen}_d{head_dim}_c{c}_scale{sb}"


def file_specs(batch, heads_q, heads_kv, seqlen, head_dim):
    """name -> (numpy dtype string, shape) of every array in a cache."""
    qs = [batch, heads_q, seqlen, head_dim]
    ks = [batch, heads_kv, seqlen, head_dim]
    rows = [batch, heads_q, seqlen]
    specs = {n: ("<f2", qs) for n in ("q.f16", "o.f16", "dout.f16")}
    specs.update({n: ("<f2", ks) for n in ("k.f16", "v.f16")})
    specs.update({n: ("<f4", rows) for n in ("scores_max.f32", "scores_sum.f32", "delta.f32")})
    specs["packed_sidecar.f32"] = ("<f4", rows + [3])
    specs["dq.f32"] = ("<f4", qs)
    specs.update({n: ("<f4", ks) for n in ("dk.f32", "dv.f32")})
    return specs


def packed_sidecar(scores_max, scores_sum, delta, scale):
    """[max * scale * log2 e, 1 / sum (0 where sum == 0), delta] per row."""
    scale_log2 = np.float32(np.float32(scale) * np.float32(1.4426950408889634))
    out = np.empty(scores_max.shape + (3,), np.float32)
    out[..., 0] = scores_max.astype(np.float32) * scale_log2
    ssum = scores_sum.astype(np.float32)
    with np.errstate(divide="ignore"):
        out[..., 1] = np.where(ssum != 0, np.float32(1.0) / ssum, np.float32(0.0))
    out[..., 2] = delta
    return out


def write(root, arrays, *, batch, heads_q, heads_kv, seqlen, head_dim, causal,
          scale=DEFAULT_SCALE, regenerate=False):
    """Write `arrays` (name -> numpy array, the names of file_specs; a missing
    packed_sidecar.f32 is derived) as a cache under `root`; returns the cache
    directory.  An existing directory is validated and kept unless
    `regenerate`."""
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    dims = dict(batch=batch, heads_q=heads_q, heads_kv=heads_kv, seqlen=seqlen,
                head_dim=head_dim)
    final = root / cache_key(causal=causal, scale=scale, **dims)
    if final.exists():
        if not regenerate:
            validate(final, causal=causal, scale=scale, **dims)
            return final
        shutil.rmtree(final)
    arrays = dict(arrays)
    if "packed_sidecar.f32" not in arrays:
        arrays["packed_sidecar.f32"] = packed_sidecar(arrays["scores_max.f32"],
                                                      arrays["scores_sum.f32"],
                                                      arrays["delta.f32"], scale)
    specs = file_specs(**dims)
    if set(arrays) != set(specs):
        raise GoldenCacheError(f"arrays {sorted(arrays)} != cache files {sorted(specs)}")
    tmp = Path(tempfile.mkdtemp(prefix=f".{final.name}.tmp-", dir=root))
    try:
        files = {}
        for name, (dtype, shape) in specs.items():
            a = np.ascontiguousarray(arrays[name], dtype=np.dtype(dtype))
            if list(a.shape) != shape:
                raise GoldenCacheError(f"{name}: shape {list(a.shape)} != {shape}")
            a.tofile(tmp / name)
            files[name] = {"dtype": dtype, "shape": shape, "nbytes": a.nbytes,
                           "sha256": _sha256(tmp / name)}
        manifest = contract(causal=causal, scale=scale, **dims)
        manifest["files"] = files
        manifest["payload_sha256"] = payload_sha256(files)
        (tmp / "manifest.json").write_text(json.dumps(manifest, indent=2, sort_keys=True) + "\n",
                                           encoding="utf-8")
        os.replace(tmp, final)
    except BaseException:
        shutil.rmtree(tmp, ignore_errors=True)
        raise
    return final


def validate(cache_dir, *, batch, heads_q, heads_kv, seqlen, head_dim, causal,
             scale=DEFAULT_SCALE):
    """Check a cache against the expected problem: contract fields, file set,
    per-file dtype / shape / size / SHA-256 and the payload digest.  Returns
    the manifest; raises GoldenCacheError on the first mismatch."""
    cache_dir = Path(cache_dir)
    mpath = cache_dir / "manifest.json"
    if not mpath.is_file():
        raise GoldenCacheError(f"missing manifest: {mpath}")
    manifest = json.loads(mpath.read_text(encoding="utf-8"))
    dims = dict(batch=batch, heads_q=heads_q, heads_kv=heads_kv, seqlen=seqlen,
                head_dim=head_dim)
    for key, want in contract(causal=causal, scale=scale, **dims).items():
        if manifest.get(key) != want:
            raise GoldenCacheError(f"manifest {key}: expected {want!r}, found {manifest.get(key)!r}")
    files = manifest.get("files")
    if not isinstance(files, dict) or not files:
        raise GoldenCacheError("manifest has no file table")
    specs = file_specs(**dims)
    if set(files) != set(specs):
        raise GoldenCacheError(f"file set {sorted(files)} != {sorted(specs)}")
    for name, meta in files.items():
        dtype, shape = specs[name]
        nbytes = int(np.prod(shape)) * np.dtype(dtype).itemsize
        path = cache_dir / name
        if meta.get("dtype") != dtype or meta.get("shape") != shape:
            raise GoldenCacheError(f"{name}: dtype / shape differ from the contract")
        if meta.get("nbytes") != nbytes:
            raise GoldenCacheError(f"{name}: byte count differs from the contract")
        if not path.is_file():
            raise GoldenCacheError(f"missing payload {path}")
        if path.stat().st_size != nbytes:
            raise GoldenCacheError(f"{name}: file size {path.stat().st_size} != {nbytes}")
        if _sha256(path) != meta.get("sha256"):
            raise GoldenCacheError(f"{name}: SHA-256 mismatch")
    if payload_sha256(files) != manifest.get("payload_sha256"):
        raise GoldenCacheError("payload digest mismatch")
    return manifest


def read(cache_dir, *, batch, heads_q, heads_kv, seqlen, head_dim, causal,
         scale=DEFAULT_SCALE):
    """Validate, then load every array (name -> numpy array)."""
    dims = dict(batch=batch, heads_q=heads_q, heads_kv=heads_kv, seqlen=seqlen,
                head_dim=head_dim)
    validate(cache_dir, causal=causal, scale=scale, **dims)
    return {name: np.fromfile(Path(cache_dir) / name, dtype=np.dtype(dtype)).reshape(shape)
            for name, (dtype, shape) in file_specs(**dims).items()}


def lse_from(scores_max, scores_sum, scale):
    """Natural-log LSE from the cache's row statistics, as the reference
    harness forms it (src/full_bwd_correctness.cpp:229-233)."""
    return (scores_max.astype(np.float32) * np.float32(scale)
            + np.log(scores_sum.astype(np.float32))).astype(np.float32)
