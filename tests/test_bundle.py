"""MIT2 weight bundle: the C++ loader and writer behind
mit2cfm_create_from_bundle (runtime/bundle.h), checked on the CPU.

Format and validation rules: reference docs/native_bundle.md:1-90 and
runtime/bundle.cpp:185-300.  Every case is opened by this project's loader
(mit2cfm_inspect_bundle) and, where the reference's own loader has been built
from its sources into oracle/_ref/ (oracle/ref/Makefile), by that loader too;
the two must accept and reject the same bundles.  The documented rules also
reject overlapping payloads and dtype/shape byte-count mismatches
(docs/native_bundle.md:57-68), which the reference's C++ loader leaves to its
Python validator: for those cases the reference loader's acceptance is
recorded, and this loader rejects as the document requires.
"""
from __future__ import annotations

import hashlib
import json
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
REF_INSPECT = ROOT / "oracle" / "_ref" / "bundle_inspect"


def payloads():
    rng = np.random.default_rng(11)
    return [
        ("a.weight", rng.standard_normal((4, 8)).astype(np.float16), "f16"),
        ("a.bias", rng.standard_normal(4).astype(np.float32), "f32"),
        ("b.weight_v", rng.standard_normal((3, 2, 5)).astype(np.float16), "f16"),
        ("ids", np.arange(7, dtype=np.int64), "i64"),
    ]


def layout(align=64, tensors=None):
    """(header bytes, records, blob) of a well-formed bundle."""
    tensors = payloads() if tensors is None else tensors
    blob = bytearray(b"MIT2" + struct.pack("<II", 1, align))
    recs = []
    for name, arr, dt in tensors:
        off = -(-len(blob) // align) * align
        blob.extend(b"\0" * (off - len(blob)))
        data = arr.tobytes()
        blob.extend(data)
        recs.append(dict(name=name, shape=list(arr.shape), dtype=dt, offset=off, nbytes=len(data),
                         sha256=hashlib.sha256(data).hexdigest(), layout="row_major",
                         component="test"))
    manifest = dict(format="MIT2", version=1, endianness="little", alignment=align,
                    weights_file="weights.bin", metadata={}, tensors=recs)
    return manifest, blob


def write_dir(path: Path, manifest, blob, manifest_text=None):
    path.mkdir(parents=True, exist_ok=True)
    (path / "weights.bin").write_bytes(bytes(blob))
    (path / "manifest.json").write_text(manifest_text or json.dumps(manifest, indent=1))
    return path


def write_single(path: Path, manifest, blob, footer_magic=b"MIT2VOIC", size_delta=0):
    data = bytearray(blob)
    text = json.dumps(manifest).encode()
    mo = len(data)
    data.extend(text)
    data.extend(struct.pack("<QQ", mo, len(text) + size_delta) + footer_magic)
    path.write_bytes(bytes(data))
    return path


def ours(mit2, path):
    try:
        return ("OK",) + mit2.inspect_bundle(path)
    except mit2.Mit2CfmError as e:
        assert e.status == mit2.E_MODEL
        return ("ERR",)


def reference(path):
    r = subprocess.run([str(REF_INSPECT), str(path)], capture_output=True, text=True, timeout=60)
    parts = r.stdout.split()
    return ("OK", int(parts[1]), int(parts[2])) if r.returncode == 0 else ("ERR",)


def mutate(kind, tmp: Path):
    m, blob = layout()
    t = m["tensors"]
    if kind == "valid_dir":
        return write_dir(tmp / kind, m, blob), "OK", "OK"
    if kind == "valid_single":
        return write_single(tmp / f"{kind}.mit2", m, blob), "OK", "OK"
    if kind == "extra_keys_and_spacing":
        m["producer"] = {"name": "x", "nested": [1, 2, {"k": "v"}]}
        t[0]["extra"] = [1, 2]
        text = json.dumps(m, indent=4, separators=(" ,", " :  "))
        return write_dir(tmp / kind, m, blob, text), "OK", "OK"
    if kind == "single_footer_magic":
        return write_single(tmp / f"{kind}.mit2", m, blob, b"MIT2VOIX"), "ERR", "ERR"
    if kind == "single_manifest_exceeds":
        return write_single(tmp / f"{kind}.mit2", m, blob, size_delta=10 ** 6), "ERR", "ERR"
    if kind == "format":
        m["format"] = "MIT3"
    elif kind == "version":
        m["version"] = 2
    elif kind == "alignment_zero":
        m["alignment"] = 0
    elif kind == "endianness":
        m["endianness"] = "big"
    elif kind == "weights_magic":
        blob[0:4] = b"MIT3"
    elif kind == "header_version":
        blob[4:8] = struct.pack("<I", 2)
    elif kind == "header_alignment":
        blob[8:12] = struct.pack("<I", 32)
    elif kind == "misaligned_offset":
        t[1]["offset"] += 4
    elif kind == "zero_bytes":
        t[3]["nbytes"] = 0
        t[3]["shape"] = [0]
    elif kind == "beyond_file":
        t[3]["offset"] = len(blob) // 64 * 64 + 64
    elif kind == "duplicate":
        t[2]["name"] = t[0]["name"]
    elif kind == "empty_name":
        t[1]["name"] = ""
    elif kind == "missing_tensors":
        del m["tensors"]
    elif kind == "missing_weights":
        d = write_dir(tmp / kind, m, blob)
        (d / "weights.bin").unlink()
        return d, "ERR", "ERR"
    elif kind == "overlap":
        t[1]["offset"] = t[0]["offset"]
        return write_dir(tmp / kind, m, blob), "ERR", "OK"
    elif kind == "shape_mismatch":
        t[0]["shape"] = [4, 9]
        return write_dir(tmp / kind, m, blob), "ERR", "OK"
    elif kind == "unknown_dtype":
        t[1]["dtype"] = "bf16"
        return write_dir(tmp / kind, m, blob), "ERR", "OK"
    else:
        raise KeyError(kind)
    return write_dir(tmp / kind, m, blob), "ERR", "ERR"


CASES = ["valid_dir", "valid_single", "extra_keys_and_spacing", "single_footer_magic",
         "single_manifest_exceeds", "format", "version", "alignment_zero", "endianness",
         "weights_magic", "header_version", "header_alignment", "misaligned_offset", "zero_bytes",
         "beyond_file", "duplicate", "empty_name", "missing_tensors", "missing_weights", "overlap",
         "shape_mismatch", "unknown_dtype"]


@pytest.mark.parametrize("kind", CASES)
def test_loader_accepts_and_rejects(mit2, tmp_path, kind):
    path, want_ours, want_ref = mutate(kind, tmp_path)
    got = ours(mit2, path)
    assert got[0] == want_ours, (kind, got)
    if want_ours == "OK":
        tensors = payloads()
        assert got[1:] == (len(tensors), sum(a.nbytes for _, a, _ in tensors))
    if REF_INSPECT.exists():
        ref = reference(path)
        assert ref[0] == want_ref, (kind, ref)
        if want_ref == want_ours == "OK":
            assert ref == got


def test_sha256_verification(mit2, tmp_path):
    m, blob = layout()
    d = write_dir(tmp_path / "ok", m, blob)
    assert ours(mit2, d)[0] == "OK"
    assert mit2.inspect_bundle(d, verify_sha256=True)[0] == 4
    blob[m["tensors"][2]["offset"] + 3] ^= 0x40
    d2 = write_dir(tmp_path / "bad", m, blob)
    assert mit2.inspect_bundle(d2)[0] == 4  # structure is still valid
    with pytest.raises(mit2.Mit2CfmError):
        mit2.inspect_bundle(d2, verify_sha256=True)


def test_synthetic_bundle_round_trip(mit2, tmp_path):
    """The C++ writer's bundle of every estimator tensor: the manifest matches
    the synthetic inventory, payloads equal the generator's tensors, each
    payload's sha256 matches hashlib, and both loaders accept it."""
    d = tmp_path / "synthetic"
    mit2.write_synthetic_bundle(d, 20240605, 0.02)
    man = json.loads((d / "manifest.json").read_text())
    specs = mit2.synthetic_tensor_specs()
    assert [t["name"] for t in man["tensors"]] == [s[0] for s in specs]
    tensors = mit2.synthetic_tensors(20240605, 0.02)
    raw = np.memmap(d / "weights.bin", dtype=np.uint8, mode="r")
    assert bytes(raw[:4]) == b"MIT2"
    for rec, (name, shape, dt) in zip(man["tensors"], specs):
        assert rec["shape"] == list(shape) and rec["dtype"] == dt
        assert rec["offset"] % man["alignment"] == 0
        data = bytes(raw[rec["offset"]:rec["offset"] + rec["nbytes"]])
        assert data == tensors[name].tobytes()
        assert rec["sha256"] == hashlib.sha256(data).hexdigest()
    count, nbytes = mit2.inspect_bundle(d, verify_sha256=True)
    assert count == len(specs) and nbytes == sum(t.nbytes for t in tensors.values())
    if REF_INSPECT.exists():
        assert reference(d) == ("OK", count, nbytes)


def test_sha256_known_answers(mit2, tmp_path):
    """FIPS 180-4 test vectors through the writer (payload sizes 3, 56, 64,
    1000 bytes cover the one- and two-block padding branches)."""
    vecs = [b"abc", b"abcdbcdecdefdefgefghfghighijhijkijkljklmjklmnklmnolmnopmnopqnopq",
            bytes(range(64)), bytes(i * 7 & 255 for i in range(1000))]
    for i, v in enumerate(vecs):
        arr = np.frombuffer(v, np.uint8).copy()
        m, blob = layout(tensors=[("v", arr, "u8")])
        d = write_dir(tmp_path / f"kat{i}", m, blob)
        m["tensors"][0]["sha256"] = hashlib.sha256(v).hexdigest()
        write_dir(d, m, blob)
        assert mit2.inspect_bundle(d, verify_sha256=True) == (1, len(v))
