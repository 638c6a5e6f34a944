"""Test-side writers of the reference's on-disk formats, byte for byte:

  * HGRAV* containers: wrap_container of the reference's own tests
    (crates/hawking-core/src/model/qwen_complete_binary/q80_mixed_decode.rs:1496-1506)
    with the header fields its parse_* functions read (823-1070);
  * HQ30UQ4 / HQ30G1B1 payloads with their 32-byte headers
    (qwen_complete_binary/uniform_q4.rs:57-150, qwen_complete_binary/mod.rs:137-233);
  * the HQ80M15 catalog + manifest (write_catalog,
    lab/operators/q80_mixed_representation_pack.py:631-712, and the manifest
    fields Qwen80MixedStreamingCatalog::open_manifest reads,
    model/qwen80_mixed_catalog.rs:176-263).

Bodies come from the oracle's packers (the canonical arrays)."""
from __future__ import annotations

import hashlib
import json
import struct
from pathlib import Path

import numpy as np

SCHEMA_BINARY = "hawking.gravity.binary_sign_scale.v1"
SCHEMA_RESIDUAL = "hawking.gravity.binary_outlier_residual.v2"
SCHEMA_HGRAVS01 = "hawking.gravity.activation_weighted_svd_low_rank.v1"
SCHEMA_UNIFORM = "hawking.gravity.uniform_group.v1"
CATALOG_SCHEMA = "hawking.ascension.qwen80_mixed_representation_candidate.v1"


def wrap(magic: bytes, header: dict, body: bytes) -> bytes:
    h = json.dumps(header, separators=(",", ":")).encode()
    return magic + struct.pack("<I", len(h)) + h + body


def binary(scales: np.ndarray, signs: np.ndarray, rows: int, cols: int, **override) -> bytes:
    hdr = {"schema": SCHEMA_BINARY, "representation": "binary_sign_scale", "shape": [rows, cols],
           "elements": rows * cols, "group_size": 128, "groups": int(scales.size), "scale_bytes": int(scales.size) * 2,
           "sign_bytes": int(signs.size)}
    hdr.update(override)
    return wrap(b"HGRAVB01", hdr, scales.astype("<u2").tobytes() + signs.tobytes())


def residual(p, **override) -> bytes:
    """p: the oracle's RiceQ1 (rice_q1_pack)."""
    body = (p.bin_scales.astype("<u2").tobytes() + p.bin_signs.tobytes() + struct.pack("<I", p.first) +
            p.rice.tobytes() + struct.pack("<H", p.res_scale) + p.res_signs.tobytes())
    hdr = {"schema": SCHEMA_RESIDUAL, "index_mode": "rice", "value_bits": 1, "value_scale": "rms",
           "shape": [p.rows, p.cols], "elements": p.rows * p.cols, "group_size": 128,
           "groups": int(p.bin_scales.size), "scale_bytes": int(p.bin_scales.size) * 2,
           "sign_bytes": int(p.bin_signs.size), "index_bytes": 4 + int(p.rice.size), "residual_scale_bytes": 2,
           "residual_bytes": int(p.res_signs.size), "outlier_count": p.count, "rice_k": p.rice_k,
           "rice_bytes": int(p.rice.size), "first_index_bytes": 4}
    hdr.update(override)
    return wrap(b"HGRAVR02", hdr, body)


def uniform8(scales: np.ndarray, codes: np.ndarray, rows: int, cols: int, **override) -> bytes:
    hdr = {"schema": SCHEMA_UNIFORM, "bits": 8, "group_size": 64, "shape": [rows, cols], "elements": rows * cols}
    hdr.update(override)
    return wrap(b"HGRAVU01", hdr, scales.astype("<u2").tobytes() + codes.tobytes())


def hgravs01(left, right, rows: int, r: int, cols: int, bits: int = 3, group: int = 64, **override) -> bytes:
    """HGRAVS01 of factors left (rows x r) and right (r x cols); header keys in
    `override` replace the written ones."""
    lb = left[0].astype("<u2").tobytes() + left[1].tobytes()
    rb = right[0].astype("<u2").tobytes() + right[1].tobytes()
    hdr = {"schema": SCHEMA_HGRAVS01, "representation": "activation_weighted_svd_low_rank_q",
           "activation_capture": {"fit_kind": "real_routed_activation_capture"},
           "matrix_shape": [rows, cols], "rank": r, "factor_bits": bits, "factor_group_size": group,
           "left_body_bytes": len(lb), "right_body_bytes": len(rb),
           "left": {"schema": SCHEMA_UNIFORM, "shape": [rows, r], "bits": bits, "group_size": group},
           "right": {"schema": SCHEMA_UNIFORM, "shape": [r, cols], "bits": bits, "group_size": group}}
    hdr.update(override)
    return wrap(b"HGRAVS01", hdr, lb + rb)


def hq30(magic: bytes, group: int, shape: list[int], scales: np.ndarray, codes: np.ndarray, version: int = 1,
         reserved: int = 0) -> bytes:
    elements = int(np.prod(shape))
    head = magic + struct.pack("<IIHHQI", version, group, len(shape), reserved, elements, 0)
    return head + b"".join(struct.pack("<I", d) for d in shape) + scales.astype("<u2").tobytes() + codes.tobytes()


def write_catalog(root: Path, tensors: list[tuple[str, int, int, list[int], bytes]], n_segments: int = 2) -> Path:
    """tensors: (name, codec, organ, shape, payload).  Payloads are spread over
    n_segments files under root/segments; returns the manifest path."""
    seg_dir = root / "segments"
    seg_dir.mkdir(parents=True, exist_ok=True)
    blobs = [bytearray() for _ in range(n_segments)]
    records = []
    for i, (name, codec, organ, shape, payload) in enumerate(tensors):
        seg = i % n_segments
        off = len(blobs[seg])
        blobs[seg].extend(payload)
        blobs[seg].extend(b"\0" * ((-len(blobs[seg])) % 16))
        records.append({"name": name, "codec": codec, "organ": organ, "shape": shape,
                        "elements": int(np.prod(shape)), "segment_id": seg, "offset": off, "nbytes": len(payload),
                        "sha256": hashlib.sha256(payload).hexdigest(), "flags": 0, "n_fit_rows": 0,
                        "achieved_rank": 0, "codec_bpw": 8.0 * len(payload) / max(int(np.prod(shape)), 1)})
    segments = []
    for s, blob in enumerate(blobs):
        fn = f"segment_{s:03d}.bin"
        (seg_dir / fn).write_bytes(bytes(blob))
        segments.append({"id": s, "filename": fn, "bytes": len(blob), "sha256": hashlib.sha256(blob).hexdigest()})
    name_blob, offs = bytearray(), []
    for r in records:
        offs.append(len(name_blob))
        name_blob.extend(r["name"].encode())
    table = bytearray()
    for r, off in zip(records, offs):
        dims = (list(r["shape"]) + [0, 0, 0, 0])[:4]
        rec = struct.pack("<IHBBBB", off, len(r["name"].encode()), r["codec"], r["organ"], len(r["shape"]), 0)
        rec += b"\0\0"
        rec += struct.pack("<IIIIQHHQQ32sIIf", *dims, r["elements"], r["segment_id"], r["achieved_rank"],
                           r["offset"], r["nbytes"], bytes.fromhex(r["sha256"]), r["flags"], r["n_fit_rows"],
                           r["codec_bpw"])
        table.extend(rec + b"\0" * (128 - len(rec)))
    seg_blob = bytearray()
    for s in segments:
        fn = s["filename"].encode()
        seg_blob.extend(struct.pack("<HHQ32s", s["id"], len(fn), s["bytes"], bytes.fromhex(s["sha256"])) + fn)
    catalog = (b"HQ80M15\0" + struct.pack("<IIIIII", 1, len(records), len(segments), 0, len(name_blob), 0) +
               bytes(seg_blob) + bytes(table) + bytes(name_blob))
    (root / "catalog.hq80m15").write_bytes(catalog)
    manifest = {"schema": CATALOG_SCHEMA, "seal_sha256": "0" * 64,
                "complete_physical_bpw_ledger": {"complete_physical_bpw": 1.4921875,
                                                 "tensor_payload_bytes": sum(len(t[4]) for t in tensors)},
                "catalog": {"path": "catalog.hq80m15", "sha256": hashlib.sha256(catalog).hexdigest()}}
    mpath = root / "QWEN80_MIXED_1P5_V1_COMPLETE_BINARY_GRAVITY_CANDIDATE.json"
    mpath.write_text(json.dumps(manifest, indent=2))
    return mpath
