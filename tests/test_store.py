"""Host-side store: GOSSMX4 repack containers (cpu_repack.rs), the cache key
(SourceIdentity::cache_key, cpu_repack.rs:92-107) and SafeTensors shard
parsing (cpu_tensor_store.rs:176-288). No device access; the containers and
checkpoints are written here in the reference's formats by independent
Python code (hashlib, json, the safetensors package)."""
import hashlib
import json
import struct

import numpy as np
import pytest
import safetensors.numpy

import gossmx as G

MAGIC = b"GOSSMX4\0"


def reference_cache_key(tensor_name, shape, layout, model_revision, hashes):
    # cpu_repack.rs:92-107, in the reference's update order.
    names = {1: "CanonicalAdjacentV1", 2: "InterleavedSplitX8V2", 3: "GpuTiledV3"}
    d = hashlib.sha256()
    d.update(b"gpt-oss-rs-mxfp4-repack")
    d.update(struct.pack("<I", 1))
    d.update(names[layout].encode())
    d.update(struct.pack("<I", layout))
    d.update(model_revision.encode())
    for h in hashes:
        d.update(h.encode())
    d.update(tensor_name.encode())
    for dim in shape:
        d.update(struct.pack("<Q", dim))
    return d.hexdigest()


def test_cache_key_follows_the_reference_recipe():
    # Tensor names of every length 0..130 put the message length at every
    # residue mod 64 (SHA-256 padding cases: 55, 56, 63, 64 bytes and more).
    for n in range(131):
        name = "t" * n
        for layout in (1, 2, 3):
            want = reference_cache_key(name, (32, 5760, 90), layout, "rev-abc", ["a.safetensors:00ff", "b:11"])
            assert G.repack_cache_key(name, (32, 5760, 90), layout, "rev-abc", ["a.safetensors:00ff", "b:11"]) == want
    assert G.repack_cache_key("x", (1, 2, 3), 1, "", []) == reference_cache_key("x", (1, 2, 3), 1, "", [])


def test_cache_key_rejects_unknown_layout():
    with pytest.raises(G.GossmxError) as e:
        G.repack_cache_key("x", (1, 2, 3), 7, "r", [])
    assert e.value.status == G.ERR_INVALID_ARGUMENT


def reference_header(layout, shape, tensor_name="model.layers.0.mlp.experts.gate_up_proj_blocks",
                     model_revision="rev", hashes=("shard.safetensors:abcd",)):
    ident = {1: "CanonicalAdjacentV1", 2: "InterleavedSplitX8V2", 3: "GpuTiledV3"}[layout]
    # serde_json::to_vec of RepackHeader: compact, declaration order.
    return {"format_version": 1, "layout_version": layout, "layout_identifier": ident, "tensor_name": tensor_name,
            "model_revision": model_revision, "source_hashes": list(hashes), "shape": list(shape),
            "records": int(np.prod(shape))}


def write_container(path, header, payload):
    text = json.dumps(header, separators=(",", ":"), ensure_ascii=False).encode()
    with open(path, "wb") as f:
        f.write(MAGIC + struct.pack("<Q", len(text)) + text + bytes(payload))
    return 16 + len(text)


def test_inspect_reads_a_reference_container(tmp_path):
    shape = (2, 40, 3)
    header = reference_header(1, shape)
    payload = np.arange(np.prod(shape) * 17, dtype=np.uint64).astype(np.uint8)
    path = tmp_path / "weights.repack"
    offset = write_container(path, header, payload)
    info = G.repack_inspect(str(path))
    assert info["format_version"] == 1 and info["layout_version"] == 1
    assert (info["experts"], info["rows"], info["blocks"]) == shape
    assert info["records"] == 240 and info["payload_offset"] == offset and info["payload_bytes"] == 240 * 17
    assert info["tensor_name"] == header["tensor_name"]


@pytest.mark.parametrize("case", ["magic", "truncated_header", "short_payload", "long_payload", "layout",
                                  "records", "json", "missing_field"])
def test_inspect_rejects_malformed_containers(tmp_path, case):
    shape = (1, 8, 2)
    header = reference_header(1, shape)
    payload = bytes(np.prod(shape) * 17)
    path = tmp_path / "bad.repack"
    if case == "layout":
        header["layout_identifier"] = "CanonicalAdjacentV9"
    if case == "records":
        header["records"] = 15
    if case == "missing_field":
        del header["model_revision"]
    if case == "short_payload":
        payload = payload[:-1]
    if case == "long_payload":
        payload = payload + b"\0"
    write_container(path, header, payload)
    if case == "magic":
        data = bytearray(path.read_bytes())
        data[0:8] = b"GOSSMX3\0"
        path.write_bytes(bytes(data))
    if case == "truncated_header":
        path.write_bytes(path.read_bytes()[:30])
    if case == "json":
        data = bytearray(path.read_bytes())
        data[16] = ord("[")
        path.write_bytes(bytes(data))
    with pytest.raises(G.GossmxError) as e:
        G.repack_inspect(str(path))
    assert e.value.status == G.ERR_BAD_FILE


def test_inspect_accepts_unknown_header_fields_and_escapes(tmp_path):
    # serde ignores unknown fields; names may hold escaped and non-ASCII text.
    shape = (1, 16, 1)
    header = reference_header(2, shape, tensor_name='w"\\é中\n', hashes=())
    header["extra"] = {"nested": [1, 2.5, None, True]}
    write_container(tmp_path / "w.repack", header, bytes(16 * 17))
    info = G.repack_inspect(str(tmp_path / "w.repack"))
    assert info["tensor_name"] == 'w"\\é中\n' and info["layout_version"] == 2


def test_safetensors_find_matches_the_file(tmp_path):
    blocks = np.arange(2 * 3 * 4 * 16, dtype=np.uint8).reshape(2, 3, 4, 16)
    bias = np.linspace(-1, 1, 7, dtype=np.float32)
    path = tmp_path / "model-00001.safetensors"
    safetensors.numpy.save_file({"experts.gate_up_proj_blocks": blocks, "experts.bias": bias}, str(path),
                                metadata={"format": "pt"})
    raw = path.read_bytes()
    header_len = struct.unpack("<Q", raw[:8])[0]
    meta = json.loads(raw[8:8 + header_len])
    for name, arr, dtype in (("experts.gate_up_proj_blocks", blocks, "U8"), ("experts.bias", bias, "F32")):
        t = G.safetensors_find(str(path), name)
        assert t["dtype"] == dtype and t["shape"] == arr.shape
        assert t["offset"] == 8 + header_len + meta[name]["data_offsets"][0]
        assert raw[t["offset"]:t["offset"] + t["bytes"]] == arr.tobytes()
    with pytest.raises(G.GossmxError) as e:
        G.safetensors_find(str(path), "missing")
    assert e.value.status == G.ERR_BAD_FILE


@pytest.mark.parametrize("case", ["byte_count", "range", "dtype", "header_len"])
def test_safetensors_rejects_inconsistent_headers(tmp_path, case):
    meta = {"t": {"dtype": "U8", "shape": [2, 3], "data_offsets": [0, 6]}}
    data = bytes(range(6))
    if case == "byte_count":
        meta["t"]["shape"] = [2, 4]
    if case == "range":
        meta["t"]["data_offsets"] = [0, 7]
    if case == "dtype":
        meta["t"]["dtype"] = "X9"
    text = json.dumps(meta).encode()
    blob = struct.pack("<Q", len(text)) + text + data
    if case == "header_len":
        blob = struct.pack("<Q", len(blob)) + blob[8:]
    path = tmp_path / "bad.safetensors"
    path.write_bytes(blob)
    with pytest.raises(G.GossmxError) as e:
        G.safetensors_find(str(path), "t")
    assert e.value.status == G.ERR_BAD_FILE


# --- truncated and corrupted files: every truncation of a valid file and
# every single-byte corruption of its header either fails with
# GOSSMX_ERR_BAD_FILE or yields a geometry that lies inside the file (run
# under AddressSanitizer/UBSan by tests/test_sanitize.py) ---

CORRUPTIONS = (0x01, 0x22, 0x80, 0xFF)


def _valid_container(tmp_path):
    shape = (2, 8, 3)
    header = reference_header(1, shape, hashes=("a.safetensors:00ff", "b:11"))
    payload = (np.arange(np.prod(shape) * 17) % 251).astype(np.uint8).tobytes()
    path = tmp_path / "w.repack"
    offset = write_container(path, header, payload)
    return path, path.read_bytes(), offset


def test_repack_truncated_at_every_length_is_rejected(tmp_path):
    path, raw, _ = _valid_container(tmp_path)
    G.repack_inspect(str(path))
    for n in range(len(raw)):
        path.write_bytes(raw[:n])
        with pytest.raises(G.GossmxError) as e:
            G.repack_inspect(str(path))
        assert e.value.status == G.ERR_BAD_FILE, n


def test_repack_header_byte_corruptions_are_rejected_or_consistent(tmp_path):
    path, raw, offset = _valid_container(tmp_path)
    for i in range(offset):
        for flip in CORRUPTIONS:
            data = bytearray(raw)
            data[i] ^= flip
            path.write_bytes(bytes(data))
            try:
                info = G.repack_inspect(str(path))
            except G.GossmxError as e:
                assert e.status == G.ERR_BAD_FILE, (i, flip)
                continue
            # accepted: a changed name or hash string, never a geometry past the file
            assert info["payload_offset"] + info["payload_bytes"] == len(data), (i, flip)
            assert info["records"] == info["experts"] * info["rows"] * info["blocks"], (i, flip)


def _valid_safetensors(tmp_path):
    blocks = (np.arange(2 * 3 * 4 * 16) % 256).astype(np.uint8).reshape(2, 3, 4, 16)
    bias = np.linspace(-1, 1, 7, dtype=np.float32)
    path = tmp_path / "model.safetensors"
    safetensors.numpy.save_file({"experts.gate_up_proj_blocks": blocks, "experts.bias": bias}, str(path),
                                metadata={"format": "pt"})
    raw = path.read_bytes()
    return path, raw, 8 + struct.unpack("<Q", raw[:8])[0]


def test_safetensors_truncated_at_every_length_is_rejected(tmp_path):
    path, raw, data_start = _valid_safetensors(tmp_path)
    for n in range(len(raw)):
        path.write_bytes(raw[:n])
        for name in ("experts.gate_up_proj_blocks", "experts.bias"):
            with pytest.raises(G.GossmxError) as e:
                G.safetensors_find(str(path), name)
            assert e.value.status == G.ERR_BAD_FILE, (n, name)


def test_safetensors_header_byte_corruptions_are_rejected_or_consistent(tmp_path):
    path, raw, data_start = _valid_safetensors(tmp_path)
    sizes = {"U8": 1, "F32": 4, "BF16": 2, "F16": 2, "I8": 1, "I32": 4, "F64": 8, "I64": 8, "U16": 2, "I16": 2,
             "U32": 4, "U64": 8, "BOOL": 1}
    for i in range(data_start):
        for flip in CORRUPTIONS:
            data = bytearray(raw)
            data[i] ^= flip
            path.write_bytes(bytes(data))
            for name in ("experts.gate_up_proj_blocks", "experts.bias"):
                try:
                    t = G.safetensors_find(str(path), name)
                except G.GossmxError as e:
                    assert e.status == G.ERR_BAD_FILE, (i, flip, name)
                    continue
                assert t["offset"] >= data_start and t["offset"] + t["bytes"] <= len(data), (i, flip, name)
                assert int(np.prod(t["shape"])) * sizes.get(t["dtype"], 0) == t["bytes"], (i, flip, name)


@pytest.mark.parametrize("case", ["tiny_file", "header_len_overflow", "header_past_file", "offset_overflow",
                                  "start_after_end", "shape_overflow", "not_an_object", "offsets_missing"])
def test_safetensors_rejects_the_reference_edge_cases(tmp_path, case):
    # parse_shard_header's checks (cpu_tensor_store.rs:200-288): a file under
    # 8 bytes, 8 + header_len overflowing or past the file, offsets that
    # overflow or run backwards, a shape whose element count overflows, and
    # headers that are not the expected JSON shapes.
    meta = {"t": {"dtype": "U8", "shape": [2, 3], "data_offsets": [0, 6]}}
    data = bytes(range(6))
    if case == "offset_overflow":
        meta["t"]["data_offsets"] = [0, 2 ** 64 - 4]
    if case == "start_after_end":
        meta["t"]["data_offsets"] = [6, 0]
    if case == "shape_overflow":
        meta["t"]["shape"] = [2 ** 33, 2 ** 33, 2 ** 33]
    if case == "offsets_missing":
        del meta["t"]["data_offsets"]
    text = json.dumps(meta).encode()
    if case == "not_an_object":
        text = b'[{"dtype": "U8"}]'
    blob = struct.pack("<Q", len(text)) + text + data
    if case == "tiny_file":
        blob = blob[:7]
    if case == "header_len_overflow":
        blob = struct.pack("<Q", 2 ** 64 - 3) + blob[8:]
    if case == "header_past_file":
        blob = struct.pack("<Q", len(blob)) + blob[8:]
    path = tmp_path / "edge.safetensors"
    path.write_bytes(blob)
    with pytest.raises(G.GossmxError) as e:
        G.safetensors_find(str(path), "t")
    assert e.value.status == G.ERR_BAD_FILE


@pytest.mark.parametrize("raw,ok", [(b"\xc3\xa9", True), (b"\xe4\xb8\xad", True), (b"\xf0\x9f\x98\x80", True),
                                    (b"\xc3\x28", False), (b"\xc0\xaf", False), (b"\xed\xa0\x80", False),
                                    (b"\xf4\x90\x80\x80", False), (b"\xe4\xb8", False), (b"\x80", False)])
def test_repack_header_strings_must_be_utf8(tmp_path, raw, ok):
    # serde_json::from_slice rejects a header whose string bytes are not
    # UTF-8 (overlong forms, surrogates, code points past U+10FFFF, cut or
    # stray continuation bytes).
    shape = (1, 16, 1)
    text = json.dumps(reference_header(1, shape, tensor_name="@"), separators=(",", ":")).encode()
    text = text.replace(b'"@"', b'"w' + raw + b'"')
    path = tmp_path / "u.repack"
    path.write_bytes(MAGIC + struct.pack("<Q", len(text)) + text + bytes(16 * 17))
    if ok:
        assert G.repack_inspect(str(path))["tensor_name"] == ("w" + raw.decode())
    else:
        with pytest.raises(G.GossmxError) as e:
            G.repack_inspect(str(path))
        assert e.value.status == G.ERR_BAD_FILE
