"""Resident weights through the store paths, on the GPU: GOSSMX4 containers
of layouts 1 and 2 written in the reference's format, the resident layout 3
saved and loaded again, SafeTensors checkpoints, and open_or_create's cache
(cpu_repack.rs:149-216). Every path must give back the same canonical bytes,
and the layout-3 weights the same matmul bits."""
import json
import os
import struct

import numpy as np
import pytest
import safetensors.numpy

import gossmx as G
import oracle as O

pytestmark = pytest.mark.gpu

E, N, B = 2, 40, 3  # rows not a multiple of 8 or 16: x8 tails and a partial tile


@pytest.fixture(scope="module")
def ctx():
    c = G.Context(0)
    yield c
    c.close()


@pytest.fixture(scope="module")
def canonical():
    return O.gen_mxfp4(77, 1, E, N, B)


def container(path, layout, payload, shape=(E, N, B), name="experts.gate_up_proj_blocks"):
    ident = {1: "CanonicalAdjacentV1", 2: "InterleavedSplitX8V2"}[layout]
    header = {"format_version": 1, "layout_version": layout, "layout_identifier": ident, "tensor_name": name,
              "model_revision": "rev", "source_hashes": ["s:1"], "shape": list(shape),
              "records": int(np.prod(shape))}
    text = json.dumps(header, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(b"GOSSMX4\0" + struct.pack("<Q", len(text)) + text + bytes(payload))


def checkpoint(canonical):
    rec = canonical.reshape(E, N, B, 17)
    return np.ascontiguousarray(rec[..., 1:]), np.ascontiguousarray(rec[..., 0])


def test_reference_containers_load(ctx, canonical, tmp_path):
    container(tmp_path / "v1.repack", 1, canonical)
    x8 = np.concatenate([O.pack_x8(canonical[e * N * B * 17:(e + 1) * N * B * 17], N, B) for e in range(E)])
    container(tmp_path / "v2.repack", 2, x8)
    for name in ("v1.repack", "v2.repack"):
        w = G.Weights.load_repack(ctx, str(tmp_path / name))
        assert (w.export_canonical() == canonical).all(), name
        w.close()


def test_layout3_round_trip_and_matmul(ctx, canonical, tmp_path):
    w = G.Weights.upload(ctx, canonical, E, N, B)
    path = tmp_path / "v3.repack"
    w.save_repack(str(path), "experts.gate_up_proj_blocks", "rev", ["s:1", "s:2"])
    info = G.repack_inspect(str(path))
    assert info["layout_version"] == 3 and (info["experts"], info["rows"], info["blocks"]) == (E, N, B)
    assert info["payload_offset"] + info["payload_bytes"] == os.path.getsize(path)
    assert not [p for p in os.listdir(tmp_path) if p.endswith(".tmp")]  # the temporary file was renamed
    v = G.Weights.load_repack(ctx, str(path))
    assert (v.export_canonical() == canonical).all()
    status, act = O.quantize_residual_q8(O.bf16_to_f32(O.gen_bf16_normal(5, 5, 3 * B * 32)))
    assert status == O.OK
    for expert in range(E):
        a = G.mxfp4_matmul(ctx, w, expert, act, 3, None, np.zeros((3, N), np.float32))
        b = G.mxfp4_matmul(ctx, v, expert, act, 3, None, np.zeros((3, N), np.float32))
        assert (a.view(np.uint32) == b.view(np.uint32)).all()
    w.close()
    v.close()


def test_safetensors_checkpoint_loads(ctx, canonical, tmp_path):
    blocks, scales = checkpoint(canonical)
    shards = [tmp_path / "model-00001-of-00002.safetensors", tmp_path / "model-00002-of-00002.safetensors"]
    safetensors.numpy.save_file({"experts.gate_up_proj_blocks": blocks, "other": np.zeros(3, np.float32)},
                                str(shards[0]))
    safetensors.numpy.save_file({"experts.gate_up_proj_scales": scales}, str(shards[1]))
    w = G.Weights.from_safetensors(ctx, [str(p) for p in shards], "experts.gate_up_proj_blocks",
                                   "experts.gate_up_proj_scales")
    assert (w.export_canonical() == canonical).all()
    w.close()
    with pytest.raises(G.GossmxError) as e:  # dtype check: the scales must be U8
        safetensors.numpy.save_file({"s": scales.astype(np.int16)}, str(tmp_path / "bad.safetensors"))
        G.Weights.from_safetensors(ctx, [str(shards[0]), str(tmp_path / "bad.safetensors")],
                                   "experts.gate_up_proj_blocks", "s")
    assert e.value.status == G.ERR_BAD_FILE


def test_open_or_create_publishes_then_reuses(ctx, canonical, tmp_path):
    blocks, scales = checkpoint(canonical)
    shard = tmp_path / "model.safetensors"
    safetensors.numpy.save_file({"b": blocks, "s": scales}, str(shard))
    root = tmp_path / "cache"
    key = G.repack_cache_key("b", (E, N, B), 3, "rev", ["model.safetensors:00"])
    target = root / "mxfp4" / key / "weights.repack"
    w = G.Weights.open_or_create(ctx, str(root), "rev", ["model.safetensors:00"], [str(shard)], "b", "s")
    assert (w.export_canonical() == canonical).all()
    assert target.is_file() and not (target.parent / "repack.lock").exists()
    stamp = target.stat().st_mtime_ns
    w.close()
    # The published container is loaded, not rewritten.
    v = G.Weights.open_or_create(ctx, str(root), "rev", ["model.safetensors:00"], [str(shard)], "b", "s")
    assert (v.export_canonical() == canonical).all()
    assert target.stat().st_mtime_ns == stamp
    v.close()
    # A lock left by a process that is gone is taken over and the container
    # written again.
    target.unlink()
    (target.parent / "repack.lock").write_text("pid=999999999\n")
    x = G.Weights.open_or_create(ctx, str(root), "rev", ["model.safetensors:00"], [str(shard)], "b", "s")
    assert (x.export_canonical() == canonical).all()
    assert target.is_file() and not (target.parent / "repack.lock").exists()
    x.close()
    # Another identity is another key and another container.
    u = G.Weights.open_or_create(ctx, str(root), "rev2", ["model.safetensors:00"], [str(shard)], "b", "s")
    assert len(os.listdir(root / "mxfp4")) == 2
    u.close()
