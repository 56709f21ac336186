"""The safetensors reader and writer (hwnpu_amd.checkpoint) on the CPU, against the format as the
reference reads it (internal/safetensors/safetensors.go:53-216) and writes it (write.go:30-85); the
loaders into device layouts are tested on the GPU (test_checkpoint_gpu.py).

The files are written here byte by byte with struct/json (not with the writer under test) where a
check is about the reader."""
import json
import os
import struct

import numpy as np
import pytest

from hwnpu_amd.checkpoint import Checkpoint, CheckpointError, SafeTensors, write_safetensors


def raw_file(path, header: dict, data: bytes, pad=True):
    h = json.dumps(header).encode()
    if pad:
        h += b" " * ((-(8 + len(h))) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + data)


def test_reader_dtypes_and_metadata(tmp_path):
    rng = np.random.default_rng(1)
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    f16 = rng.standard_normal(7).astype(np.float16)
    bf = (rng.standard_normal(6).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    u8 = rng.integers(0, 256, (2, 2, 16), dtype=np.uint8)
    blobs = [f32.tobytes(), f16.tobytes(), bf.tobytes(), u8.tobytes()]
    offs, o = [], 0
    for b in blobs:
        offs.append([o, o + len(b)])
        o += len(b)
    hdr = {"__metadata__": {"format": "pt"},
           "a": {"dtype": "F32", "shape": [3, 5], "data_offsets": offs[0]},
           "b": {"dtype": "F16", "shape": [7], "data_offsets": offs[1]},
           "c": {"dtype": "BF16", "shape": [2, 3], "data_offsets": offs[2]},
           "d": {"dtype": "U8", "shape": [2, 2, 16], "data_offsets": offs[3]}}
    p = tmp_path / "m.safetensors"
    raw_file(p, hdr, b"".join(blobs))
    st = SafeTensors(str(p))
    assert st.metadata == {"format": "pt"} and st.names() == ["a", "b", "c", "d"]
    assert np.array_equal(st.float32("a"), f32)
    assert np.array_equal(st.float32("b"), f16.astype(np.float32))
    # BF16 is the high half of a float32 (vecops.BF16ToF32)
    assert np.array_equal(st.float32("c").reshape(-1).view(np.uint32), bf.astype(np.uint32) << 16)
    assert np.array_equal(st.raw("d"), u8)
    with pytest.raises(CheckpointError, match="no tensor"):
        st.raw("zz")
    with pytest.raises(CheckpointError, match="cannot convert"):
        st.float32("d")
    st.close()


def test_reader_rejects_bad_files(tmp_path):
    p = tmp_path / "bad.safetensors"
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", 200 << 20))
    with pytest.raises(CheckpointError, match="MiB this reader accepts"):
        SafeTensors(str(p))
    raw_file(p, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}, b"\0" * 8)
    with pytest.raises(CheckpointError, match="past the end"):
        SafeTensors(str(p))
    raw_file(p, {"a": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}, b"\0" * 16)
    with pytest.raises(CheckpointError, match="bytes for"):
        SafeTensors(str(p))
    raw_file(p, {"a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 0]}}, b"\0" * 8)
    with pytest.raises(CheckpointError, match="data_offsets"):
        SafeTensors(str(p))


def test_writer_round_trip_alignment_and_index(tmp_path):
    rng = np.random.default_rng(2)
    t = {"x": ("F32", rng.standard_normal((4, 4)).astype(np.float32)),
         "y": ("U8", rng.integers(0, 256, 33, dtype=np.uint8)),
         "z": ("F16", rng.standard_normal(3).astype(np.float16))}
    p = str(tmp_path / "a.safetensors")
    write_safetensors(p, t, {"k": "v"})
    with open(p, "rb") as f:
        (n,) = struct.unpack("<Q", f.read(8))
    assert (8 + n) % 8 == 0  # the data starts 8-byte aligned (write.go:50-53)
    assert not os.path.exists(p + ".tmp")
    st = SafeTensors(p)
    for k, (dt, a) in t.items():
        assert st.info(k) == (dt, list(a.shape)) and np.array_equal(st.raw(k), a)
    st.close()
    # an index over two shards (experts.shardOf)
    write_safetensors(str(tmp_path / "b.safetensors"), {"w": ("F32", np.arange(5, dtype=np.float32))})
    idx = tmp_path / "model.safetensors.index.json"
    idx.write_text(json.dumps({"weight_map": {"x": "a.safetensors", "w": "b.safetensors"}}))
    with Checkpoint(str(idx)) as ck:
        assert ck.has("w") and not ck.has("y")
        assert np.array_equal(ck.float32("w"), np.arange(5, dtype=np.float32))
        assert np.array_equal(ck.float32("x"), t["x"][1])
        with pytest.raises(CheckpointError, match="has no"):
            ck.raw("nope")


def test_qwen3_loader_refuses_untied_head_and_non_u8_blocks(tmp_path):
    """hwk_qwen3 has only the tied head: a checkpoint holding lm_head.weight, or one whose config.json
    says tie_word_embeddings false (the reference then reads lm_head.weight,
    internal/llm/qwen3/config.go:142-147), is refused before anything touches a device; so are MXFP4
    blocks or scales stored as anything but U8."""
    from hwnpu_amd import checkpoint

    class NoModel:  # the checks come before the model is read
        cfg = None

    p = str(tmp_path / "m.safetensors")
    write_safetensors(p, {"lm_head.weight": ("F16", np.zeros((4, 32), np.float16))})
    with Checkpoint(p) as ck, pytest.raises(CheckpointError, match="untied head"):
        checkpoint.load_qwen3(NoModel(), ck)
    q = str(tmp_path / "n.safetensors")
    write_safetensors(q, {"model.norm.weight": ("F32", np.ones(32, np.float32))})
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"tie_word_embeddings": False}, f)
    with Checkpoint(q) as ck, pytest.raises(CheckpointError, match="tie_word_embeddings"):
        checkpoint.load_qwen3(NoModel(), ck)
    with Checkpoint(q) as ck, pytest.raises(CheckpointError, match="tie_word_embeddings"):
        checkpoint.load_qwen3(NoModel(), ck, config={"tie_word_embeddings": False})
    r = str(tmp_path / "b.safetensors")
    write_safetensors(r, {"x.q_proj_blocks": ("I8", np.zeros((4, 1, 16), np.int8)),
                          "x.q_proj_scales": ("U8", np.zeros((4, 1), np.uint8))})
    with Checkpoint(r) as ck, pytest.raises(CheckpointError, match="want U8"):
        checkpoint._linear_into(ck, "x.q_proj.weight", 4, 32, 0, 0)


def test_reader_refuses_oversized_header_length(tmp_path):
    p = str(tmp_path / "big.safetensors")
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", (100 << 20) + 1) + b"{}")
    with pytest.raises(CheckpointError, match="MiB"):
        SafeTensors(p)
