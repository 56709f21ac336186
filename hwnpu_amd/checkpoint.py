"""On-disk checkpoints into libhwk's device layouts.

The format is Hugging Face safetensors as the reference reads it (internal/safetensors/
safetensors.go:53-216): a little-endian uint64 header length (at most 100 MB), a JSON header mapping
each tensor name to its dtype, shape and byte range, an optional "__metadata__" entry, then the raw
little-endian data; tensors are read on demand through a memory map, so a checkpoint costs the
memory of the tensors in use. A checkpoint is one file or a model.safetensors.index.json whose
weight_map names each tensor's shard (experts.shardOf, internal/llm/experts/host.go:345-366).
``write_safetensors`` writes the same format (safetensors/write.go:30-85: the header padded with
spaces so that the data starts 8-byte aligned, written to path.tmp and renamed).

Loaders:
- ``load_experts``: a layer's MXFP4 experts named as the reference's experts.MXFP4 record names them
  (host.go:21-43; gpt-oss ``...mlp.experts.gate_up_proj_blocks`` etc.): blocks (E, 2I, H/32, 16) and
  scales (E, 2I, H/32) uint8 with the gate on even rows, down (E, H, I/32, 16) + (E, H, I/32), biases
  (E, 2I) and (E, H) of any float dtype, or none. The bytes go to the device as they are: the
  layout hwk_moe_experts / hwk_moe_layer take is the checkpoint's.
- ``load_qwen3``: a Qwen3 decoder (Hugging Face names, ``model.layers.{i}.self_attn.q_proj.weight``
  ...) into hwk_qwen3's layout (hwk_qwen3_tensor): each linear either as MXFP4 (``{name}_blocks``
  and ``{name}_scales`` with ``name`` the weight's name without ``.weight``, the gpt-oss
  convention), copied as it is, or as a float matrix encoded to MXFP4 on the device by the
  reference's Encode (hwk_mxfp4_encode, internal/mxfp4/encode.go:11-78); q/k/v stacked, gate/up
  interleaved row by row; norm weights as fp32; the tied embedding as fp16.

Nothing here computes on the CPU beyond dtype decoding of small tensors (biases, norms); every
weight matrix is copied to the GPU or encoded there.
"""
from __future__ import annotations

import json
import mmap
import os
import struct

import numpy as np
import torch

from . import hwk
from .ops import _stream

DTYPES = {"U8": np.uint8, "I8": np.int8, "BF16": np.uint16, "F16": np.float16, "F32": np.float32,
          "I32": np.int32, "I64": np.int64, "F64": np.float64}
HEADER_MAX = 100 << 20


class CheckpointError(ValueError):
    """A checkpoint that cannot be read or does not hold what a loader needs."""


class SafeTensors:
    """One safetensors file, its tensors read on demand from a memory map."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        try:
            raw = self._f.read(8)
            if len(raw) != 8:
                raise CheckpointError(f"safetensors: {path}: no header length")
            (n,) = struct.unpack("<Q", raw)
            if n > HEADER_MAX:
                raise CheckpointError(f"safetensors: {path}: the header length field says {n} bytes, "
                                      f"past the {HEADER_MAX >> 20} MiB this reader accepts")
            hdr = self._f.read(n)
            if len(hdr) != n:
                raise CheckpointError(f"safetensors: {path}: header cut off")
            try:
                entries = json.loads(hdr)
            except json.JSONDecodeError as e:
                raise CheckpointError(f"safetensors: {path}: {e}") from e
            self.base = 8 + n
            self.metadata = entries.pop("__metadata__", None) or {}
            size = os.fstat(self._f.fileno()).st_size
            self.tensors = {}
            for name, h in entries.items():
                off = h.get("data_offsets")
                if not isinstance(off, list) or len(off) != 2 or not 0 <= off[0] <= off[1]:
                    raise CheckpointError(f"safetensors: {path}: {name}: bad data_offsets")
                if self.base + off[1] > size:
                    raise CheckpointError(f"safetensors: {path}: {name}: data past the end of the file")
                dt = h.get("dtype")
                shape = [int(d) for d in h.get("shape", [])]
                if dt in DTYPES:
                    want = int(np.prod(shape, dtype=np.int64)) * np.dtype(DTYPES[dt]).itemsize
                    if want != off[1] - off[0]:
                        raise CheckpointError(f"safetensors: {path}: {name}: {off[1] - off[0]} bytes for "
                                              f"{dt} {shape}")
                self.tensors[name] = (dt, shape, off[0], off[1])
            self._map = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ) if size else None
        except Exception:
            self._f.close()
            raise

    def close(self):
        if getattr(self, "_map", None) is not None:
            try:
                self._map.close()
            except BufferError:  # arrays of raw() still view the map: it closes when they go
                pass
            self._map = None
        self._f.close()

    def names(self):
        return sorted(self.tensors)

    def info(self, name: str):
        if name not in self.tensors:
            raise CheckpointError(f"safetensors: {self.path}: no tensor {name!r}")
        dt, shape, _, _ = self.tensors[name]
        return dt, list(shape)

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as an array of its dtype (BF16 as uint16 bit patterns), a view of the map."""
        dt, shape = self.info(name)
        if dt not in DTYPES:
            raise CheckpointError(f"safetensors: {self.path}: {name}: dtype {dt} not supported")
        _, _, b, e = self.tensors[name]
        return np.frombuffer(self._map, dtype=DTYPES[dt], count=(e - b) // np.dtype(DTYPES[dt]).itemsize,
                             offset=self.base + b).reshape(shape)

    def float32(self, name: str) -> np.ndarray:
        """BF16, F16 or F32 data as float32 (safetensors.go:130-183; BF16 is the high half of a float32)."""
        dt, _ = self.info(name)
        a = self.raw(name)
        if dt == "BF16":
            return (a.astype(np.uint32) << 16).view(np.float32)
        if dt in ("F16", "F32", "F64"):
            return a.astype(np.float32, copy=False)  # F32: the mapped view itself (read-only)
        raise CheckpointError(f"safetensors: {self.path}: {name}: cannot convert {dt} to float32")


class Checkpoint:
    """A checkpoint: one safetensors file, or an index whose weight_map names each tensor's shard."""

    def __init__(self, path: str):
        self.path = path
        self._files = {}
        if path.endswith(".json"):
            with open(path) as f:
                idx = json.load(f)
            wm = idx.get("weight_map")
            if not isinstance(wm, dict):
                raise CheckpointError(f"checkpoint: {path}: no weight_map")
            d = os.path.dirname(path)
            self._shard = {k: os.path.join(d, v) for k, v in wm.items()}
        else:
            self._shard = None
            self._files[path] = SafeTensors(path)

    def _file(self, name: str) -> SafeTensors:
        if self._shard is None:
            return self._files[self.path]
        if name not in self._shard:
            raise CheckpointError(f"checkpoint: {self.path} has no {name}")
        p = self._shard[name]
        if p not in self._files:
            self._files[p] = SafeTensors(p)
        return self._files[p]

    def has(self, name: str) -> bool:
        if self._shard is not None:
            return name in self._shard
        return name in self._files[self.path].tensors

    def info(self, name):
        return self._file(name).info(name)

    def raw(self, name):
        return self._file(name).raw(name)

    def float32(self, name):
        return self._file(name).float32(name)

    def close(self):
        for f in self._files.values():
            f.close()
        self._files = {}

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()


def write_safetensors(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """Writes name -> (dtype, array) as one safetensors file, in the dict's order (BF16 arrays as uint16
    bit patterns)."""
    hdr = {}
    if metadata:
        hdr["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    off = 0
    blobs = []
    for name, (dt, a) in tensors.items():
        if dt not in DTYPES:
            raise CheckpointError(f"write_safetensors: {name}: dtype {dt}")
        a = np.ascontiguousarray(a, dtype=DTYPES[dt])
        hdr[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        off += a.nbytes
        blobs.append(a)
    raw = json.dumps(hdr).encode()
    raw += b" " * ((-(8 + len(raw))) % 8)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(struct.pack("<Q", len(raw)))
        f.write(raw)
        for a in blobs:
            f.write(a.tobytes())
    os.replace(tmp, path)


# ---------------- device copies ----------------

_TORCH = {np.dtype(np.uint8): torch.uint8, np.dtype(np.int8): torch.int8, np.dtype(np.uint16): torch.int16,
          np.dtype(np.float16): torch.float16, np.dtype(np.float32): torch.float32, np.dtype(np.int32): torch.int32,
          np.dtype(np.int64): torch.int64, np.dtype(np.float64): torch.float64}


def _to_device(a: np.ndarray) -> torch.Tensor:
    """A new device tensor holding a's values, copied straight from a (a read-only view of the mapped
    file is read in place: no host staging copy; uint16 bit patterns arrive as int16)."""
    a = np.ascontiguousarray(a)
    t = torch.empty(a.shape, dtype=_TORCH[a.dtype], device="cuda")
    if a.nbytes:
        from .qwen3 import h2d

        h2d(t.data_ptr(), a)
    return t


def _copy_into(ptr: int, nbytes: int, src: torch.Tensor) -> None:
    """src's bytes into the device memory at ptr (exactly nbytes)."""
    if src.numel() * src.element_size() != nbytes:
        raise CheckpointError(f"checkpoint: {src.numel() * src.element_size()} bytes for a slot of {nbytes}")
    from .qwen3 import d2d

    src = src.contiguous()
    d2d(ptr, src.data_ptr(), nbytes)


def _host_into(ptr: int, nbytes: int, a: np.ndarray, what: str) -> None:
    """A host array (a mapped view) straight into the device memory at ptr (exactly nbytes)."""
    a = np.ascontiguousarray(a)
    if a.nbytes != nbytes:
        raise CheckpointError(f"checkpoint: {what}: {a.nbytes} bytes for a slot of {nbytes}")
    from .qwen3 import h2d

    h2d(ptr, a)


# ---------------- MoE experts ----------------

def expert_names(prefix: str) -> dict:
    """The record of a gpt-oss layer's experts (internal/llm/gptoss/config.go:193-194): prefix is
    ``model.layers.{i}.mlp.experts.``."""
    return {"gate_up_blocks": prefix + "gate_up_proj_blocks", "gate_up_scales": prefix + "gate_up_proj_scales",
            "gate_up_bias": prefix + "gate_up_proj_bias", "down_blocks": prefix + "down_proj_blocks",
            "down_scales": prefix + "down_proj_scales", "down_bias": prefix + "down_proj_bias"}


def load_experts(ck: Checkpoint, names: dict) -> dict:
    """A layer's experts on the GPU in the layout of hwk_moe_experts: gu_w, gu_e, dn_w, dn_e (uint8) and
    gu_b, dn_b (fp32, or None when the record names none or the checkpoint lacks them)."""
    need = ("gate_up_blocks", "gate_up_scales", "down_blocks", "down_scales")
    for k in need:
        if not names.get(k) or not ck.has(names[k]):
            raise CheckpointError(f"experts: no {k} tensor {names.get(k)!r}")
    out = {}
    for k, key in zip(need, ("gu_w", "gu_e", "dn_w", "dn_e")):
        dt, shape = ck.info(names[k])
        if dt != "U8":
            raise CheckpointError(f"experts: {names[k]} is {dt}, want U8")
        out[key] = _to_device(ck.raw(names[k]))
    E, I2, nbh = out["gu_e"].shape
    _, H, nbi = out["dn_e"].shape
    if tuple(out["gu_w"].shape) != (E, I2, nbh, 16) or tuple(out["dn_w"].shape) != (E, H, nbi, 16) or \
            H != nbh * 32 or I2 != 2 * nbi * 32 or out["dn_e"].shape[0] != E:
        raise CheckpointError(f"experts: shapes {tuple(out['gu_w'].shape)} {tuple(out['gu_e'].shape)} "
                              f"{tuple(out['dn_w'].shape)} {tuple(out['dn_e'].shape)} do not agree")
    for k, key, shape in (("gate_up_bias", "gu_b", (E, I2)), ("down_bias", "dn_b", (E, H))):
        n = names.get(k)
        if n and ck.has(n):
            b = ck.float32(n)
            if tuple(b.shape) != shape:
                raise CheckpointError(f"experts: {n} has shape {tuple(b.shape)}, want {shape}")
            out[key] = _to_device(b)
        else:
            out[key] = None
    return out


# ---------------- the Qwen3 decoder ----------------

def _linear_into(ck: Checkpoint, name: str, rows: int, cols: int, w_ptr: int, e_ptr: int, stride: int = 1) -> None:
    """Writes the linear `name` (``....q_proj.weight``) as MXFP4 into device memory: codes (rows,
    cols/32, 16) at w_ptr, scales (rows, cols/32) at e_ptr, row r at row r*stride of the destination
    (stride 2: gate/up interleaved row by row). Its MXFP4 blocks and scales go straight from the
    mapped file if the checkpoint holds them; else its float matrix is copied to the device and
    encoded there."""
    from .qwen3 import copy_rows

    nb = cols // 32
    base = name[:-len(".weight")] if name.endswith(".weight") else name
    if ck.has(base + "_blocks"):
        for part in ("_blocks", "_scales"):
            dt, _ = ck.info(base + part)
            if dt != "U8":
                raise CheckpointError(f"qwen3: {base}{part} is {dt}, want U8")
        w, e = ck.raw(base + "_blocks"), ck.raw(base + "_scales")
        if tuple(w.shape) != (rows, nb, 16) or tuple(e.shape) != (rows, nb):
            raise CheckpointError(f"qwen3: {base}_blocks/_scales have shapes {tuple(w.shape)} {tuple(e.shape)}, "
                                  f"want ({rows}, {nb}, 16)")
        w, e = np.ascontiguousarray(w), np.ascontiguousarray(e)
        copy_rows(w_ptr, stride * nb * 16, w.ctypes.data, nb * 16, nb * 16, rows, 1)
        copy_rows(e_ptr, stride * nb, e.ctypes.data, nb, nb, rows, 1)
        return
    dt, shape = ck.info(name)
    if tuple(shape) != (rows, cols):
        raise CheckpointError(f"qwen3: {name} has shape {shape}, want {[rows, cols]}")
    x = _to_device(ck.float32(name))
    if stride == 1:
        hwk.load().hwk_mxfp4_encode(_stream(), x.data_ptr(), w_ptr, e_ptr, rows, cols)
    else:
        w = torch.empty((rows, nb, 16), dtype=torch.uint8, device="cuda")
        e = torch.empty((rows, nb), dtype=torch.uint8, device="cuda")
        hwk.load().hwk_mxfp4_encode(_stream(), x.data_ptr(), w.data_ptr(), e.data_ptr(), rows, cols)
        copy_rows(w_ptr, stride * nb * 16, w.data_ptr(), nb * 16, nb * 16, rows, 3)
        copy_rows(e_ptr, stride * nb, e.data_ptr(), nb, nb, rows, 3)
    torch.cuda.current_stream().synchronize()  # x (and w, e) stay alive until the encode has read them


def _tied(ck: Checkpoint, prefix: str, config: dict | None) -> None:
    """hwk_qwen3 has only a tied head (the embedding rows). The reference reads lm_head.weight instead
    when the config unties them (internal/llm/qwen3/config.go:142-147); such a checkpoint is refused
    rather than run with the wrong head."""
    if config is None:
        p = os.path.join(os.path.dirname(os.path.abspath(ck.path)), "config.json")
        if os.path.exists(p):
            with open(p) as f:
                config = json.load(f)
    if config is not None and config.get("tie_word_embeddings", True) is False:
        raise CheckpointError("qwen3: the config unties the output head (tie_word_embeddings false); "
                              "hwk_qwen3 has only the tied head")
    for name in ("lm_head.weight", prefix + "lm_head.weight"):
        if ck.has(name):
            raise CheckpointError(f"qwen3: the checkpoint holds {name}, an untied head; hwk_qwen3 has only the tied head")


def load_qwen3(model, ck: Checkpoint, prefix: str = "model.", config: dict | None = None) -> None:
    """Fills a hwnpu_amd.qwen3.Qwen3's weights from a checkpoint of the Hugging Face Qwen3 names.
    config: the model's config.json as a dict (read from beside the checkpoint when None and present),
    consulted for tie_word_embeddings."""
    _tied(ck, prefix, config)
    c = model.cfg
    hd = c.head_dim
    qn, kn, H, I = c.heads * hd, c.kv_heads * hd, c.hidden, c.inter
    for i in range(c.layers):
        p = f"{prefix}layers.{i}."
        qkv_w, _ = model.tensor(f"layers.{i}.qkv.blocks")
        qkv_e, _ = model.tensor(f"layers.{i}.qkv.scales")
        for name, row0, rows in (("q", 0, qn), ("k", qn, kn), ("v", qn + kn, kn)):
            _linear_into(ck, p + f"self_attn.{name}_proj.weight", rows, H, qkv_w + row0 * (H // 2),
                         qkv_e + row0 * (H // 32))
        _linear_into(ck, p + "self_attn.o_proj.weight", H, qn, model.tensor(f"layers.{i}.o.blocks")[0],
                     model.tensor(f"layers.{i}.o.scales")[0])
        gu_w, _ = model.tensor(f"layers.{i}.gate_up.blocks")
        gu_e, _ = model.tensor(f"layers.{i}.gate_up.scales")
        # gate row r at 2r, up row r at 2r+1
        _linear_into(ck, p + "mlp.gate_proj.weight", I, H, gu_w, gu_e, stride=2)
        _linear_into(ck, p + "mlp.up_proj.weight", I, H, gu_w + H // 2, gu_e + H // 32, stride=2)
        _linear_into(ck, p + "mlp.down_proj.weight", H, I, model.tensor(f"layers.{i}.down.blocks")[0],
                     model.tensor(f"layers.{i}.down.scales")[0])
        for name, t in (("input_layernorm.weight", "input_norm"), ("post_attention_layernorm.weight", "post_norm"),
                        ("self_attn.q_norm.weight", "q_norm"), ("self_attn.k_norm.weight", "k_norm")):
            ptr, n = model.tensor(f"layers.{i}.{t}")
            _host_into(ptr, n, ck.float32(p + name), p + name)
    ptr, n = model.tensor("norm")
    _host_into(ptr, n, ck.float32(prefix + "norm.weight"), prefix + "norm.weight")
    ptr, n = model.tensor("embed")
    emb = prefix + "embed_tokens.weight"
    dt, shape = ck.info(emb)
    if tuple(shape) != (c.vocab, c.hidden):
        raise CheckpointError(f"qwen3: {emb} has shape {shape}, want {[c.vocab, c.hidden]}")
    if dt == "F16":
        _host_into(ptr, n, ck.raw(emb), emb)
    else:  # the fp16 of the float32 value, round to nearest even
        _copy_into(ptr, n, _to_device(ck.float32(emb)).to(torch.float16))
    torch.cuda.synchronize()
