"""The on-disk form of GGUF routed experts, and its way into HBM.

A GGUF file (v2 / v3, llama.cpp's container) holds each MoE layer's routed experts as three tensors
``blk.N.ffn_{gate,up,down}_exps.weight`` of ne = [row length, rows, experts] in one ggml block type. The pack
(tools/gguf_repack.py:1-181 in the reference) rewrites them as ``experts.bin`` + ``experts_index.json``: per
projection, one record per expert, each record the expert's bytes (part "gguf": uint8 [rows, row bytes], its ggml
type and ne in the part) followed by a zero "pad" part up to a 4 KiB stride, so every record starts 4 KiB aligned.

    read_header(f)                    GGUF header -> (metadata, tensors, data start)   gguf_repack.py:70-104
    expert_tensors(shards, layers)    the routed-expert tensors to pack, checked        gguf_repack.py:107-125
    pack(shards, out_bin, ...)        experts.bin + experts_index.json, read back       gguf_repack.py:138-177
    load_packed(model_path)           {"index", "fd"} or None                           stream_fast.py:6654-6661
    gguf_types(packed, gate_key)      "Q4_0/Q4_0/Q4_0" of a layer, or None              stream_fast.py:8050-8062
    read_records(packed, key, ids)    expert records as uint8 [n, rows, row bytes]      stream_fast.py:3402-3423
    fill_slots(packed, key, ids, buf, slots)   records into device slot buffers [S, rows, row bytes]
    load_layer(packed, layer)         a layer's three projections resident in HBM, [E, rows, row bytes] each

The last two are this build's: on a GPU with 288 GB of HBM a whole model's experts (16 GB for the 48-layer
Q4_0 stack) stay resident, so the loader streams records through a pinned staging buffer into device tensors the
expert kernels read directly (the arena slots of the reference's store, stream_fast.py:3936-3941).
"""
import json
import os
import re
import struct
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import numpy as np

__all__ = ["GGML_BLOCKS", "DECODED", "RECORD_ALIGN", "read_header", "expert_tensors", "pack", "load_packed",
           "gguf_types", "read_records", "fill_slots", "load_layer", "check_scales"]

# ggml type id -> (name, weights a block, bytes a block): llama.cpp gguf-py constants.py GGML_QUANT_SIZES, so the
# header of any file parses, whatever its types (the same table as gguf_repack.py:29-39).
GGML_BLOCKS = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20), 6: ("Q5_0", 32, 22),
    7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 9: ("Q8_1", 32, 36), 10: ("Q2_K", 256, 84), 11: ("Q3_K", 256, 110),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210), 15: ("Q8_K", 256, 292),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50),
    20: ("IQ4_NL", 32, 18), 21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8),
    29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66),
    39: ("MXFP4", 32, 17), 40: ("NVFP4", 64, 36), 41: ("Q1_0", 128, 18), 42: ("Q2_0", 64, 18),
    43: ("F8_E4M3", 1, 1)}

# The types the expert kernels decode, with the byte offsets of each block's f16 scale fields (the fields
# llama.cpp's ggml_validate_row_data checks for finiteness; gguf_ref.py:557-560 in the reference).
DECODED = {"Q4_0": (0,), "Q4_K": (0, 2), "Q4_1": (0, 2), "Q8_0": (0,), "Q5_K": (0, 2), "Q6_K": (208,)}

RECORD_ALIGN = 4096          # every record starts 4 KiB aligned (direct reads), a pad part filling the stride
_CHUNK = 32                  # experts copied at a time while packing
_EXPS = re.compile(r"blk\.(\d+)\.ffn_(gate|up|down)_exps\.weight")
_PROJ = ("gate", "up", "down")
# GGUF metadata value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array,
# 10 u64, 11 i64, 12 f64
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
_KEEP = 64                   # metadata arrays longer than this keep only their length (tokenizer tables)


def _key(layer, proj):
    return f"model.layers.{layer}.mlp.switch_mlp.{proj}_proj"


class _Reader:
    def __init__(self, f):
        self.f = f

    def take(self, fmt):
        n = struct.calcsize(fmt)
        b = self.f.read(n)
        if len(b) != n:
            raise ValueError(f"{getattr(self.f, 'name', 'GGUF file')}: the header ends early")
        return struct.unpack(fmt, b)[0]

    def string(self):
        return self.f.read(self.take("<Q")).decode("utf-8", "replace")

    def value(self, vt):
        if vt in _SCALAR:
            return self.take(_SCALAR[vt])
        if vt == 8:
            return self.string()
        if vt != 9:
            raise ValueError(f"{getattr(self.f, 'name', 'GGUF file')}: metadata value type {vt} is not GGUF's")
        et, n = self.take("<I"), self.take("<Q")
        if et in _SCALAR and n > _KEEP:
            self.f.seek(n * struct.calcsize(_SCALAR[et]), os.SEEK_CUR)
            return {"array_len": n}
        vals = [self.value(et) for _ in range(n)]
        return vals if n <= _KEEP else {"array_len": n, "head": vals[:4]}


def read_header(f):
    """(metadata, tensors, data start) of the GGUF file object ``f`` read from offset 0 (gguf_repack.py:70-104).
    tensors: dicts of name, ne (ggml order, innermost first), type (ggml id), offset (absolute in the file) and
    nbytes (None for a type id this table does not know). Versions 2 and 3; anything else raises ValueError."""
    r = _Reader(f)
    name = getattr(f, "name", "GGUF file")
    if f.read(4) != b"GGUF":
        raise ValueError(f"{name}: not a GGUF file")
    version = r.take("<I")
    if version not in (2, 3):
        raise ValueError(f"{name}: GGUF version {version} (2 and 3 are read)")
    n_tensors, n_kv = r.take("<Q"), r.take("<Q")
    meta = {"version": version}
    for _ in range(n_kv):
        k = r.string()
        meta[k] = r.value(r.take("<I"))
    tensors = []
    for _ in range(n_tensors):
        tname = r.string()
        ne = [r.take("<Q") for _ in range(r.take("<I"))]
        tid, off = r.take("<I"), r.take("<Q")
        tensors.append({"name": tname, "ne": ne, "type": tid, "offset": off})
    align = int(meta.get("general.alignment", 32))
    pos = f.tell()
    start = pos + (-pos) % align
    for t in tensors:
        t["offset"] += start
        blk = GGML_BLOCKS.get(t["type"])
        if blk is None:
            t["nbytes"] = None
            continue
        n = int(np.prod(t["ne"], dtype=np.int64)) if t["ne"] else 1
        if n % blk[1]:
            raise ValueError(f"{name}: {t['name']} has {n} weights, not whole {blk[0]} blocks")
        t["nbytes"] = n // blk[1] * blk[2]
    return meta, tensors, start


def _type_name(tid):
    return GGML_BLOCKS[tid][0] if tid in GGML_BLOCKS else f"ggml type id {tid}"


def expert_tensors(shards, layers=None):
    """[(index key, shard, tensor)] of every routed-expert tensor of the layers below ``layers`` (all when None),
    by layer, then gate, up, down (gguf_repack.py:107-125). A layer missing one of its three projections, or an
    expert tensor in a type the kernels do not decode, raises ValueError naming the file and the type."""
    found = {}
    for sh in shards:
        with open(sh, "rb") as f:
            _, tensors, _ = read_header(f)
        for t in tensors:
            m = _EXPS.fullmatch(t["name"])
            if m and (layers is None or int(m.group(1)) < layers):
                found[int(m.group(1)), _PROJ.index(m.group(2))] = (sh, t)
    for L in sorted({L for L, _ in found}):
        missing = [_PROJ[p] for p in range(3) if (L, p) not in found]
        if missing:
            raise ValueError(f"layer {L} has no {'/'.join(missing)} expert tensor")
    for sh, t in found.values():
        tn = _type_name(t["type"])
        if tn not in DECODED:
            raise ValueError(f"{Path(sh).name}: {t['name']} is {tn}, which these kernels do not decode "
                             f"(they decode {', '.join(DECODED)})")
        if len(t["ne"]) != 3:
            raise ValueError(f"{Path(sh).name}: {t['name']} has ne {t['ne']}, not [row length, rows, experts]")
    return [(_key(L, _PROJ[p]), *found[L, p]) for L, p in sorted(found)]


def check_scales(records, t):
    """True when every block's f16 scale fields are finite (llama.cpp's ggml_validate_row_data, the check the
    reference's pack runs on each chunk, gguf_repack.py:128-131). records: uint8 array of whole blocks."""
    bb = _block_bytes(t)
    b = np.ascontiguousarray(records).reshape(-1, bb)
    for at in DECODED[t]:
        h = b[:, at:at + 2].copy().view(np.float16).astype(np.float32)
        if not np.isfinite(h).all():
            return False
    return True


def _block_bytes(t):
    for name, _, bb in GGML_BLOCKS.values():
        if name == t:
            return bb
    raise ValueError(f"unknown ggml type {t}")


def _drop_cache(fd, off, n):
    if hasattr(os, "posix_fadvise"):
        os.posix_fadvise(fd, off, n, os.POSIX_FADV_DONTNEED)


def pack(shards, out_bin, log=print, layers=None, drop_src=True):
    """Write ``out_bin`` and experts_index.json beside it from the routed experts of the GGUF ``shards``, and
    return the index (gguf_repack.py:138-177). Each chunk of records is written, flushed, dropped from the page
    cache, read back and compared byte for byte with the source slices; a non-finite scale raises ValueError."""
    out_bin = Path(out_bin)
    todo = expert_tensors(shards, layers)
    index, written = {}, 0
    with open(out_bin, "wb") as dst, open(out_bin, "rb") as back:
        for i, (key, shard, t) in enumerate(todo):
            tn = GGML_BLOCKS[t["type"]][0]
            ne0, ne1, n_exp = t["ne"]
            nbytes = t["nbytes"] // n_exp
            stride = nbytes + (-nbytes) % RECORD_ALIGN
            parts = [{"name": "gguf", "bytes": nbytes, "shape": [ne1, nbytes // ne1], "dtype": "U8",
                      "ggml_type": tn, "ne": [ne0, ne1]}]
            if stride > nbytes:
                parts.append({"name": "pad", "bytes": stride - nbytes, "shape": [stride - nbytes], "dtype": "U8"})
            index[key] = {"offset": written, "stride": stride, "n_experts": n_exp, "parts": parts}
            with open(shard, "rb") as src:
                for e0 in range(0, n_exp, _CHUNK):
                    n = min(_CHUNK, n_exp - e0)
                    at = t["offset"] + e0 * nbytes
                    raw = os.pread(src.fileno(), n * nbytes, at)
                    if len(raw) != n * nbytes:
                        raise ValueError(f"{Path(shard).name}: {t['name']} ends before expert {e0 + n - 1}")
                    if drop_src:
                        _drop_cache(src.fileno(), at, n * nbytes)
                    rec = np.zeros((n, stride), np.uint8)
                    rec[:, :nbytes] = np.frombuffer(raw, np.uint8).reshape(n, nbytes)
                    if not check_scales(rec[:, :nbytes], tn):
                        raise ValueError(f"{Path(shard).name}: {t['name']} experts {e0}..{e0 + n - 1} hold a "
                                         f"non-finite {tn} scale")
                    dst.write(rec.data)
                    dst.flush()
                    os.fsync(dst.fileno())
                    _drop_cache(dst.fileno(), written, n * stride)
                    if os.pread(back.fileno(), n * stride, written) != rec.tobytes():
                        raise OSError(f"{out_bin.name}: {key} experts {e0}..{e0 + n - 1} read back differently")
                    written += n * stride
            if log is not None:
                log(f"  [{i + 1}/{len(todo)}] {key}: {tn} {n_exp} x {stride:,} B, {written / 1e9:.2f} GB")
    out_bin.with_name("experts_index.json").write_text(json.dumps(index, indent=1))
    return index


def load_packed(model_path):
    """{"index": experts_index.json, "fd": experts.bin opened for reading} of a packed model directory, or None
    when it has no pack (stream_fast.py:6654-6661)."""
    idx = Path(model_path) / "experts_index.json"
    binf = Path(model_path) / "experts.bin"
    if not (idx.exists() and binf.exists()):
        return None
    return {"index": json.loads(idx.read_text()), "fd": open(binf, "rb")}


def gguf_types(packed, gate_key):
    """The gate, up and down ggml types of the layer whose gate projection is ``gate_key`` as one "Q4_0/Q4_0/Q4_0"
    string, None when that layer's records are not GGUF blocks; ValueError (one sentence naming the file and the
    types) for types the kernels do not decode (stream_fast.py:8050-8062)."""
    index = (packed or {}).get("index", {})
    m = index.get(gate_key)
    if m is None or m["parts"][0]["name"] != "gguf":
        return None
    base = gate_key[:-len("gate_proj")]
    types = tuple(index[base + p]["parts"][0]["ggml_type"] for p in ("gate_proj", "up_proj", "down_proj"))
    bad = [t for t in types if t not in DECODED]
    if bad:
        where = getattr(packed.get("fd"), "name", "experts.bin")
        raise ValueError(f"{where}: {base}* holds GGUF experts in {'/'.join(types)}, which these kernels do not "
                         f"decode ({', '.join(bad)})")
    return "/".join(types)


def _record(packed, key):
    m = packed["index"][key]
    part = m["parts"][0]
    if part["name"] != "gguf":
        raise ValueError(f"{key}: its records are {part['name']}, not GGUF blocks")
    return m, part


_POOL = None


def _pool():
    global _POOL
    if _POOL is None:
        _POOL = ThreadPoolExecutor(max_workers=8)
    return _POOL


def read_records(packed, key, ids, out=None):
    """The records of experts ``ids`` of projection ``key`` as uint8 [len(ids), rows, row bytes], one pread per
    record on a thread pool (stream_fast.py:3402-3423). ``out`` (a numpy array of that shape, pinned memory
    included) is filled in place when given."""
    m, part = _record(packed, key)
    rows, rb = part["shape"]
    ids = [int(i) for i in np.asarray(ids).reshape(-1)]
    for e in ids:
        if not 0 <= e < m["n_experts"]:
            raise ValueError(f"{key}: expert {e} of {m['n_experts']}")
    if out is None:
        out = np.empty((len(ids), rows, rb), np.uint8)
    fd = packed["fd"].fileno()

    def fill(j):
        b = os.pread(fd, part["bytes"], m["offset"] + ids[j] * m["stride"])
        if len(b) != part["bytes"]:
            raise OSError(f"{key}: expert {ids[j]}'s record is cut short")
        out[j] = np.frombuffer(b, np.uint8).reshape(rows, rb)

    if len(ids) > 1:
        list(_pool().map(fill, range(len(ids))))
    elif ids:
        fill(0)
    return out


def fill_slots(packed, key, ids, buf, slots, chunk=16, stream=None):
    """Copy the records of experts ``ids`` of projection ``key`` into device slot buffer ``buf`` (uint8
    [S, rows, row bytes], a torch tensor on the GPU) at ``slots`` (same length as ids): preads into two pinned
    staging buffers in turn, each chunk copied to the device on ``stream`` while the next is read."""
    import torch

    m, part = _record(packed, key)
    rows, rb = part["shape"]
    ids = np.asarray(ids).reshape(-1)
    slots = np.asarray(slots).reshape(-1)
    if ids.shape != slots.shape:
        raise ValueError(f"{len(ids)} experts for {len(slots)} slots")
    if buf.dtype != torch.uint8 or tuple(buf.shape[1:]) != (rows, rb):
        raise ValueError(f"slot buffer {tuple(buf.shape)} {buf.dtype} for records of [{rows}, {rb}] uint8")
    if len(slots) and not (0 <= slots.min() and slots.max() < buf.shape[0]):
        raise ValueError(f"slots outside 0..{buf.shape[0] - 1}")
    st = stream or torch.cuda.current_stream(buf.device)
    stage = [torch.empty((chunk, rows, rb), dtype=torch.uint8, pin_memory=True) for _ in range(2)]
    done = [None, None]
    with torch.cuda.stream(st):
        for c0 in range(0, len(ids), chunk):
            s = (c0 // chunk) % 2
            if done[s] is not None:
                done[s].synchronize()
            n = min(chunk, len(ids) - c0)
            read_records(packed, key, ids[c0:c0 + n], out=stage[s].numpy()[:n])
            sl = slots[c0:c0 + n]
            if n and (np.diff(sl) == 1).all():
                buf[int(sl[0]):int(sl[0]) + n].copy_(stage[s][:n], non_blocking=True)
            else:
                for j in range(n):
                    buf[int(sl[j])].copy_(stage[s][j], non_blocking=True)
            done[s] = torch.cuda.Event()
            done[s].record(st)
    for e in done:
        if e is not None:
            e.synchronize()
    return buf


def load_layer(packed, layer, device="cuda", block="mlp"):
    """The routed experts of ``layer`` resident in HBM: ((gate, up, down) uint8 tensors [E, rows, row bytes],
    "gate/up/down" types). Each projection is one device allocation, filled through pinned staging."""
    import torch

    base = f"model.layers.{layer}.{block}.switch_mlp."
    types = gguf_types(packed, base + "gate_proj")
    if types is None:
        raise ValueError(f"layer {layer}: no GGUF expert records")
    out = []
    for p in ("gate_proj", "up_proj", "down_proj"):
        m, part = _record(packed, base + p)
        e = m["n_experts"]
        buf = torch.empty((e,) + tuple(part["shape"]), dtype=torch.uint8, device=device)
        fill_slots(packed, base + p, np.arange(e), buf, np.arange(e))
        out.append(buf)
    return tuple(out), types
