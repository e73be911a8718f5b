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
import mmap
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
_PROJ = ("gate", "up", "down")
_EXPERT_TENSOR = re.compile(r"blk\.(?P<layer>\d+)\.ffn_(?P<proj>gate|up|down)_exps\.weight")

# GGUF metadata value types -> (struct code, name); 8 is a string, 9 an array
_VT = {0: ("B", "u8"), 1: ("b", "i8"), 2: ("H", "u16"), 3: ("h", "i16"), 4: ("I", "u32"), 5: ("i", "i32"),
       6: ("f", "f32"), 7: ("?", "bool"), 10: ("Q", "u64"), 11: ("q", "i64"), 12: ("d", "f64")}
_NP = {"B": np.uint8, "b": np.int8, "H": np.uint16, "h": np.int16, "I": np.uint32, "i": np.int32, "f": np.float32,
       "?": np.bool_, "Q": np.uint64, "q": np.int64, "d": np.float64}


def _key(layer, proj):
    return f"model.layers.{layer}.mlp.switch_mlp.{proj}_proj"


class _Cursor:
    """Little-endian reads at a moving position in an in-memory (memory-mapped) GGUF header."""

    def __init__(self, buf, where):
        self.buf, self.at, self.where = buf, 0, where

    def _span(self, n):
        if self.at + n > len(self.buf):
            raise ValueError(f"{self.where}: the header ends early")
        a = self.at
        self.at += n
        return a

    def num(self, code):
        return struct.unpack_from("<" + code, self.buf, self._span(struct.calcsize(code)))[0]

    def text(self):
        n = self.num("Q")
        a = self._span(n)
        return bytes(self.buf[a:a + n]).decode("utf-8", "replace")

    def meta_value(self, vt):
        """One metadata value: a Python scalar or str; an array of numbers as a numpy array, of strings (or of
        arrays) as a list."""
        if vt in _VT:
            v = self.num(_VT[vt][0])
            return bool(v) if vt == 7 else v
        if vt == 8:
            return self.text()
        if vt != 9:
            raise ValueError(f"{self.where}: metadata value type {vt} is not a GGUF type")
        et, count = self.num("I"), self.num("Q")
        if et in _VT:
            code = _VT[et][0]
            a = self._span(count * struct.calcsize(code))
            return np.frombuffer(self.buf, dtype=np.dtype(_NP[code]).newbyteorder("<"), count=count, offset=a).copy()
        return [self.meta_value(et) for _ in range(count)]


def read_header(f):
    """(metadata, tensors, data start) of the GGUF file object ``f``, versions 2 and 3 (the layout llama.cpp's gguf
    writer produces; the reference reads it in tools/gguf_repack.py:70-104). tensors: dicts of name, ne (ggml order,
    innermost first), type (ggml id), offset (absolute in the file) and nbytes (None for a type id GGML_BLOCKS does
    not know). Anything that is not such a file raises ValueError."""
    where = getattr(f, "name", "GGUF file")
    size = os.fstat(f.fileno()).st_size
    if size < 24:
        raise ValueError(f"{where}: not a GGUF file")
    with mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        c = _Cursor(memoryview(mm), where)
        try:
            if bytes(mm[:4]) != b"GGUF":
                raise ValueError(f"{where}: not a GGUF file")
            c.at = 4
            version = c.num("I")
            if version not in (2, 3):
                raise ValueError(f"{where}: GGUF version {version} (2 and 3 are read)")
            n_tensors, n_meta = c.num("Q"), c.num("Q")
            meta = {"version": version}
            for _ in range(n_meta):
                k = c.text()
                meta[k] = c.meta_value(c.num("I"))
            infos = []
            for _ in range(n_tensors):
                tname = c.text()
                dims = [c.num("Q") for _ in range(c.num("I"))]
                infos.append((tname, dims, c.num("I"), c.num("Q")))
            header_end = c.at
        finally:
            # release the view before the mmap closes: a raised error's traceback frames still hold the cursor, and
            # an unreleased view of the map would make mmap's close raise BufferError in place of that error
            c.buf.release()
            del c
    align = int(meta.get("general.alignment", 32))
    start = -(-header_end // align) * align
    tensors = []
    for tname, dims, tid, rel in infos:
        count = int(np.prod(dims, dtype=np.int64)) if dims else 1
        nbytes = None
        if tid in GGML_BLOCKS:
            tn, per, width = GGML_BLOCKS[tid]
            if count % per:
                raise ValueError(f"{where}: {tname} has {count} weights, not whole {tn} blocks")
            nbytes = count // per * width
        tensors.append({"name": tname, "ne": dims, "type": tid, "offset": start + rel, "nbytes": nbytes})
    return meta, tensors, start


def _type_name(tid):
    return GGML_BLOCKS[tid][0] if tid in GGML_BLOCKS else f"ggml type id {tid}"


def expert_tensors(shards, layers=None):
    """[(index key, shard, tensor)] of every routed-expert tensor (blk.N.ffn_{gate,up,down}_exps.weight) of the
    layers below ``layers`` (all when None), ordered by layer, then gate, up, down. The reference builds the same
    list in tools/gguf_repack.py:107-125. A layer missing one of its three projections, an expert tensor that is not
    [row length, rows, experts], or one in a type the kernels do not decode raises ValueError naming the file and the
    type."""
    by_layer = {}
    for shard in shards:
        with open(shard, "rb") as f:
            _, tensors, _ = read_header(f)
        for t in tensors:
            m = _EXPERT_TENSOR.fullmatch(t["name"])
            if m is None or (layers is not None and int(m["layer"]) >= layers):
                continue
            by_layer.setdefault(int(m["layer"]), {})[m["proj"]] = (shard, t)
    out = []
    for layer in sorted(by_layer):
        have = by_layer[layer]
        absent = [p for p in _PROJ if p not in have]
        if absent:
            raise ValueError(f"layer {layer} has no {'/'.join(absent)} expert tensor")
        for proj in _PROJ:
            shard, t = have[proj]
            tn = _type_name(t["type"])
            if tn not in DECODED:
                raise ValueError(f"{Path(shard).name}: {t['name']} is {tn}, which these kernels do not decode "
                                 f"(they decode {', '.join(DECODED)})")
            if len(t["ne"]) != 3:
                raise ValueError(f"{Path(shard).name}: {t['name']} has ne {t['ne']}, not [row length, rows, experts]")
            out.append((_key(layer, proj), shard, t))
    return out


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


def _uncache(fd, off, n):
    """Drop [off, off + n) of fd from the page cache where the OS allows (so a read-back comes from the drive)."""
    if hasattr(os, "posix_fadvise"):
        os.posix_fadvise(fd, off, n, os.POSIX_FADV_DONTNEED)


def _record_entry(t, offset):
    """The experts_index.json entry of tensor t written from byte ``offset`` of experts.bin: one record an expert, the
    expert's blocks as part "gguf" [rows, row bytes] and zeros as part "pad" up to a 4 KiB multiple."""
    row_len, rows, n_exp = t["ne"]
    body = t["nbytes"] // n_exp
    stride = -(-body // RECORD_ALIGN) * RECORD_ALIGN
    parts = [{"name": "gguf", "bytes": body, "shape": [rows, body // rows], "dtype": "U8",
              "ggml_type": GGML_BLOCKS[t["type"]][0], "ne": [row_len, rows]}]
    if stride != body:
        parts.append({"name": "pad", "bytes": stride - body, "shape": [stride - body], "dtype": "U8"})
    return {"offset": offset, "stride": stride, "n_experts": n_exp, "parts": parts}


class _RecordWriter:
    """experts.bin under construction. Each projection's records go out with positioned writes in groups of experts
    taken straight from the memory-mapped GGUF shard; after a group is synced and dropped from the page cache, a
    second descriptor reads it back and it is compared with the source before the next group is taken."""

    def __init__(self, path, group=32):
        self.path = Path(path)
        self.group = group
        self.fd = os.open(self.path, os.O_WRONLY | os.O_CREAT | os.O_TRUNC, 0o644)
        self.check_fd = os.open(self.path, os.O_RDONLY)
        self.end = 0

    def close(self):
        os.close(self.fd)
        os.close(self.check_fd)

    def _write_groups(self, key, t, src, entry, src_fd):
        body, stride, n_exp = entry["parts"][0]["bytes"], entry["stride"], entry["n_experts"]
        tn = entry["parts"][0]["ggml_type"]
        out = np.zeros((self.group, stride), np.uint8)
        for first in range(0, n_exp, self.group):
            last = min(first + self.group, n_exp)
            n = last - first
            if not check_scales(src[first:last], tn):
                raise ValueError(f"{t['name']} experts {first}..{last - 1} hold a non-finite {tn} scale")
            out[:n, :body] = src[first:last]
            at = self.end + first * stride
            view = memoryview(out[:n].reshape(-1))
            done = 0
            while done < len(view):
                done += os.pwrite(self.fd, view[done:], at + done)
            os.fsync(self.fd)
            _uncache(self.fd, at, n * stride)
            if os.pread(self.check_fd, n * stride, at) != view.tobytes():
                raise OSError(f"{self.path.name}: {key} experts {first}..{last - 1} read back differently")
            if src_fd is not None:
                _uncache(src_fd, t["offset"] + first * body, n * body)

    def add(self, key, shard, t, drop_src):
        entry = _record_entry(t, self.end)
        body, stride, n_exp = entry["parts"][0]["bytes"], entry["stride"], entry["n_experts"]
        with open(shard, "rb") as f:
            mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
            src = None
            try:
                if t["offset"] + n_exp * body > len(mm):
                    raise ValueError(f"{Path(shard).name}: {t['name']} runs past the end of the file")
                src = np.frombuffer(mm, np.uint8, count=n_exp * body, offset=t["offset"]).reshape(n_exp, body)
                self._write_groups(key, t, src, entry, f.fileno() if drop_src else None)
            finally:
                del src
                try:
                    mm.close()
                except BufferError:  # an exception in flight still holds a view of the map: it closes when collected
                    pass
        self.end += n_exp * stride
        return entry


def pack(shards, out_bin, log=print, layers=None, drop_src=True):
    """Write ``out_bin`` and experts_index.json beside it from the routed experts of the GGUF ``shards``, and
    return the index: the on-disk form the reference's tools/gguf_repack.py:138-177 writes and its loader reads
    (stream_fast.py:6654-6661). Every group of records is verified against its source slice after it is synced; a
    non-finite scale raises ValueError."""
    out_bin = Path(out_bin)
    todo = expert_tensors(shards, layers)
    writer = _RecordWriter(out_bin)
    index = {}
    try:
        for n, (key, shard, t) in enumerate(todo, 1):
            index[key] = writer.add(key, shard, t, drop_src)
            if log is not None:
                e = index[key]
                log(f"  {key} ({n} of {len(todo)}): {e['n_experts']} {e['parts'][0]['ggml_type']} records of "
                    f"{e['stride']:,} B; {writer.end / 1e9:.2f} GB written")
    finally:
        writer.close()
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
