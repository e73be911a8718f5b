"""The GGUF pack and loader (larder_amd.gguf_pack) on synthetic GGUF files written here, after the reference's
tests/test_gguf_repack.py:1-117: two shards, two MoE layers (one whose records are whole 4 KiB pages, one padded),
non-expert tensors between. Every record must be its expert's bytes, 4 KiB aligned, the pad zero and the index
right; a missing projection, a non-finite scale and a type the kernels do not decode are refused with one
sentence. The header reader is also held to every GGUF metadata value type, versions 2 and 3, and an alignment
other than 32. The GPU half (the loaded records through the expert kernels) is in test_gpu_gguf_pack.py."""
import json
import struct

import numpy as np
import pytest

from larder_amd import gguf_pack as gp
from oracle import gguf

HID, E = 512, 6
LAYERS = [(128, ("Q4_K", "Q4_K", "Q4_0")), (64, ("Q4_0", "Q4_0", "Q4_K"))]   # (intermediate, types)
TID = {"Q4_0": 2, "Q4_K": 12, "F32": 0, "Q8_K": 15}


def _s(x):
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(k, v):
    """A metadata pair: str -> string, int -> u32, float -> f32, bool -> bool, list of int -> array of i32,
    tuple (vtype, fmt, value) -> that scalar type."""
    if isinstance(v, bool):
        return _s(k) + struct.pack("<I?", 7, v)
    if isinstance(v, str):
        return _s(k) + struct.pack("<I", 8) + _s(v)
    if isinstance(v, int):
        return _s(k) + struct.pack("<II", 4, v)
    if isinstance(v, float):
        return _s(k) + struct.pack("<If", 6, v)
    if isinstance(v, list):
        if v and isinstance(v[0], str):
            return _s(k) + struct.pack("<IIQ", 9, 8, len(v)) + b"".join(_s(x) for x in v)
        return _s(k) + struct.pack("<IIQ", 9, 5, len(v)) + b"".join(struct.pack("<i", x) for x in v)
    vt, fmt, val = v
    return _s(k) + struct.pack("<I", vt) + struct.pack(fmt, val)


def write_gguf(path, kv, tensors, version=3, align=32):
    """A GGUF file: kv [(key, value)], tensors [(name, ne, type id, raw bytes)], data aligned to ``align``."""
    h = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    for k, v in kv:
        h += _kv(k, v)
    data, off = b"", 0
    for name, ne, t, raw in tensors:
        h += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        h += struct.pack("<IQ", t, off)
        raw = raw + b"\0" * ((-len(raw)) % align)
        data += raw
        off += len(raw)
    path.write_bytes(h + b"\0" * ((-len(h)) % align) + data)


def blocks(rng, t, n_weights):
    """Random blocks of type t with finite f16 scales."""
    _, be, bb = gguf.TYPES[t]
    b = rng.integers(0, 256, (n_weights // be, bb), dtype=np.uint8)
    for at in ((0,) if t == "Q4_0" else (0, 2)):
        b[:, at:at + 2] = (rng.standard_normal((len(b), 1)) * 0.01).astype(np.float16).view(np.uint8)
    return b.tobytes()


def expert_tensors(rng):
    out = []
    for L, (inter, ts) in enumerate(LAYERS):
        for p, t in zip(("gate", "up", "down"), ts):
            ne = [HID, inter, E] if p != "down" else [inter, HID, E]
            out.append((f"blk.{L}.ffn_{p}_exps.weight", ne, TID[t], blocks(rng, t, HID * inter * E)))
    return out


KV = [("general.architecture", "qwen3moe"), ("general.alignment", 32), ("general.name", "synthetic"),
      ("qwen3moe.expert_count", E), ("rope.scale", 1.5), ("flag", True), ("short", [1, -2, 3]),
      ("tokens", ["a", "bc", "def"]), ("u8", (0, "<B", 200)), ("i64", (11, "<q", -5)), ("f64", (12, "<d", 0.25)),
      ("long", list(range(100)))]


def test_pack_records_and_index(tmp_path):
    rng = np.random.default_rng(1)
    exps = expert_tensors(rng)
    other = [("token_embd.weight", [16, 4], 0, rng.standard_normal(64).astype(np.float32).tobytes()),
             ("blk.0.ffn_gate_shexp.weight", [HID, 64], 12, blocks(rng, "Q4_K", HID * 64))]
    s1, s2 = tmp_path / "m-00001-of-00002.gguf", tmp_path / "m-00002-of-00002.gguf"
    write_gguf(s1, KV, [other[0]] + exps[:4])
    write_gguf(s2, KV, [other[1]] + exps[4:])
    index = gp.pack([s1, s2], tmp_path / "experts.bin", log=None)
    idx = json.loads((tmp_path / "experts_index.json").read_text())
    assert idx == index and len(idx) == 6
    binb = (tmp_path / "experts.bin").read_bytes()
    padded = 0
    for name, ne, tid, raw in exps:
        L, p = int(name.split(".")[1]), name.split("_")[1]
        m = idx[f"model.layers.{L}.mlp.switch_mlp.{p}_proj"]
        part = m["parts"][0]
        nb = len(raw) // E
        assert part["ggml_type"] == gp.GGML_BLOCKS[tid][0] and part["bytes"] == nb and part["ne"] == ne[:2]
        assert part["shape"] == [ne[1], nb // ne[1]]
        assert m["stride"] % 4096 == 0 and m["offset"] % 4096 == 0 and m["n_experts"] == E
        assert sum(q["bytes"] for q in m["parts"]) == m["stride"]
        padded += m["stride"] > nb
        for e in range(E):
            rec = binb[m["offset"] + e * m["stride"]:m["offset"] + (e + 1) * m["stride"]]
            assert rec[:nb] == raw[e * nb:(e + 1) * nb], (name, e)
            assert rec[nb:] == b"\0" * (m["stride"] - nb)
    assert 0 < padded < 6                       # both the aligned and the padded case ran
    assert len(binb) == sum(m["stride"] * E for m in idx.values())

    packed = gp.load_packed(tmp_path)
    assert packed["index"] == idx
    assert gp.gguf_types(packed, "model.layers.0.mlp.switch_mlp.gate_proj") == "Q4_K/Q4_K/Q4_0"
    assert gp.gguf_types(packed, "model.layers.1.mlp.switch_mlp.gate_proj") == "Q4_0/Q4_0/Q4_K"
    assert gp.gguf_types(packed, "model.layers.7.mlp.switch_mlp.gate_proj") is None
    ids = [5, 0, 3, 3]
    for name, ne, tid, raw in exps:
        L, p = int(name.split(".")[1]), name.split("_")[1]
        got = gp.read_records(packed, f"model.layers.{L}.mlp.switch_mlp.{p}_proj", ids)
        nb = len(raw) // E
        assert got.shape == (4, ne[1], nb // ne[1])
        for j, e in enumerate(ids):
            assert got[j].tobytes() == raw[e * nb:(e + 1) * nb]
    with pytest.raises(ValueError, match="expert 6 of 6"):
        gp.read_records(packed, "model.layers.0.mlp.switch_mlp.up_proj", [6])
    packed["fd"].close()
    assert gp.load_packed(tmp_path / "nothing") is None

    # only the layers below 1
    index1 = gp.pack([s1, s2], tmp_path / "one.bin", log=None, layers=1)
    assert sorted(index1) == sorted(k for k in idx if ".layers.0." in k)


def test_refusals(tmp_path):
    rng = np.random.default_rng(2)
    exps = expert_tensors(rng)
    s1 = tmp_path / "a.gguf"
    # a layer without its down projection
    write_gguf(s1, KV, exps[:5])
    with pytest.raises(ValueError, match="layer 1 has no down"):
        gp.expert_tensors([s1])
    # a NaN scale, before anything is kept
    bad = bytearray(exps[0][3])
    bad[0:2] = np.array([np.nan], np.float16).tobytes()
    write_gguf(s1, KV, [(exps[0][0], exps[0][1], exps[0][2], bytes(bad))] + exps[1:6])
    with pytest.raises(ValueError, match="non-finite Q4_K scale"):
        gp.pack([s1], tmp_path / "bad.bin", log=None)
    # a type the kernels do not decode, and an id no table knows: one sentence naming the file and the type
    for tid, name in ((15, "Q8_K"), (99, "ggml type id 99")):
        n = HID * 128 * E // 256 * 292
        write_gguf(s1, KV, exps[:2] + [(exps[2][0], exps[2][1], tid, bytes(n))] + exps[3:6])
        with pytest.raises(ValueError) as ei:
            gp.expert_tensors([s1])
        msg = str(ei.value)
        assert s1.name in msg and name in msg and msg.count(". ") == 0
    # not GGUF, a version the reader does not know
    (tmp_path / "x.gguf").write_bytes(b"GGML" + bytes(60))
    with pytest.raises(ValueError, match="not a GGUF file"):
        gp.expert_tensors([tmp_path / "x.gguf"])
    write_gguf(tmp_path / "v1.gguf", KV, exps[:3], version=1)
    with pytest.raises(ValueError, match="GGUF version 1"):
        gp.expert_tensors([tmp_path / "v1.gguf"])


@pytest.mark.parametrize("version,align", [(2, 32), (3, 32), (3, 64)])
def test_header_values(tmp_path, version, align):
    rng = np.random.default_rng(3)
    exps = expert_tensors(rng)[:3]
    kv = [(k, align) if k == "general.alignment" else (k, v) for k, v in KV]
    path = tmp_path / "h.gguf"
    write_gguf(path, kv, exps, version=version, align=align)
    with open(path, "rb") as f:
        meta, tensors, start = gp.read_header(f)
    assert meta["version"] == version and meta["general.alignment"] == align
    assert meta["general.architecture"] == "qwen3moe" and meta["qwen3moe.expert_count"] == E
    assert meta["rope.scale"] == 1.5 and meta["flag"] is True and meta["short"].tolist() == [1, -2, 3]
    assert meta["tokens"] == ["a", "bc", "def"] and meta["u8"] == 200 and meta["i64"] == -5
    assert meta["f64"] == 0.25 and meta["long"].dtype == np.int32 and meta["long"].tolist() == list(range(100))
    assert start % align == 0
    body = path.read_bytes()
    for (name, ne, tid, raw), t in zip(exps, tensors):
        assert t["name"] == name and t["ne"] == ne and t["type"] == tid and t["nbytes"] == len(raw)
        assert body[t["offset"]:t["offset"] + len(raw)] == raw


def test_malformed_headers_raise_value_error(tmp_path):
    """A header cut short anywhere, or holding a metadata value type GGUF does not define, raises ValueError (not
    the BufferError an unreleased view of the mapped file would leave behind when the map closes)."""
    rng = np.random.default_rng(4)
    exps = expert_tensors(rng)[:3]
    good = tmp_path / "g.gguf"
    write_gguf(good, KV, exps)
    body = good.read_bytes()
    with open(good, "rb") as f:
        _, _, start = gp.read_header(f)
    # every cut inside the metadata and tensor infos (the header ends at most align - 1 = 31 bytes before the data):
    # a key length running past the end, a value cut short, ...
    cuts = sorted(set(range(24, 64)) | set(range(24, start - 32, 37)) | {start - 40, start - 33})
    for cut in cuts:
        p = tmp_path / f"cut{cut}.gguf"
        p.write_bytes(body[:cut])
        with open(p, "rb") as f, pytest.raises(ValueError):
            gp.read_header(f)
    # a metadata key whose length field claims more bytes than the file holds
    h = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1 << 40) + b"abc"
    (tmp_path / "long.gguf").write_bytes(h + bytes(32))
    with open(tmp_path / "long.gguf", "rb") as f, pytest.raises(ValueError, match="ends early"):
        gp.read_header(f)
    # an unknown metadata value type (13), and an array of an unknown element type
    for raw in (_s("k") + struct.pack("<I", 13) + bytes(8),
                _s("k") + struct.pack("<IIQ", 9, 13, 2) + bytes(16)):
        p = tmp_path / "vt.gguf"
        p.write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + raw + bytes(32))
        with open(p, "rb") as f, pytest.raises(ValueError, match="not a GGUF type"):
            gp.read_header(f)
    # the reader stays usable on the good file afterwards
    with open(good, "rb") as f:
        assert gp.read_header(f)[2] == start
