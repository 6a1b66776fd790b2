"""The native GGUF reader (g4_gguf_*) and configFromGGUF on the CPU.

Pins: a header assembled byte by byte whose data offset is worked out by
hand; files from the test-side writer (written from the published layout,
no code shared with the reader) carrying every value type, every tensor
type the reference sizes (src/gguf.ts:385-395) and a non-default alignment;
every truncation of a file and a set of corrupted headers, each of which
must be refused with an error, never read past the buffer; and
configFromGGUF (src/config/gemma4-e2b.ts:70-148) on Gemma-4-E2B's metadata
against the layout its documentation states (35 layers, global every fifth,
FFN 6144 / 12288 split at 15, head dims 256 / 512, producers 13 and 14)."""
import struct

import numpy as np
import pytest

from g4hip import G4Error
from g4hip.gguf import GGUFFile, config_from_gguf, default_config, kv_producer_map, shape_from_config
from g4hip.decoder import E2BShape
from gguf_writer import ARR, BOOL, F32, F64, GGUFWriter, I8, I16, I32, I64, STR, U8, U16, U32, U64


def test_hand_assembled_header():
    # magic, version 3, 1 tensor, 1 key/value
    b = struct.pack("<IIQQ", 0x46554747, 3, 1, 1)                      # 24 bytes
    b += struct.pack("<Q", 1) + b"a" + struct.pack("<II", U32, 7)       # +17 = 41
    b += struct.pack("<Q", 1) + b"t" + struct.pack("<IQIQ", 1, 4, 0, 0)  # +33 = 74 -> data at 96
    b += b"\0" * (96 - len(b)) + np.arange(4, dtype=np.float32).tobytes()
    g = GGUFFile(data=b)
    assert (g.version, g.tensor_count, g.kv_count, g.data_offset, g.alignment) == (3, 1, 1, 96, 32)
    assert g.kv == {"a": (U32, 7)}
    t = g.tensor("t")
    assert (t.dims, t.type, t.offset, t.nbytes) == ((4,), 0, 0, 16)
    assert np.array_equal(g.data("t").view(np.float32), np.arange(4, dtype=np.float32))


def _all_values(w: GGUFWriter) -> dict:
    want = {
        "u8": (U8, 200), "i8": (I8, -7), "u16": (U16, 65000), "i16": (I16, -30000), "u32": (U32, 4000000000),
        "i32": (I32, -2000000000), "f32": (F32, 0.5), "bool": (BOOL, True), "str": (STR, "héllo"),
        "u64": (U64, 2**63 + 5), "i64": (I64, -(2**62)), "f64": (F64, 1e-300), "empty": (STR, ""),
    }
    for k, (t, v) in want.items():
        w.kv(k, t, v)
    arrays = {
        "a_u32": (U32, [6144] * 3 + [12288] * 2), "a_f32": (F32, [1.0, -2.5]), "a_bool": (BOOL, [True, False, True]),
        "a_str": (STR, ["x", "", "yz" * 40]), "a_i64": (I64, [-1, 2**40]), "a_empty": (U8, []),
    }
    for k, (et, items) in arrays.items():
        w.array(k, et, items)
        want[k] = (ARR, list(items))
    return want


def test_every_value_type_round_trips():
    w = GGUFWriter()
    want = _all_values(w)
    w.kv("nested", ARR, (ARR, [(U8, [1, 2]), (STR, ["q"])]))
    g = GGUFFile(data=w.to_bytes())
    for k, (t, v) in want.items():
        gt, gv = g.kv[k]
        assert gt == t, k
        if t == F32:
            assert gv == np.float32(v), k
        elif t == ARR and want[k][1] and isinstance(v[0], float):
            assert np.array_equal(np.float32(gv), np.float32(v)), k
        else:
            assert gv == v, k
    assert g.kv["nested"][0] == ARR
    assert g.number("u32") == 4000000000 and g.number("a_u32") is None
    assert g.array("a_u32") == [6144, 6144, 6144, 12288, 12288] and g.array("u32") is None


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_tensor_infos_and_bytes(tmp_path, alignment):
    rng = np.random.default_rng(5)
    w = GGUFWriter(alignment=alignment)
    w.kv("gemma4.block_count", U32, 2)
    specs = [("f32", (3, 5), 0, 4 * 15), ("f16", (7,), 1, 14), ("q8", (64, 2), 8, 4 * 34),
             ("q4k", (512, 3), 12, 6 * 144), ("q5k", (256,), 13, 176), ("q6k", (256, 2, 2), 14, 4 * 210),
             ("bf16", (9,), 30, 18)]
    blobs = {}
    for name, dims, t, nb in specs:
        blobs[name] = rng.integers(0, 256, nb, dtype=np.uint8).tobytes()
        w.tensor(name, dims, t, blobs[name])
    path = w.write(str(tmp_path / "t.gguf"))
    for g in (GGUFFile(path), GGUFFile(data=open(path, "rb").read())):
        a = alignment or 32
        assert g.alignment == a and g.data_offset % a == 0
        assert [t.name for t in g.tensors] == [s[0] for s in specs]
        for name, dims, t, nb in specs:
            ti = g.tensor(name)
            assert (ti.dims, ti.type, ti.nbytes) == (dims, t, nb)
            assert ti.offset % a == 0
            assert g.data(name).tobytes() == blobs[name]
            assert g.find(name).index == ti.index
        assert g.find("absent") is None
        g.close()


def _small_file() -> bytes:
    w = GGUFWriter()
    w.kv("general.architecture", STR, "gemma4").kv("gemma4.block_count", U32, 1)
    w.array("gemma4.feed_forward_length", U32, [6144])
    w.array("tokenizer.ggml.tokens", STR, ["<pad>", "a", "bc"])
    w.tensor("token_embd.weight", (256, 1), 12, bytes(range(144)))
    w.tensor("output_norm.weight", (3,), 0, np.ones(3, np.float32))
    return w.to_bytes()


def test_every_truncation_is_refused():
    full = _small_file()
    GGUFFile(data=full).close()
    for n in range(len(full)):
        with pytest.raises(G4Error):
            GGUFFile(data=full[:n])


def _patch(b: bytes, off: int, fmt: str, v) -> bytes:
    return b[:off] + struct.pack(fmt, v) + b[off + struct.calcsize(fmt):]


def test_corrupt_headers_are_refused():
    full = _small_file()
    bad = [
        _patch(full, 0, "<I", 0x46554748),            # magic
        _patch(full, 4, "<I", 1),                     # version 1 (u32 counts)
        _patch(full, 4, "<I", 4),
        _patch(full, 8, "<Q", 2**40),                 # tensor count past the file
        _patch(full, 16, "<Q", 2**40),                # key/value count past the file
        _patch(full, 24, "<Q", 2**50),                # first key's length past the file
    ]
    first_type = 24 + 8 + len("general.architecture")
    bad.append(_patch(full, first_type, "<I", 13))    # unknown value type
    g = GGUFFile(data=full)
    t = g.tensor("output_norm.weight")
    hdr = full.find(b"output_norm.weight") + len("output_norm.weight")
    bad.append(_patch(full, hdr, "<I", 5))            # 5 dims
    bad.append(_patch(full, hdr + 4, "<Q", 0))        # a zero dim
    bad.append(_patch(full, hdr + 16, "<Q", t.offset + 4))  # misaligned offset
    bad.append(_patch(full, hdr + 16, "<Q", 1 << 40))  # data past the end
    # element counts whose byte size wraps 64 bits to a few bytes (F32 x 4, F16 / BF16 x 2)
    bad.append(_patch(full, hdr + 4, "<Q", (1 << 62) + 1))
    bad.append(_patch(full, hdr + 4, "<Q", 1 << 62))
    for t16 in (1, 30):
        bad.append(_patch(_patch(full, hdr + 12, "<I", t16), hdr + 4, "<Q", (1 << 63) + 1))
    for i, b in enumerate(bad):
        with pytest.raises(G4Error):
            GGUFFile(data=b)
    # a string array whose count exceeds what the file could hold
    arr = full.find(b"tokenizer.ggml.tokens") + len("tokenizer.ggml.tokens") + 4 + 4
    with pytest.raises(G4Error):
        GGUFFile(data=_patch(full, arr, "<Q", 2**33))


def test_version_2_and_unknown_tensor_type():
    w = GGUFWriter(version=2)
    w.kv("k", U32, 1).tensor("x", (4,), 0, np.zeros(4, np.float32))
    g = GGUFFile(data=w.to_bytes())
    assert g.version == 2
    # a type the reference does not size (Q2_K = 10) parses with nbytes 0
    b = bytearray(w.to_bytes())
    i = bytes(b).find(b"x") + 1 + 4 + 8
    b[i:i + 4] = struct.pack("<I", 10)
    g = GGUFFile(data=bytes(b))
    assert g.tensor("x").nbytes == 0
    with pytest.raises(G4Error):
        g.data("x")


def _e2b_metadata(w: GGUFWriter) -> GGUFWriter:
    n = 35
    w.kv("general.architecture", STR, "gemma4")
    w.kv("gemma4.embedding_length", U32, 1536).kv("gemma4.block_count", U32, n)
    w.kv("gemma4.attention.head_count", U32, 8).kv("gemma4.attention.head_count_kv", U32, 1)
    w.kv("gemma4.context_length", U32, 131072)
    w.array("gemma4.feed_forward_length", I32, [6144] * 15 + [12288] * 20)
    w.kv("gemma4.attention.key_length", U32, 512).kv("gemma4.attention.key_length_swa", U32, 256)
    w.kv("gemma4.rope.freq_base", F32, 1e6).kv("gemma4.rope.freq_base_swa", F32, 1e4)
    w.kv("gemma4.attention.sliding_window", U32, 512)
    w.array("gemma4.attention.sliding_window_pattern", BOOL, [(i % 5) != 4 for i in range(n)])
    w.kv("gemma4.embedding_length_per_layer_input", U32, 256)
    w.kv("gemma4.final_logit_softcapping", F32, 30.0)
    w.kv("gemma4.attention.shared_kv_layers", U32, 20)
    return w


def test_config_from_gguf_e2b():
    g = GGUFFile(data=_e2b_metadata(GGUFWriter()).to_bytes())
    cfg = config_from_gguf(g)
    assert cfg["context_length"] == 2048
    assert config_from_gguf(g, 8192)["context_length"] == 8192
    assert cfg["num_unshared_layers"] == 15
    assert [i for i, s in enumerate(cfg["attention_is_sliding"]) if not s] == [4, 9, 14, 19, 24, 29, 34]
    assert cfg["intermediate_size"] == 12288
    assert (cfg["q_dim"], cfg["kv_dim"]) == (4096, 512)
    prod = cfg["kv_producer_for_layer"]
    assert prod[:15] == list(range(15))
    assert all(prod[i] == (14 if i % 5 == 4 else 13) for i in range(15, 35))
    # the hardcoded baseline agrees with the file on every key it carries
    base = default_config()
    for k in ("hidden_size", "num_layers", "num_q_heads", "num_kv_heads", "head_dim_global", "head_dim_local",
              "intermediate_sizes", "attention_is_sliding", "num_unshared_layers", "per_layer_input_dim",
              "final_logit_softcapping", "sliding_window", "kv_producer_for_layer"):
        assert cfg[k] == base[k], k
    s = shape_from_config(cfg)
    r = E2BShape.real()
    for f in ("hidden", "n_q_heads", "n_kv_heads", "head_dim", "ffn", "vocab", "n_layers", "window",
              "global_layers", "head_dim_global", "ffn_shared", "n_unshared", "softcap"):
        assert getattr(s, f) == getattr(r, f), f
    assert (s.theta_local, s.theta_global) == (r.theta_local, r.theta_global)
    assert [s.producer(i) for i in range(35)] == prod


def test_config_overrides_and_errors():
    g = GGUFFile(data=GGUFWriter().kv("gemma4.block_count", U32, 35).to_bytes())
    assert config_from_gguf(g) == default_config()
    w = GGUFWriter().kv("gemma4.block_count", U32, 6).kv("gemma4.feed_forward_length", U32, 4096)
    w.array("gemma4.attention.sliding_window_pattern", BOOL, [True, True, False, True, True, False])
    w.kv("gemma4.attention.shared_kv_layers", U32, 2)
    cfg = config_from_gguf(GGUFFile(data=w.to_bytes()))
    assert cfg["intermediate_sizes"] == [4096] * 6 and cfg["num_unshared_layers"] == 4
    assert cfg["kv_producer_for_layer"] == [0, 1, 2, 3, 3, 2]
    with pytest.raises(ValueError):
        config_from_gguf(GGUFFile(data=GGUFWriter().kv("llama.block_count", U32, 2).to_bytes()))
    # a consumer layer with no unshared layer of its kind
    cfg = dict(num_layers=3, num_unshared_layers=1, attention_is_sliding=[True, False, True])
    assert kv_producer_map(cfg) == [0, -1, 0]


def test_random_corruptions_parse_or_refuse():
    """2000 random corruptions of a valid file (byte flips, 64-bit length
    fields set to huge values, splices of the file into itself): each one
    either parses, and then every key, string and tensor is readable, or is
    refused with an error; none may crash the process or read outside the
    buffer (the reader bounds-checks every access)."""
    full = bytearray(_small_file())
    rng = np.random.default_rng(2024)
    parsed = refused = 0
    for it in range(2000):
        b = bytearray(full)
        kind = it % 4
        if kind == 0:
            for _ in range(int(rng.integers(1, 6))):
                b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        elif kind == 1:
            at = int(rng.integers(0, len(b) - 8))
            b[at:at + 8] = struct.pack("<Q", int(rng.integers(0, 2**63)))
        elif kind == 2:
            at = int(rng.integers(0, len(b) - 4))
            b[at:at + 4] = struct.pack("<I", int(rng.integers(0, 2**32)))
        else:
            i, j = sorted(int(x) for x in rng.integers(0, len(b), 2))
            b = b[:i] + b[j:] + b[i:j]
        try:
            g = GGUFFile(data=bytes(b))
        except G4Error:
            refused += 1
            continue
        parsed += 1
        for k in g.kv:
            g.kv[k]
        for t in g.tensors:
            if t.nbytes:
                assert g.data(t.name).size == t.nbytes
        g.close()
    assert parsed > 0 and refused > 0
