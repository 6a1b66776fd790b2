"""GGUF model files through the library's native reader (g4_gguf_*).

`GGUFFile` mirrors what GGUFParser.parse() returns (src/gguf.ts:75-101):
version, tensor and key/value counts, the key/value map, the tensor infos and
the data offset; tensor bytes are views into the library's memory mapping,
and `upload` copies a tensor's GGUF bytes to device memory unchanged (the
quantized blocks the matvecs read). `config_from_gguf` restates
configFromGGUF (src/config/gemma4-e2b.ts:70-148) and `shape_from_config`
turns its result into the decoder's layer layout.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Any, Dict, Iterator, List, Optional, Tuple

import numpy as np

from ._lib import G4Error, check, lib

# GGUF value types (src/gguf.ts:50-72)
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
# tensor types whose sizes the reference knows (src/gguf.ts:385-395)
T_F32, T_F16, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_BF16 = 0, 1, 8, 12, 13, 14, 30
TYPE_NAMES = {T_F32: "F32", T_F16: "F16", T_Q8_0: "Q8_0", T_Q4_K: "Q4_K", T_Q5_K: "Q5_K", T_Q6_K: "Q6_K",
              T_BF16: "BF16"}
# the matvec weight formats: GGUF type -> the library's wtype name
MATVEC_TYPES = {T_Q4_K: "q4k", T_Q6_K: "q6k"}

_FLOATS = (F32, F64)
_SIGNED = (I8, I16, I32, I64)


@dataclass
class GGUFTensor:
    name: str
    dims: Tuple[int, ...]   # GGUF order: dims[0] is the contiguous one
    type: int
    offset: int             # relative to the data section
    nbytes: int             # 0 for a type whose size is not known
    index: int

    @property
    def n_elements(self) -> int:
        return int(np.prod(self.dims, dtype=np.int64))

    @property
    def type_name(self) -> str:
        return TYPE_NAMES.get(self.type, str(self.type))


class GGUFFile:
    """A parsed GGUF v2/v3 file (memory-mapped by the library, or parsed from
    `data` bytes that this object keeps alive). Malformed files raise G4Error
    with the reader's reason."""

    def __init__(self, path: Optional[str] = None, data: Optional[bytes] = None):
        self._h = ctypes.c_void_p()
        self._keep = None
        if (path is None) == (data is None):
            raise ValueError("give a path or data")
        if path is not None:
            check(lib().g4_gguf_open(str(path).encode(), ctypes.byref(self._h)))
        else:
            self._keep = ctypes.create_string_buffer(bytes(data), len(data))
            check(lib().g4_gguf_open_memory(self._keep, len(data), ctypes.byref(self._h)))
        v, nt, nkv, off, al = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64(), \
            ctypes.c_uint32()
        check(lib().g4_gguf_info(self._h, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nkv), ctypes.byref(off),
                                 ctypes.byref(al)))
        self.version, self.tensor_count, self.kv_count = v.value, nt.value, nkv.value
        self.data_offset, self.alignment = off.value, al.value
        self.tensors: List[GGUFTensor] = [self._tensor(i) for i in range(self.tensor_count)]
        self._by_name = {t.name: t for t in self.tensors}
        self._kv: Optional[Dict[str, Tuple[int, Any]]] = None

    # ---- lifetime --------------------------------------------------------
    def close(self) -> None:
        if self._h:
            lib().g4_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self) -> "GGUFFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- key/values ------------------------------------------------------
    def _kv_entry(self, i: int) -> Tuple[str, int, Any]:
        key, t, at, n = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
        check(lib().g4_gguf_kv(self._h, i, ctypes.byref(key), ctypes.byref(t), ctypes.byref(at), ctypes.byref(n)))
        name = key.value.decode("utf-8", "replace")
        if t.value == ARR:
            if at.value == ARR:
                return name, ARR, None  # nested arrays: the reference's keys use none
            return name, ARR, [self._scalar(i, j, at.value) for j in range(n.value)]
        return name, t.value, self._scalar(i, 0, t.value)

    def _scalar(self, i: int, j: int, t: int) -> Any:
        if t == STR:
            s, n = ctypes.c_void_p(), ctypes.c_uint64()
            check(lib().g4_gguf_kv_string(self._h, i, j, ctypes.byref(s), ctypes.byref(n)))
            return ctypes.string_at(s.value, n.value).decode("utf-8", "replace") if n.value else ""
        f, iv, u = ctypes.c_double(), ctypes.c_int64(), ctypes.c_uint64()
        check(lib().g4_gguf_kv_number(self._h, i, j, ctypes.byref(f), ctypes.byref(iv), ctypes.byref(u)))
        if t in _FLOATS:
            return f.value
        if t == BOOL:
            return u.value != 0
        return iv.value if t in _SIGNED else u.value

    @property
    def kv(self) -> Dict[str, Tuple[int, Any]]:
        """key -> (value type, value); arrays are Python lists of their elements."""
        if self._kv is None:
            self._kv = {}
            for i in range(self.kv_count):
                k, t, v = self._kv_entry(i)
                self._kv[k] = (t, v)
        return self._kv

    def get(self, key: str, default: Any = None) -> Any:
        e = self.kv.get(key)
        return default if e is None else e[1]

    def number(self, key: str) -> Optional[float]:
        """kvNumberOrNull (src/gguf.ts:476-485): None when absent or an array."""
        e = self.kv.get(key)
        if e is None or e[0] == ARR or e[1] is None:
            return None
        t, v = e
        if t == STR:
            try:
                return float(v)
            except ValueError:
                return math.nan
        return v

    def array(self, key: str) -> Optional[list]:
        """kvArray (src/gguf.ts:488-492): None when absent or not an array."""
        e = self.kv.get(key)
        return e[1] if e is not None and e[0] == ARR else None

    # ---- tensors ---------------------------------------------------------
    def _tensor(self, i: int) -> GGUFTensor:
        name, nd, t, off, nb = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64(), \
            ctypes.c_uint64()
        dims = (ctypes.c_uint64 * 4)()
        check(lib().g4_gguf_tensor(self._h, i, ctypes.byref(name), ctypes.byref(nd), dims, ctypes.byref(t),
                                   ctypes.byref(off), ctypes.byref(nb)))
        return GGUFTensor(name.value.decode("utf-8", "replace"), tuple(int(dims[d]) for d in range(nd.value)),
                          t.value, off.value, nb.value, i)

    def __contains__(self, name: str) -> bool:
        return name in self._by_name

    def __iter__(self) -> Iterator[GGUFTensor]:
        return iter(self.tensors)

    def tensor(self, name: str) -> GGUFTensor:
        t = self._by_name.get(name)
        if t is None:
            raise KeyError(f"GGUF has no tensor {name!r}")
        return t

    def find(self, name: str) -> Optional[GGUFTensor]:
        idx = ctypes.c_int64()
        check(lib().g4_gguf_find_tensor(self._h, name.encode(), ctypes.byref(idx)))
        return None if idx.value < 0 else self.tensors[idx.value]

    def data(self, name: str) -> np.ndarray:
        """The tensor's bytes (a read-only uint8 view of the mapping)."""
        t = self.tensor(name)
        p = ctypes.c_void_p()
        check(lib().g4_gguf_tensor_data(self._h, t.index, ctypes.byref(p)))
        a = np.ctypeslib.as_array((ctypes.c_uint8 * t.nbytes).from_address(p.value))
        a.flags.writeable = False
        return a

    def upload(self, ctx, name: str, dst=None):
        """The tensor's GGUF bytes into device memory (a new Buffer, or `dst`)."""
        t = self.tensor(name)
        if not t.nbytes:
            raise G4Error(-1, f"{name}: type {t.type_name} has no known size")
        buf = dst if dst is not None else ctx.alloc(t.nbytes)
        check(lib().g4_gguf_upload(ctx.h, self._h, t.index, ctypes.c_void_p(buf.ptr), buf.nbytes))
        return buf

    def upload_f16(self, ctx, name: str, dst=None):
        """An F32 / F16 / BF16 tensor as f16 (round to nearest even)."""
        t = self.tensor(name)
        n = t.n_elements
        buf = dst if dst is not None else ctx.alloc(max(n, 2) * 2)
        check(lib().g4_gguf_upload_f16(ctx.h, self._h, t.index, ctypes.c_void_p(buf.ptr), buf.nbytes // 2))
        return buf


# ---- configFromGGUF ----------------------------------------------------------

def default_config() -> dict:
    """defaultConfig (src/config/gemma4-e2b.ts:16-63)."""
    n = 35
    sliding = [True] * n
    for i in (4, 9, 14, 19, 24, 29, 34):
        sliding[i] = False
    unshared = 15
    cfg = dict(hidden_size=1536, num_q_heads=8, num_kv_heads=1, head_dim=256, intermediate_size=12288,
               vocab_size=262144, num_layers=n, context_length=2048, rms_norm_eps=1e-6,
               rope_theta_global=1_000_000.0, rope_theta_swa=10_000.0, head_dim_local=256, head_dim_global=512,
               sliding_window=512, attention_is_sliding=sliding,
               intermediate_sizes=[6144 if i < unshared else 12288 for i in range(n)],
               num_unshared_layers=unshared, per_layer_input_dim=256, final_logit_softcapping=30.0)
    _derive(cfg)
    return cfg


def _derive(cfg: dict) -> None:
    hd = max(cfg["head_dim_local"], cfg["head_dim_global"])
    cfg["q_dim"] = cfg["num_q_heads"] * hd
    cfg["kv_dim"] = cfg["num_kv_heads"] * hd
    cfg["kv_producer_for_layer"] = kv_producer_map(cfg)


def kv_producer_map(cfg: dict) -> List[int]:
    """computeKvProducerMap (src/config/gemma4-e2b.ts:159-180): each layer at
    or past num_unshared_layers reads the last unshared layer of its kind
    (-1 when there is none)."""
    n, unshared, sliding = cfg["num_layers"], cfg["num_unshared_layers"], cfg["attention_is_sliding"]
    last_local = last_global = -1
    for i in range(min(unshared, n)):
        if sliding[i]:
            last_local = i
        else:
            last_global = i
    return [i if i < unshared else (last_local if sliding[i] else last_global) for i in range(n)]


def config_from_gguf(g: GGUFFile, max_context_length: Optional[int] = None) -> dict:
    """configFromGGUF (src/config/gemma4-e2b.ts:70-148): the E2B defaults,
    overridden by every gemma4.* key the file holds."""
    if "gemma4.block_count" not in g.kv and "gemma4.embedding_length" not in g.kv:
        raise ValueError("Not a Gemma 4 GGUF: no gemma4.* metadata keys found")
    cfg = default_config()

    def num(key: str):
        v = g.number(key)
        return None if v is None else v

    for key, field in (("gemma4.embedding_length", "hidden_size"), ("gemma4.block_count", "num_layers"),
                       ("gemma4.attention.head_count", "num_q_heads"),
                       ("gemma4.attention.head_count_kv", "num_kv_heads")):
        v = num(key)
        if v is not None:
            cfg[field] = int(v)
    ctx_len = num("gemma4.context_length")
    if ctx_len is not None:
        cfg["context_length"] = int(min(ctx_len, max_context_length if max_context_length is not None else 2048))
    ffn = g.array("gemma4.feed_forward_length")
    if ffn is not None:
        cfg["intermediate_sizes"] = [int(v) for v in ffn]
        cfg["intermediate_size"] = max(cfg["intermediate_sizes"])
    else:
        v = num("gemma4.feed_forward_length")
        if v is not None:
            cfg["intermediate_size"] = int(v)
            cfg["intermediate_sizes"] = [int(v)] * cfg["num_layers"]
    v = num("gemma4.attention.key_length")
    if v is not None:
        cfg["head_dim_global"] = int(v)
    v = num("gemma4.attention.key_length_swa")
    if v is not None:
        cfg["head_dim_local"] = int(v)
    cfg["head_dim"] = cfg["head_dim_local"]
    v = num("gemma4.rope.freq_base")
    if v is not None:
        cfg["rope_theta_global"] = float(v)
    v = num("gemma4.rope.freq_base_swa")
    if v is not None:
        cfg["rope_theta_swa"] = float(v)
    v = num("gemma4.attention.sliding_window")
    if v is not None:
        cfg["sliding_window"] = int(v)
    pat = g.array("gemma4.attention.sliding_window_pattern")
    if pat is not None:
        cfg["attention_is_sliding"] = [bool(x) for x in pat]
    v = num("gemma4.embedding_length_per_layer_input")
    if v is not None:
        cfg["per_layer_input_dim"] = int(v)
    v = num("gemma4.final_logit_softcapping")
    if v is not None:
        cfg["final_logit_softcapping"] = float(v)
    v = num("gemma4.attention.shared_kv_layers")
    if v is not None:
        cfg["num_unshared_layers"] = cfg["num_layers"] - int(v)
    _derive(cfg)
    return cfg


def shape_from_config(cfg: dict, vocab: Optional[int] = None):
    """The decoder layout of a configFromGGUF result. Every layer below
    num_unshared_layers must share one FFN width and every later layer
    another (the decoder's two widths), and the window and head dims must be
    ones its attention kernels take; anything else is ValueError."""
    from .decoder import E2BShape

    n, unshared = cfg["num_layers"], cfg["num_unshared_layers"]
    sliding = cfg["attention_is_sliding"]
    if len(sliding) < n or len(cfg["intermediate_sizes"]) < n:
        raise ValueError("per-layer arrays shorter than block_count")
    ffn_lo = sorted(set(cfg["intermediate_sizes"][:min(unshared, n)]))
    ffn_hi = sorted(set(cfg["intermediate_sizes"][unshared:n]))
    if len(ffn_lo) > 1 or len(ffn_hi) > 1:
        raise ValueError(f"FFN widths {ffn_lo} / {ffn_hi}: one width per side of the shared-KV split")
    if any(p < 0 for p in cfg["kv_producer_for_layer"][:n]):
        raise ValueError("a layer past the shared-KV split has no unshared layer of its attention kind")
    ffn = ffn_lo[0] if ffn_lo else ffn_hi[0]
    ffn_shared = ffn_hi[0] if ffn_hi and ffn_hi[0] != ffn else 0
    glob = tuple(i for i in range(n) if not sliding[i])
    return E2BShape(hidden=cfg["hidden_size"], n_q_heads=cfg["num_q_heads"], n_kv_heads=cfg["num_kv_heads"],
                    head_dim=cfg["head_dim_local"], ffn=ffn, vocab=int(vocab or cfg["vocab_size"]), n_layers=n,
                    eps=cfg["rms_norm_eps"], window=cfg["sliding_window"], theta_local=cfg["rope_theta_swa"],
                    theta_global=cfg["rope_theta_global"], softcap=cfg["final_logit_softcapping"],
                    global_layers=glob,
                    head_dim_global=cfg["head_dim_global"] if cfg["head_dim_global"] != cfg["head_dim_local"] else 0,
                    ffn_shared=ffn_shared, n_unshared=unshared if unshared < n else 0)
