"""Device context, buffers and the per-kernel entry points of libg4hip.

Method names are the reference's kernel keys (src/shaders.ts:34-56); their
arguments are the WGSL bindings in order followed by the Params fields
(src/engine.ts:432-545 builds the same Params). Buffers are device
allocations owned by the caller, as in the reference (src/engine.ts:1001-1064).
"""
from __future__ import annotations

import ctypes
from typing import Optional, Union

import numpy as np

from ._lib import (
    AttnFusedParams,
    AttnOutputParams,
    AttnScoreParams,
    KvStoreParams,
    MatmulParams,
    NormAddParams,
    NormRopeParams,
    WarmRegion,
    PagedAttnFusedParams,
    PagedAttnParams,
    PerHeadNormParams,
    RmsNormParams,
    SoftcapParams,
    EmbeddingParams,
    SoftmaxParams,
    check,
    lib,
)


class Buffer:
    """A device allocation (pointer + size); `offset(n)` views a byte offset."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int, owned: bool = True):
        self.ctx = ctx
        self.ptr = ptr
        self.nbytes = nbytes
        self._owned = owned

    def offset(self, nbytes: int) -> "Buffer":
        assert 0 <= nbytes <= self.nbytes
        return Buffer(self.ctx, self.ptr + nbytes, self.nbytes - nbytes, owned=False)

    def upload(self, arr: np.ndarray, offset: int = 0) -> "Buffer":
        a = np.ascontiguousarray(arr)
        assert offset + a.nbytes <= self.nbytes, "upload past the end of the buffer"
        check(lib().g4_upload(self.ctx.h, ctypes.c_void_p(self.ptr), a.ctypes.data_as(ctypes.c_void_p),
                              a.nbytes, offset))
        return self

    def download(self, dtype, count: Optional[int] = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dt.itemsize
        out = np.empty(count, dt)
        assert offset + out.nbytes <= self.nbytes, "download past the end of the buffer"
        check(lib().g4_download(self.ctx.h, out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(self.ptr),
                                out.nbytes, offset))
        return out

    def zero(self) -> "Buffer":
        check(lib().g4_memset(self.ctx.h, ctypes.c_void_p(self.ptr), 0, self.nbytes))
        return self

    def free(self) -> None:
        if self._owned and self.ptr:
            check(lib().g4_free(self.ctx.h, ctypes.c_void_p(self.ptr)))
        self.ptr = 0

    def __del__(self):
        try:
            if self._owned and self.ptr and self.ctx.h:
                lib().g4_free(self.ctx.h, ctypes.c_void_p(self.ptr))
                self.ptr = 0
        except Exception:
            pass


Ptr = Union[Buffer, int, None]


def _p(b: Ptr) -> ctypes.c_void_p:
    if b is None:
        return ctypes.c_void_p(0)
    if isinstance(b, Buffer):
        return ctypes.c_void_p(b.ptr)
    return ctypes.c_void_p(int(b))


class Context:
    """One HIP device + stream. All kernels enqueue on `stream`."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(lib().g4_init(device, ctypes.byref(h)))
        self.h = h
        self.device = device

    def close(self) -> None:
        if self.h:
            lib().g4_destroy(self.h)
            self.h = ctypes.c_void_p(0)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- info / memory ----
    def info(self):
        name = ctypes.create_string_buffer(128)
        cus = ctypes.c_int()
        hbm = ctypes.c_size_t()
        check(lib().g4_device_info(self.h, name, 128, ctypes.byref(cus), ctypes.byref(hbm)))
        return {"name": name.value.decode(), "num_cus": cus.value, "hbm_bytes": hbm.value}

    @property
    def stream(self) -> int:
        return lib().g4_get_stream(self.h) or 0

    def set_stream(self, hip_stream: int) -> None:
        check(lib().g4_set_stream(self.h, ctypes.c_void_p(hip_stream)))

    def alloc(self, nbytes: int) -> Buffer:
        p = ctypes.c_void_p()
        check(lib().g4_alloc(self.h, max(int(nbytes), 1), ctypes.byref(p)))
        return Buffer(self, p.value, int(nbytes))

    def empty(self, count: int, dtype) -> Buffer:
        return self.alloc(int(count) * np.dtype(dtype).itemsize)

    def zeros(self, count: int, dtype) -> Buffer:
        return self.empty(count, dtype).zero()

    def from_numpy(self, arr: np.ndarray) -> Buffer:
        a = np.ascontiguousarray(arr)
        return self.alloc(a.nbytes).upload(a)

    def copy(self, dst: Ptr, src: Ptr, nbytes: int) -> None:
        check(lib().g4_copy_d2d(self.h, _p(dst), _p(src), nbytes))

    def sync(self) -> None:
        check(lib().g4_stream_sync(self.h))

    def clear_stall(self) -> None:
        """Acknowledges a G4_ERR_STALLED (the kernel status word)."""
        check(lib().g4_clear_stall(self.h))

    def test_stage_wait(self, spin_limit: int, skip_matvec: bool) -> None:
        """Test hook: poll limit of the q/k/v hand-off and whether the one
        q/k/v + attention launch leaves out its matvec workgroups."""
        check(lib().g4_test_stage_wait(self.h, spin_limit, 1 if skip_matvec else 0))

    # ---- events / graphs ----
    def record(self) -> ctypes.c_void_p:
        ev = ctypes.c_void_p()
        check(lib().g4_event_record(self.h, ctypes.byref(ev)))
        return ev

    @staticmethod
    def elapsed_ms(a, b) -> float:
        ms = ctypes.c_float()
        check(lib().g4_event_wait(b))
        check(lib().g4_event_elapsed_ms(a, b, ctypes.byref(ms)))
        return float(ms.value)

    @staticmethod
    def destroy_event(ev) -> None:
        lib().g4_event_destroy(ev)

    def graph_begin(self) -> None:
        check(lib().g4_graph_begin(self.h))

    @staticmethod
    def graph_kernel_nodes(g) -> int:
        """Kernel launches one replay of the captured graph issues."""
        n = ctypes.c_size_t()
        check(lib().g4_graph_kernel_nodes(g, ctypes.byref(n)))
        return int(n.value)

    def graph_end(self) -> ctypes.c_void_p:
        g = ctypes.c_void_p()
        check(lib().g4_graph_end(self.h, ctypes.byref(g)))
        return g

    def graph_launch(self, g) -> None:
        check(lib().g4_graph_launch(self.h, g))

    @staticmethod
    def graph_destroy(g) -> None:
        lib().g4_graph_destroy(g)

    # ---- matvec (shaders/matmul_quant.wgsl, matmul_quant_mr4.wgsl) ----
    def matmulQuant(self, x: Ptr, w: Ptr, y: Ptr, M: int, N: int, wtype: str = "q4k") -> None:
        fn = {"q4k": lib().g4_matmulQuant_q4k, "q6k": lib().g4_matmulQuant_q6k,
              "f16": lib().g4_matmulQuant_f16}[wtype]
        check(fn(self.h, _p(x), _p(w), _p(y), MatmulParams(M, N)))

    def matmulQuantMR4(self, x: Ptr, w: Ptr, y: Ptr, M: int, N: int) -> None:
        check(lib().g4_matmulQuantMR4_q4k(self.h, _p(x), _p(w), _p(y), MatmulParams(M, N)))

    def matmulQuantBatch(self, x: Ptr, w: Ptr, y: Ptr, M: int, N: int, batch: int, wtype: str = "q4k") -> None:
        fn = {"q4k": lib().g4_matmulQuantBatch_q4k, "q6k": lib().g4_matmulQuantBatch_q6k}[wtype]
        check(fn(self.h, _p(x), _p(w), _p(y), MatmulParams(M, N), batch))

    def rmsNormMatmul_q4k(self, x: Ptr, norm_w: Ptr, w: Ptr, y: Ptr, M: int, N: int, eps: float = 1e-6) -> None:
        check(lib().g4_rmsNormMatmul_q4k(self.h, _p(x), _p(norm_w), _p(w), _p(y), MatmulParams(M, N), eps))

    def normAddGateUpGelu_q4k(self, o: Ptr, w_post: Ptr, residual: Ptr, w_pre: Ptr, w_gate: Ptr, w_up: Ptr,
                              h_out: Ptr, out: Ptr, M: int, N: int, eps: float = 1e-6) -> None:
        check(lib().g4_normAddGateUpGelu_q4k(self.h, _p(o), _p(w_post), _p(residual), _p(w_pre), _p(w_gate),
                                             _p(w_up), _p(h_out), _p(out), MatmulParams(M, N), eps))

    def normAddMatmulSegments(self, wtype: str, x: Ptr, w1: Ptr, residual: Ptr, w2: Ptr, h_out: Ptr,
                              weights, outputs, rows, N: int, eps: float = 1e-6, softcap: float = 0.0) -> None:
        """[residual + norm(x)*w1 ->] norm(.)*w -> y_i = W_i . x' for up to 4 matrices."""
        n = len(weights)
        W = (ctypes.c_void_p * n)(*[_p(w).value for w in weights])
        Y = (ctypes.c_void_p * n)(*[_p(y).value for y in outputs])
        R = (ctypes.c_uint32 * n)(*rows)
        check(lib().g4_normAddMatmulSegments(self.h, {"q4k": 0, "q6k": 1}[wtype], _p(x), _p(w1), _p(residual),
                                             _p(w2), _p(h_out), W, Y, R, n, N, eps, softcap))

    def normAddScaleMatmulSegments(self, wtype: str, x: Ptr, w1: Ptr, residual: Ptr, out_scale: Ptr, w2: Ptr,
                                   h_out: Ptr, weights, outputs, rows, N: int, eps: float = 1e-6,
                                   softcap: float = 0.0) -> None:
        """h = (residual + norm(x)*w1) * out_scale[0] -> norm(h)*w2 -> y_i = W_i . x'."""
        n = len(weights)
        W = (ctypes.c_void_p * n)(*[_p(w).value for w in weights])
        Y = (ctypes.c_void_p * n)(*[_p(y).value for y in outputs])
        R = (ctypes.c_uint32 * n)(*rows)
        check(lib().g4_normAddScaleMatmulSegments(self.h, {"q4k": 0, "q6k": 1}[wtype], _p(x), _p(w1),
                                                  _p(residual), _p(out_scale), _p(w2), _p(h_out), W, Y, R, n, N,
                                                  eps, softcap))

    def digits_bytes(self, K: int) -> int:
        n = ctypes.c_size_t(0)
        check(lib().g4_digitsBytes(K, ctypes.byref(n)))
        return int(n.value)

    def normAddGateUpGeluDigits_q4k(self, o: Ptr, w_post: Ptr, residual: Ptr, w_pre: Ptr, w_gate: Ptr, w_up: Ptr,
                                    h_out: Ptr, out: Ptr, digits: Ptr, M: int, N: int, eps: float = 1e-6) -> None:
        """normAddGateUpGelu_q4k that also writes `out` as a digit block for matmulQuantDigits_q6k."""
        check(lib().g4_normAddGateUpGeluDigits_q4k(self.h, _p(o), _p(w_post), _p(residual), _p(w_pre), _p(w_gate),
                                                   _p(w_up), _p(h_out), _p(out), _p(digits), MatmulParams(M, N),
                                                   eps))

    def matmulQuantDigits_q6k(self, digits: Ptr, weight: Ptr, out: Ptr, M: int, N: int) -> None:
        """y[M] = W[M, N] . x with x given as the digit block a gate/up launch wrote."""
        check(lib().g4_matmulQuantDigits_q6k(self.h, _p(digits), _p(weight), _p(out), MatmulParams(M, N)))

    def normAddMatmulArgmax(self, wtype: str, x: Ptr, w1: Ptr, residual: Ptr, w2: Ptr, h_out: Ptr, weight: Ptr,
                            logits: Ptr, rows: int, N: int, result: Ptr, eps: float = 1e-6, softcap: float = 0.0,
                            positions: Ptr = None, delta: int = 1) -> None:
        """normAddMatmulSegments over one matrix into `logits`, and *result = argmax(logits) (reference ties
        and NaN rule) from the matvec's own per-workgroup candidates; *positions += delta when given."""
        check(lib().g4_normAddMatmulArgmax(self.h, {"q4k": 0, "q6k": 1}[wtype], _p(x), _p(w1), _p(residual),
                                           _p(w2), _p(h_out), _p(weight), _p(logits), rows, N, eps, softcap,
                                           _p(result), _p(positions), delta))

    def normAddMatmulTopk(self, wtype: str, x: Ptr, w1: Ptr, residual: Ptr, w2: Ptr, h_out: Ptr, weight: Ptr,
                          logits: Ptr, rows: int, N: int, result: Ptr, eps: float = 1e-6,
                          softcap: float = 0.0) -> None:
        """normAddMatmulSegments over one matrix into `logits`, and result f32[512] = topk256(logits)
        (per residue class, reference ties and NaN rule) from the matvec's own per-workgroup candidates."""
        check(lib().g4_normAddMatmulTopk(self.h, {"q4k": 0, "q6k": 1}[wtype], _p(x), _p(w1), _p(residual),
                                         _p(w2), _p(h_out), _p(weight), _p(logits), rows, N, eps, softcap,
                                         _p(result)))

    def normAddMatmulSegmentsBatch(self, wtype: str, x: Ptr, w1: Ptr, residual: Ptr, w2: Ptr, h_out: Ptr,
                                   weights, outputs, rows, N: int, batch: int, eps: float = 1e-6,
                                   softcap: float = 0.0) -> None:
        """normAddMatmulSegments over `batch` vectors: x [batch][N] -> outputs[i] [batch][rows[i]]."""
        n = len(weights)
        W = (ctypes.c_void_p * n)(*[_p(w).value for w in weights])
        Y = (ctypes.c_void_p * n)(*[_p(y).value for y in outputs])
        R = (ctypes.c_uint32 * n)(*rows)
        check(lib().g4_normAddMatmulSegmentsBatch(self.h, {"q4k": 0, "q6k": 1}[wtype], _p(x), _p(w1),
                                                  _p(residual), _p(w2), _p(h_out), W, Y, R, n, N, eps, softcap,
                                                  batch))

    def normAddGateUpGeluBatch(self, o: Ptr, w_post: Ptr, residual: Ptr, w_pre: Ptr, w_gate: Ptr, w_up: Ptr,
                               h_out: Ptr, out: Ptr, M: int, N: int, batch: int, eps: float = 1e-6) -> None:
        """normAddGateUpGelu_q4k over `batch` vectors: o/residual/h_out [batch][N], out [batch][M]."""
        check(lib().g4_normAddGateUpGeluBatch(self.h, _p(o), _p(w_post), _p(residual), _p(w_pre), _p(w_gate),
                                              _p(w_up), _p(h_out), _p(out), MatmulParams(M, N), eps, batch))

    def matmulSegmentsBatchPartial(self, wtype: str, x: Ptr, weights, outputs, rows, N: int, batch: int,
                                   max_ksplit: int, ops: Ptr = None, softcap: float = 0.0) -> int:
        """x [batch][N] (and its operand blocks `ops`, or None) times each weight; outputs[i] gets
        [ksplit][batch][rows[i]] partial sums. Returns ksplit (<= max_ksplit)."""
        n = len(weights)
        W = (ctypes.c_void_p * n)(*[_p(w).value for w in weights])
        Y = (ctypes.c_void_p * n)(*[_p(y).value for y in outputs])
        R = (ctypes.c_uint32 * n)(*rows)
        ks = ctypes.c_uint32(0)
        check(lib().g4_matmulSegmentsBatchPartial(self.h, {"q4k": 0, "q6k": 1}[wtype], _p(x), _p(ops), W, Y, R, n,
                                                  N, batch, max_ksplit, softcap, ctypes.byref(ks)))
        return int(ks.value)

    @staticmethod
    def batch_operand_bytes(N: int, batch: int) -> int:
        n = ctypes.c_size_t()
        check(lib().g4_batchOperandBytes(N, batch, ctypes.byref(n)))
        return int(n.value)

    def batchPrep(self, x_parts: Ptr, nparts: int, w1: Ptr, residual: Ptr, w2: Ptr, h_out: Ptr, out: Ptr, N: int,
                  batch: int, eps: float = 1e-6, ops: Ptr = None) -> None:
        """out = prologue(sum of nparts chunks of x_parts) per vector (rmsNorm / fusedNormAdd + rmsNorm);
        `ops` (optional) receives the matrix-core operand blocks of out."""
        check(lib().g4_batchPrep(self.h, _p(x_parts), nparts, _p(w1), _p(residual), _p(w2), _p(h_out), _p(out),
                                 _p(ops), N, batch, eps))

    def batchPrepScale(self, x_parts: Ptr, nparts: int, w1: Ptr, residual: Ptr, out_scale: Ptr, w2: Ptr,
                       h_out: Ptr, out: Ptr, N: int, batch: int, eps: float = 1e-6, ops: Ptr = None) -> None:
        """batchPrep with h = (residual + norm(x)*w1) * out_scale[0]; w2 None: out = h."""
        check(lib().g4_batchPrepScale(self.h, _p(x_parts), nparts, _p(w1), _p(residual), _p(out_scale), _p(w2),
                                      _p(h_out), _p(out), _p(ops), N, batch, eps))

    # ---- per-layer embeddings (shaders/ple_*.wgsl) ----
    def pleStage1Fuse(self, projected: Ptr, norm_w: Ptr, table: Ptr, table_rows: int, ple_inputs: Ptr,
                      num_layers: int, per_layer_dim: int = 256, eps: float = 1e-6, token: int = 0,
                      tokens_dev: Ptr = None, count: int = 1) -> None:
        check(lib().g4_pleStage1Fuse(self.h, _p(projected), _p(norm_w), _p(table), table_rows, token,
                                     _p(tokens_dev), _p(ple_inputs), num_layers, per_layer_dim, eps, count))

    def pleGeluMul(self, gate: Ptr, ple_inputs: Ptr, out: Ptr, layer_offset: int, size: int) -> None:
        check(lib().g4_pleGeluMul(self.h, _p(gate), _p(ple_inputs), _p(out), layer_offset, size))

    def pleSkipScaleAdd(self, hidden: Ptr, post_normed: Ptr, scale: Ptr, size: int) -> None:
        check(lib().g4_pleSkipScaleAdd(self.h, _p(hidden), _p(post_normed), _p(scale), size))

    def matmulF16(self, x: Ptr, w: Ptr, y: Ptr, M: int, N: int, batch: int = 1) -> None:
        check(lib().g4_matmulF16(self.h, _p(x), _p(w), _p(y), M, N, batch))

    def pleGate(self, x: Ptr, w1: Ptr, residual: Ptr, h_out: Ptr, w_gate: Ptr, ple_inputs: Ptr, ple_stride: int,
                layer_offset: int, out: Ptr, M: int, N: int, eps: float = 1e-6, batch: int = 1) -> None:
        check(lib().g4_pleGate(self.h, _p(x), _p(w1), _p(residual), _p(h_out), _p(w_gate), _p(ple_inputs),
                               ple_stride, layer_offset, _p(out), M, N, eps, batch))


    def gateUpGeluBatch(self, x: Ptr, w_gate: Ptr, w_up: Ptr, out: Ptr, M: int, N: int, batch: int,
                        ops: Ptr = None) -> None:
        check(lib().g4_gateUpGeluBatch(self.h, _p(x), _p(ops), _p(w_gate), _p(w_up), _p(out), MatmulParams(M, N),
                                       batch))

    @staticmethod
    def batch_sub_operand_bytes(K: int, batch: int) -> int:
        n = ctypes.c_size_t(0)
        check(lib().g4_batchSubOperandBytes(K, batch, ctypes.byref(n)))
        return int(n.value)

    def gateUpGeluBatchOps(self, x: Ptr, ops: Ptr, w_gate: Ptr, w_up: Ptr, out: Ptr, down_ops: Ptr, M: int, N: int,
                           batch: int) -> None:
        """gateUpGeluBatch that also writes the product's sub-block-scaled operand blocks (down_ops)."""
        check(lib().g4_gateUpGeluBatchOps(self.h, _p(x), _p(ops), _p(w_gate), _p(w_up), _p(out), _p(down_ops),
                                          MatmulParams(M, N), batch))

    def matmulSubBatchPartial(self, ops: Ptr, weight: Ptr, out: Ptr, M: int, K: int, batch: int,
                              max_ksplit: int) -> int:
        """Q6_K weight [M][K] times the vectors of sub-block-scaled operand blocks; out gets
        [ksplit][batch][M] partial sums. Returns ksplit (<= max_ksplit)."""
        ks = ctypes.c_uint32(0)
        check(lib().g4_matmulSubBatchPartial(self.h, _p(ops), _p(weight), _p(out), M, K, batch, max_ksplit,
                                             ctypes.byref(ks)))
        return int(ks.value)

    # ---- attention (kv_cache_store / attn_score / softmax / attn_output) ----
    def kvCacheStore(self, k_in: Ptr, v_in: Ptr, k_cache: Ptr, v_cache: Ptr, num_kv_heads: int, head_dim: int,
                     position: int, max_seq_len: int, position_dev: Ptr = None) -> None:
        p = KvStoreParams(num_kv_heads, head_dim, position, max_seq_len)
        if position_dev is None:
            check(lib().g4_kvCacheStore(self.h, _p(k_in), _p(v_in), _p(k_cache), _p(v_cache), p))
        else:
            check(lib().g4_kvCacheStore_dev(self.h, _p(k_in), _p(v_in), _p(k_cache), _p(v_cache), p,
                                            _p(position_dev)))

    def attnScore(self, q: Ptr, k_cache: Ptr, scores: Ptr, nqh: int, nkh: int, hd: int, seq_len: int,
                  scale: float = 1.0, window: int = 0, position_dev: Ptr = None) -> None:
        """With position_dev, seq_len = *position_dev + 1 on the device and the
        `seq_len` argument is the maximum (g4_attnScore_dev)."""
        p = AttnScoreParams(nqh, nkh, hd, seq_len, scale, window)
        if position_dev is None:
            check(lib().g4_attnScore(self.h, _p(q), _p(k_cache), _p(scores), p))
        else:
            check(lib().g4_attnScore_dev(self.h, _p(q), _p(k_cache), _p(scores), p, _p(position_dev)))

    def softmax(self, scores: Ptr, num_heads: int, seq_len: int, position_dev: Ptr = None) -> None:
        p = SoftmaxParams(num_heads, seq_len)
        if position_dev is None:
            check(lib().g4_softmax(self.h, _p(scores), p))
        else:
            check(lib().g4_softmax_dev(self.h, _p(scores), p, _p(position_dev)))

    def attnOutput(self, probs: Ptr, v_cache: Ptr, out: Ptr, nqh: int, nkh: int, hd: int, seq_len: int,
                   position_dev: Ptr = None) -> None:
        p = AttnOutputParams(nqh, nkh, hd, seq_len)
        if position_dev is None:
            check(lib().g4_attnOutput(self.h, _p(probs), _p(v_cache), _p(out), p))
        else:
            check(lib().g4_attnOutput_dev(self.h, _p(probs), _p(v_cache), _p(out), p, _p(position_dev)))

    @staticmethod
    def attn_workspace_bytes(nqh: int, nkh: int, hd: int, seq_len: int, window: int = 0) -> int:
        n = ctypes.c_size_t()
        check(lib().g4_attnDecode_workspace_size(AttnScoreParams(nqh, nkh, hd, seq_len, 1.0, window),
                                                 ctypes.byref(n)))
        return int(n.value)

    def attnDecode(self, q: Ptr, k_cache: Ptr, v_cache: Ptr, out: Ptr, nqh: int, nkh: int, hd: int, seq_len: int,
                   scale: float = 1.0, window: int = 0, workspace: Optional[Buffer] = None,
                   position_dev: Ptr = None) -> None:
        p = AttnScoreParams(nqh, nkh, hd, seq_len, scale, window)
        ws = workspace
        if ws is None:
            ws = self.zeros(self.attn_workspace_bytes(nqh, nkh, hd, seq_len, window), np.uint8)
        if position_dev is None:
            check(lib().g4_attnDecode(self.h, _p(q), _p(k_cache), _p(v_cache), _p(out), p, _p(ws), ws.nbytes))
        else:
            check(lib().g4_attnDecode_dev(self.h, _p(q), _p(k_cache), _p(v_cache), _p(out), p, _p(ws), ws.nbytes,
                                          _p(position_dev)))
        if workspace is None:
            self.sync()
            ws.free()

    def attnDecodeNoAlloc(self, q: Ptr, k_cache: Ptr, v_cache: Ptr, out: Ptr, nqh: int, nkh: int, hd: int,
                          seq_len: int, scale: float = 1.0, window: int = 0) -> None:
        """g4_attnDecode_noalloc: the partials in the library's static device
        array; no workspace, nothing allocated."""
        check(lib().g4_attnDecode_noalloc(self.h, _p(q), _p(k_cache), _p(v_cache), _p(out),
                                          AttnScoreParams(nqh, nkh, hd, seq_len, scale, window)))

    @staticmethod
    def attn_fused_params(nqh, nkh, hd, max_seq_len, window=0, eps=1e-6, theta=1e4, apply_divisor=0,
                          scale=1.0) -> AttnFusedParams:
        return AttnFusedParams(nqh, nkh, hd, max_seq_len, scale, window, eps, theta, apply_divisor)

    @staticmethod
    def attn_fused_workspace_bytes(p: AttnFusedParams) -> int:
        n = ctypes.c_size_t()
        check(lib().g4_attnDecodeFused_workspace_size(p, ctypes.byref(n)))
        return int(n.value)

    @staticmethod
    def attn_fused_single_launch(p: AttnFusedParams) -> bool:
        """Whether g4_attnDecodeFused runs as one launch (the matrix-core plan
        with its merge in the launch: head dim 256 or 512, 8 query heads per
        KV head, at most 64 KV heads, a window of at most 1024 positions)
        rather than an attention launch and a merge launch."""
        eff = min(p.max_seq_len, p.sliding_window) if p.sliding_window else p.max_seq_len
        return (p.head_dim in (256, 512) and p.num_q_heads == 8 * p.num_kv_heads and p.num_kv_heads <= 64
                and eff <= 1024)

    @staticmethod
    def qkv_attn_single_launch(p: AttnFusedParams, N: int, nseg: int = 3) -> bool:
        """Whether g4_qkvAttnDecodeFusedWarm runs as one launch: q, k and v
        (nseg 3), hidden 1536, one KV head of dim 256, a window of at most 1024
        positions."""
        eff = min(p.max_seq_len, p.sliding_window) if p.sliding_window else p.max_seq_len
        return (nseg == 3 and N == 1536 and p.head_dim == 256 and p.num_kv_heads == 1 and p.num_q_heads == 8
                and eff <= 1024)

    def attnDecodeFused(self, q_raw: Ptr, k_raw: Ptr, v_raw: Ptr, q_norm_w: Ptr, k_norm_w: Ptr, rope_freqs: Ptr,
                        k_cache: Ptr, v_cache: Ptr, out: Ptr, p: AttnFusedParams, workspace: Buffer,
                        position_dev: Ptr) -> None:
        """q/k norm + RoPE, v_norm, KV row store at *position_dev and decode attention in one launch."""
        check(lib().g4_attnDecodeFused(self.h, _p(q_raw), _p(k_raw), _p(v_raw), _p(q_norm_w), _p(k_norm_w),
                                       _p(rope_freqs), _p(k_cache), _p(v_cache), _p(out), p, _p(workspace),
                                       workspace.nbytes, _p(position_dev)))

    def matmulWarmRegion(self, wtype: str, M: int, N: int, weight: Ptr) -> WarmRegion:
        """The bytes each workgroup of the one-vector matvec launch over W [M x N] reads."""
        r = WarmRegion()
        check(lib().g4_matmulWarmRegion(self.h, {"q4k": 0, "q6k": 1}[wtype], M, N, _p(weight), ctypes.byref(r)))
        return r

    def attnDecodeFusedWarm(self, q_raw: Ptr, k_raw: Ptr, v_raw: Ptr, q_norm_w: Ptr, k_norm_w: Ptr,
                            rope_freqs: Ptr, k_cache: Ptr, v_cache: Ptr, out: Ptr, p: AttnFusedParams,
                            workspace: Buffer, position_dev: Ptr, regions, rope_cs: Ptr = None,
                            rope_rows: int = 0) -> None:
        """attnDecodeFused whose launch also reads `regions` (WarmRegion list, <= 4) into the L2 caches
        the matvecs that follow will read them through, taking the RoPE cos/sin from `rope_cs`
        (ropeTable) when given."""
        n = len(regions)
        arr = (WarmRegion * max(n, 1))(*regions)
        check(lib().g4_attnDecodeFusedWarm(self.h, _p(q_raw), _p(k_raw), _p(v_raw), _p(q_norm_w), _p(k_norm_w),
                                           _p(rope_freqs), _p(k_cache), _p(v_cache), _p(out), p, _p(workspace),
                                           workspace.nbytes, _p(position_dev), arr, n, _p(rope_cs), rope_rows))

    def qkvAttnDecodeFusedWarm(self, x: Ptr, w1: Ptr, residual: Ptr, out_scale: Ptr, w2: Ptr, h_out: Ptr,
                               weights, outputs, N: int, eps: float, q_norm_w: Ptr, k_norm_w: Ptr, rope_freqs: Ptr,
                               k_cache: Ptr, v_cache: Ptr, out: Ptr, p: AttnFusedParams, workspace: Buffer,
                               position_dev: Ptr, regions, rope_cs: Ptr = None, rope_rows: int = 0) -> None:
        """normAddScaleMatmulSegments('q4k', ...) into `outputs` (q, or q/k/v), then attnDecodeFusedWarm
        over them; one launch where the shape allows (g4_qkvAttnDecodeFusedWarm)."""
        n = len(weights)
        W = (ctypes.c_void_p * n)(*[_p(w).value for w in weights])
        Y = (ctypes.c_void_p * n)(*[_p(y).value for y in outputs])
        nr = len(regions)
        arr = (WarmRegion * max(nr, 1))(*regions)
        check(lib().g4_qkvAttnDecodeFusedWarm(self.h, _p(x), _p(w1), _p(residual), _p(out_scale), _p(w2), _p(h_out),
                                              W, Y, n, N, eps, _p(q_norm_w), _p(k_norm_w), _p(rope_freqs),
                                              _p(k_cache), _p(v_cache), _p(out), p, _p(workspace), workspace.nbytes,
                                              _p(position_dev), arr, nr, _p(rope_cs), rope_rows))

    def qkvAttnDecodePartials(self, x: Ptr, w1: Ptr, residual: Ptr, out_scale: Ptr, w2: Ptr, h_out: Ptr,
                              weights, outputs, N: int, eps: float, q_norm_w: Ptr, k_norm_w: Ptr, rope_freqs: Ptr,
                              k_cache: Ptr, v_cache: Ptr, p: AttnFusedParams, workspace: Buffer,
                              position_dev: Ptr, regions, rope_cs: Ptr = None, rope_rows: int = 0) -> None:
        """The one q/k/v + attention launch with its chunk merge left to
        attnHeadsMatmul_q4k (g4_qkvAttnDecodePartials)."""
        n = len(weights)
        W = (ctypes.c_void_p * n)(*[_p(w).value for w in weights])
        Y = (ctypes.c_void_p * n)(*[_p(y).value for y in outputs])
        nr = len(regions)
        arr = (WarmRegion * max(nr, 1))(*regions)
        check(lib().g4_qkvAttnDecodePartials(self.h, _p(x), _p(w1), _p(residual), _p(out_scale), _p(w2), _p(h_out),
                                             W, Y, n, N, eps, _p(q_norm_w), _p(k_norm_w), _p(rope_freqs),
                                             _p(k_cache), _p(v_cache), p, _p(workspace), workspace.nbytes,
                                             _p(position_dev), arr, nr, _p(rope_cs), rope_rows))

    def attnHeadsMatmul_q4k(self, workspace: Buffer, p: AttnFusedParams, position_dev: Ptr, weight: Ptr, out: Ptr,
                            M: int) -> None:
        """Chunk merge + o projection by group of heads: out[g][M] = sum over the group's heads h of
        W_o[:, 256h:256h+256] . merged head h (O_SHARES groups of 8 / O_SHARES heads)."""
        check(lib().g4_attnHeadsMatmul_q4k(self.h, _p(workspace), workspace.nbytes, p, _p(position_dev), _p(weight),
                                           _p(out), M))

    def normAddPartsGateUpGeluDigits_q4k(self, o_parts: Ptr, w_post: Ptr, residual: Ptr, w_pre: Ptr, w_gate: Ptr,
                                         w_up: Ptr, h_out: Ptr, out: Ptr, digits: Ptr, M: int, N: int,
                                         eps: float = 1e-6) -> None:
        """normAddGateUpGeluDigits_q4k with o given as O_SHARES shares [O_SHARES][N], added in order."""
        check(lib().g4_normAddPartsGateUpGeluDigits_q4k(self.h, _p(o_parts), _p(w_post), _p(residual), _p(w_pre),
                                                        _p(w_gate), _p(w_up), _p(h_out), _p(out), _p(digits),
                                                        MatmulParams(M, N), eps))

    def ropeTable(self, theta: float, apply_divisor: int, rope_freqs: Ptr, head_dim: int, rows: int,
                  table: Ptr) -> None:
        """table[t][i] = (cos, sin) of position t's RoPE angle for pair i (rows x head_dim/2 float2)."""
        check(lib().g4_ropeTable(self.h, theta, apply_divisor, _p(rope_freqs), head_dim, rows, _p(table)))

    @staticmethod
    def paged_params(num_seqs, nqh, nkh, hd, page_size, max_pages, max_seq_len, num_pages, scale=1.0, window=0):
        return PagedAttnParams(num_seqs, nqh, nkh, hd, page_size, max_pages, max_seq_len, num_pages, scale, window)

    @staticmethod
    def paged_workspace_bytes(p: PagedAttnParams) -> int:
        n = ctypes.c_size_t()
        check(lib().g4_pagedAttnDecode_workspace_size(p, ctypes.byref(n)))
        return int(n.value)

    def pagedAttnDecode(self, q: Ptr, k_pool: Ptr, v_pool: Ptr, page_table: Ptr, seq_lens: Ptr, out: Ptr,
                        p: PagedAttnParams, workspace: Buffer, ops: Ptr = None) -> None:
        """With `ops`, the output also as the o projection's operand blocks (g4_pagedAttnDecodeOps)."""
        if ops is None:
            check(lib().g4_pagedAttnDecode(self.h, _p(q), _p(k_pool), _p(v_pool), _p(page_table), _p(seq_lens),
                                           _p(out), p, _p(workspace), workspace.nbytes))
        else:
            check(lib().g4_pagedAttnDecodeOps(self.h, _p(q), _p(k_pool), _p(v_pool), _p(page_table),
                                              _p(seq_lens), _p(out), p, _p(workspace), workspace.nbytes, _p(ops)))

    def pagedKvStore(self, k_in: Ptr, v_in: Ptr, k_pool: Ptr, v_pool: Ptr, page_table: Ptr, seq_lens: Ptr,
                     p: PagedAttnParams) -> None:
        check(lib().g4_pagedKvStore(self.h, _p(k_in), _p(v_in), _p(k_pool), _p(v_pool), _p(page_table),
                                    _p(seq_lens), p))

    @staticmethod
    def paged_fused_params(num_seqs, nqh, nkh, hd, page_size, max_pages, max_seq_len, num_pages, window, eps,
                           theta, apply_divisor, scale=1.0):
        return PagedAttnFusedParams(num_seqs, nqh, nkh, hd, page_size, max_pages, max_seq_len, num_pages, scale,
                                    window, eps, theta, apply_divisor)

    @staticmethod
    def paged_fused_workspace_bytes(p: PagedAttnFusedParams) -> int:
        n = ctypes.c_size_t()
        check(lib().g4_pagedAttnDecodeFused_workspace_size(p, ctypes.byref(n)))
        return int(n.value)

    def pagedAttnDecodeFused(self, q_raw: Ptr, k_raw: Ptr, v_raw: Ptr, q_norm_w: Ptr, k_norm_w: Ptr,
                             rope_freqs: Ptr, k_pool: Ptr, v_pool: Ptr, page_table: Ptr, seq_lens: Ptr, out: Ptr,
                             p: PagedAttnFusedParams, workspace: Buffer) -> None:
        """Per sequence: q/k norm + RoPE, v_norm, KV row store into the pool page and decode attention."""
        check(lib().g4_pagedAttnDecodeFused(self.h, _p(q_raw), _p(k_raw), _p(v_raw), _p(q_norm_w), _p(k_norm_w),
                                            _p(rope_freqs), _p(k_pool), _p(v_pool), _p(page_table), _p(seq_lens),
                                            _p(out), p, _p(workspace), workspace.nbytes))

    def pagedAttnPrologue(self, q_parts: Ptr, k_parts: Ptr, v_parts: Ptr, nparts: int, q_norm_w: Ptr, k_norm_w: Ptr,
                          rope_freqs: Ptr, q_out: Ptr, k_pool: Ptr, v_pool: Ptr, page_table: Ptr, seq_lens: Ptr,
                          p: PagedAttnFusedParams, rope_cs: Ptr = None, rope_rows: int = 0) -> None:
        """Per sequence: q_norm + RoPE into q_out, K/V row (k_norm + RoPE, v_norm) appended to the pool
        (RoPE cos/sin from the ropeTable `rope_cs` when given)."""
        check(lib().g4_pagedAttnPrologue(self.h, _p(q_parts), _p(k_parts), _p(v_parts), nparts, _p(q_norm_w),
                                         _p(k_norm_w), _p(rope_freqs), _p(q_out), _p(k_pool), _p(v_pool),
                                         _p(page_table), _p(seq_lens), p, _p(rope_cs), rope_rows))

    @staticmethod
    def paged_block_workspace_bytes(p: PagedAttnFusedParams, nparts: int) -> int:
        n = ctypes.c_size_t()
        check(lib().g4_pagedAttnBlock_workspace_size(p, nparts, ctypes.byref(n)))
        return int(n.value)

    def pagedAttnBlock(self, q_parts: Ptr, k_parts: Ptr, v_parts: Ptr, nparts: int, q_norm_w: Ptr, k_norm_w: Ptr,
                       rope_freqs: Ptr, q_out: Ptr, k_pool: Ptr, v_pool: Ptr, page_table: Ptr, seq_lens: Ptr,
                       out: Ptr, p: PagedAttnFusedParams, workspace: Buffer, ops: Ptr = None, rope_cs: Ptr = None,
                       rope_rows: int = 0) -> None:
        """pagedAttnPrologue + pagedAttnDecode(Ops) in one launch where the window allows
        (g4_pagedAttnBlock); workspace: paged_block_workspace_bytes, zeroed once."""
        check(lib().g4_pagedAttnBlock(self.h, _p(q_parts), _p(k_parts), _p(v_parts), nparts, _p(q_norm_w),
                                      _p(k_norm_w), _p(rope_freqs), _p(q_out), _p(k_pool), _p(v_pool),
                                      _p(page_table), _p(seq_lens), _p(out), _p(ops), p, _p(workspace),
                                      workspace.nbytes, _p(rope_cs), rope_rows))

    def advanceSeqLens(self, seq_lens: Ptr, num_seqs: int, delta: int = 1) -> None:
        check(lib().g4_advanceSeqLens(self.h, _p(seq_lens), num_seqs, delta))

    # ---- norms / activations ----
    def perHeadRmsNormNoWeight(self, data: Ptr, num_heads: int, head_dim: int, eps: float = 1e-6) -> None:
        check(lib().g4_perHeadRmsNormNoWeight(self.h, _p(data), PerHeadNormParams(num_heads, head_dim, eps, 0)))

    def fusedPerHeadNormRope(self, data: Ptr, weight: Ptr, num_heads: int, head_dim: int, eps: float,
                             position: int, theta: float, apply_divisor: int, rope_freqs: Ptr,
                             position_dev: Ptr = None) -> None:
        p = NormRopeParams(num_heads, head_dim, eps, position, theta, apply_divisor)
        if position_dev is None:
            check(lib().g4_fusedPerHeadNormRope(self.h, _p(data), _p(weight), p, _p(rope_freqs)))
        else:
            check(lib().g4_fusedPerHeadNormRope_dev(self.h, _p(data), _p(weight), p, _p(rope_freqs),
                                                    _p(position_dev)))

    def rmsNorm(self, x: Ptr, w: Ptr, out: Ptr, hidden_size: int, eps: float = 1e-6) -> None:
        check(lib().g4_rmsNorm(self.h, _p(x), _p(w), _p(out), RmsNormParams(hidden_size, eps)))

    def fusedNormAdd(self, x: Ptr, w: Ptr, residual: Ptr, out: Ptr, size: int, eps: float = 1e-6) -> None:
        check(lib().g4_fusedNormAdd(self.h, _p(x), _p(w), _p(residual), _p(out), NormAddParams(size, eps)))

    def geluMul(self, gate: Ptr, up: Ptr, out: Ptr, size: int) -> None:
        check(lib().g4_geluMul(self.h, _p(gate), _p(up), _p(out), size))

    def logitSoftcap(self, logits: Ptr, size: int, cap: float = 30.0) -> None:
        check(lib().g4_logitSoftcap(self.h, _p(logits), SoftcapParams(size, cap)))

    def embeddingLookup(self, embedding: Ptr, num_rows: int, out: Ptr, hidden_size: int, token_id: int = 0,
                        token_dev: Ptr = None) -> None:
        """shaders/embedding_lookup.wgsl: out = f32(embedding[token row]) * sqrt(hidden_size)."""
        p = EmbeddingParams(hidden_size, token_id)
        if token_dev is None:
            check(lib().g4_embeddingLookup(self.h, _p(embedding), num_rows, _p(out), p))
        else:
            check(lib().g4_embeddingLookup_dev(self.h, _p(embedding), num_rows, _p(out), p, _p(token_dev)))

    def embeddingLookupBatch(self, embedding: Ptr, num_rows: int, out: Ptr, hidden_size: int, tokens_dev: Ptr,
                             count: int) -> None:
        """Row r of out [count][hidden_size] = the embedding of tokens_dev[r]."""
        check(lib().g4_embeddingLookupBatch(self.h, _p(embedding), num_rows, _p(out), hidden_size, _p(tokens_dev),
                                            count))

    def advancePosition(self, position_dev: Ptr, delta: int = 1) -> None:
        check(lib().g4_advancePosition(self.h, _p(position_dev), delta))

    def argmax(self, logits: Ptr, result: Ptr, size: int) -> None:
        check(lib().g4_argmax(self.h, _p(logits), _p(result), size))

    def topk256(self, logits: Ptr, result: Ptr, size: int) -> None:
        check(lib().g4_topk256(self.h, _p(logits), _p(result), size))

    def argmaxBatch(self, logits: Ptr, result: Ptr, size: int, batch: int) -> None:
        check(lib().g4_argmaxBatch(self.h, _p(logits), _p(result), size, batch))

    def argmaxAdvance(self, logits: Ptr, result: Ptr, size: int, batch: int, positions: Ptr, delta: int = 1) -> None:
        """argmaxBatch, then positions[r] += delta for each row (done by the reduction's final stage)."""
        check(lib().g4_argmaxAdvance(self.h, _p(logits), _p(result), size, batch, _p(positions), delta))

    def topk256Batch(self, logits: Ptr, result: Ptr, size: int, batch: int) -> None:
        check(lib().g4_topk256Batch(self.h, _p(logits), _p(result), size, batch))

    # ---- debug / synthetic inputs ----
    def dequant_q4k(self, blocks: Ptr, nblocks: int, out: Ptr) -> None:
        check(lib().g4_dequant_q4k(self.h, _p(blocks), nblocks, _p(out)))

    def dequant_q6k(self, blocks: Ptr, nblocks: int, out: Ptr) -> None:
        check(lib().g4_dequant_q6k(self.h, _p(blocks), nblocks, _p(out)))

    def dequantPath(self, wtype: str, path: int, blocks: Ptr, nblocks: int, out: Ptr) -> None:
        """Weight values through the unpack of one kernel family (0: register
        units, 1: LDS units, 2: matrix-core operands)."""
        check(lib().g4_dequantPath(self.h, {"q4k": 0, "q6k": 1}[wtype], path, _p(blocks), nblocks, _p(out)))

    def dequantF16(self, wtype: str, blocks: Ptr, nblocks: int, out: Ptr) -> None:
        """Blocks ("q4k", "q6k", "q5k": 256 values; "q8_0": 32) to f16 values
        (round to nearest even of the f32 dequant)."""
        check(lib().g4_dequantF16(self.h, {"q4k": 0, "q6k": 1, "q5k": 2, "q8_0": 3}[wtype], _p(blocks), nblocks,
                                  _p(out)))

    def streamRead(self, src: Ptr, nbytes: int, policy: int, nwgs: int, sink: Ptr) -> None:
        """Measurement probe: one pass of 16-byte loads over nbytes (policy 0
        plain, 1 non-temporal, 2 device scope)."""
        check(lib().g4_streamRead(self.h, _p(src), nbytes, policy, nwgs, _p(sink)))

    def fill_q4k(self, dst: Ptr, nblocks: int, seed: int) -> None:
        check(lib().g4_fill_q4k(self.h, _p(dst), nblocks, seed))

    def fill_q6k(self, dst: Ptr, nblocks: int, seed: int) -> None:
        check(lib().g4_fill_q6k(self.h, _p(dst), nblocks, seed))

    def fill_q5k(self, dst: Ptr, nblocks: int, seed: int) -> None:
        check(lib().g4_fill_q5k(self.h, _p(dst), nblocks, seed))

    def fill_normal_f32(self, dst: Ptr, n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> None:
        check(lib().g4_fill_normal_f32(self.h, _p(dst), n, seed, mean, std))

    def fill_normal_f16(self, dst: Ptr, n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> None:
        check(lib().g4_fill_normal_f16(self.h, _p(dst), n, seed, mean, std))


def splitmix64(seed: int, idx: int) -> int:
    return int(lib().g4_splitmix64(seed, idx))
