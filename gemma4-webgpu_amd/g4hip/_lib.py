"""ctypes declarations of the libg4hip C ABI (include/g4hip.h)."""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG, "libg4hip.so")

G4_OK = 0
O_SHARES = 4  # G4_O_SHARES: shares of o g4_attnHeadsMatmul_q4k writes
ERRORS = {
    -1: "G4_ERR_INVALID",
    -2: "G4_ERR_HIP",
    -3: "G4_ERR_DEVICE_LOST",
    -4: "G4_ERR_OOM",
    -5: "G4_ERR_UNSUPPORTED",
    -6: "G4_ERR_NO_DEVICE",
    -7: "G4_ERR_STALLED",
}


class G4Error(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{ERRORS.get(code, code)}: {msg}")
        self.code = code


# --- Params structs: field for field the WGSL `Params` of each kernel --------

class MatmulParams(ctypes.Structure):  # shaders/matmul_quant.wgsl:12
    _fields_ = [("M", ctypes.c_uint32), ("N", ctypes.c_uint32)]


class KvStoreParams(ctypes.Structure):  # shaders/kv_cache_store.wgsl:1
    _fields_ = [("num_kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("position", ctypes.c_uint32), ("max_seq_len", ctypes.c_uint32)]


class AttnScoreParams(ctypes.Structure):  # shaders/attn_score.wgsl:9
    _fields_ = [("num_q_heads", ctypes.c_uint32), ("num_kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("seq_len", ctypes.c_uint32),
                ("scale", ctypes.c_float), ("sliding_window", ctypes.c_uint32)]


class SoftmaxParams(ctypes.Structure):  # shaders/softmax.wgsl:1
    _fields_ = [("num_heads", ctypes.c_uint32), ("seq_len", ctypes.c_uint32)]


class AttnOutputParams(ctypes.Structure):  # shaders/attn_output.wgsl:1
    _fields_ = [("num_q_heads", ctypes.c_uint32), ("num_kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("seq_len", ctypes.c_uint32)]


class WarmRegion(ctypes.Structure):  # g4_warm_region
    _fields_ = [("base", ctypes.c_void_p), ("total_bytes", ctypes.c_uint64), ("wg_bytes", ctypes.c_uint64),
                ("nwgs", ctypes.c_uint32), ("reserved", ctypes.c_uint32)]


class AttnFusedParams(ctypes.Structure):
    _fields_ = [("num_q_heads", ctypes.c_uint32), ("num_kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("max_seq_len", ctypes.c_uint32),
                ("scale", ctypes.c_float), ("sliding_window", ctypes.c_uint32),
                ("eps", ctypes.c_float), ("theta", ctypes.c_float), ("apply_divisor", ctypes.c_uint32)]


class PagedAttnParams(ctypes.Structure):
    _fields_ = [("num_seqs", ctypes.c_uint32), ("num_q_heads", ctypes.c_uint32),
                ("num_kv_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("page_size", ctypes.c_uint32), ("max_pages", ctypes.c_uint32),
                ("max_seq_len", ctypes.c_uint32), ("num_pages", ctypes.c_uint32),
                ("scale", ctypes.c_float), ("sliding_window", ctypes.c_uint32)]


class PagedAttnFusedParams(ctypes.Structure):
    _fields_ = PagedAttnParams._fields_ + [("eps", ctypes.c_float), ("theta", ctypes.c_float),
                                           ("apply_divisor", ctypes.c_uint32)]


class PerHeadNormParams(ctypes.Structure):  # shaders/per_head_rms_norm_no_weight.wgsl:8
    _fields_ = [("num_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("eps", ctypes.c_float), ("pad", ctypes.c_uint32)]


class NormRopeParams(ctypes.Structure):  # shaders/fused_per_head_norm_rope.wgsl:13
    _fields_ = [("num_heads", ctypes.c_uint32), ("head_dim", ctypes.c_uint32),
                ("eps", ctypes.c_float), ("position", ctypes.c_uint32),
                ("theta", ctypes.c_float), ("apply_divisor", ctypes.c_uint32)]


class RmsNormParams(ctypes.Structure):  # shaders/rms_norm.wgsl:2
    _fields_ = [("hidden_size", ctypes.c_uint32), ("eps", ctypes.c_float)]


class NormAddParams(ctypes.Structure):  # shaders/fused_norm_add.wgsl:2
    _fields_ = [("size", ctypes.c_uint32), ("eps", ctypes.c_float)]


class SoftcapParams(ctypes.Structure):  # shaders/logit_softcap.wgsl:5
    _fields_ = [("size", ctypes.c_uint32), ("cap", ctypes.c_float)]


class EmbeddingParams(ctypes.Structure):  # shaders/embedding_lookup.wgsl:2
    _fields_ = [("hidden_size", ctypes.c_uint32), ("token_id", ctypes.c_uint32)]


_P = ctypes.c_void_p
_I = ctypes.c_int
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_SZ = ctypes.c_size_t
_F = ctypes.c_float
_PP = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes); every int-returning entry is status-checked.
SIGNATURES = {
    "g4_last_error": (ctypes.c_char_p, []),
    "g4_version": (_I, []),
    "g4_init": (_I, [_I, _PP]),
    "g4_destroy": (_I, [_P]),
    "g4_set_stream": (_I, [_P, _P]),
    "g4_get_stream": (_P, [_P]),
    "g4_device_info": (_I, [_P, ctypes.c_char_p, _SZ, ctypes.POINTER(_I), ctypes.POINTER(_SZ)]),
    "g4_alloc": (_I, [_P, _SZ, _PP]),
    "g4_free": (_I, [_P, _P]),
    "g4_memset": (_I, [_P, _P, _I, _SZ]),
    "g4_upload": (_I, [_P, _P, _P, _SZ, _SZ]),
    "g4_download": (_I, [_P, _P, _P, _SZ, _SZ]),
    "g4_download_async": (_I, [_P, _P, _P, _SZ, _SZ, _PP]),
    "g4_copy_d2d": (_I, [_P, _P, _P, _SZ]),
    "g4_stream_sync": (_I, [_P]),
    "g4_clear_stall": (_I, [_P]),
    "g4_host_alloc": (_I, [_P, _SZ, ctypes.POINTER(_P)]),
    "g4_host_free": (_I, [_P]),
    "g4_graph_kernel_nodes": (_I, [_P, ctypes.POINTER(ctypes.c_size_t)]),
    "g4_test_stage_wait": (_I, [_P, _U32, _I]),
    "g4_event_record": (_I, [_P, _PP]),
    "g4_event_query": (_I, [_P]),
    "g4_event_wait": (_I, [_P]),
    "g4_event_elapsed_ms": (_I, [_P, _P, ctypes.POINTER(_F)]),
    "g4_event_destroy": (_I, [_P]),
    "g4_graph_begin": (_I, [_P]),
    "g4_graph_end": (_I, [_P, _PP]),
    "g4_graph_launch": (_I, [_P, _P]),
    "g4_graph_destroy": (_I, [_P]),
    "g4_matmulQuant_q4k": (_I, [_P, _P, _P, _P, MatmulParams]),
    "g4_matmulQuant_q6k": (_I, [_P, _P, _P, _P, MatmulParams]),
    "g4_matmulQuant_f16": (_I, [_P, _P, _P, _P, MatmulParams]),
    "g4_matmulQuantMR4_q4k": (_I, [_P, _P, _P, _P, MatmulParams]),
    "g4_matmulQuantBatch_q4k": (_I, [_P, _P, _P, _P, MatmulParams, _U32]),
    "g4_matmulQuantBatch_q6k": (_I, [_P, _P, _P, _P, MatmulParams, _U32]),
    "g4_kvCacheStore": (_I, [_P, _P, _P, _P, _P, KvStoreParams]),
    "g4_kvCacheStore_dev": (_I, [_P, _P, _P, _P, _P, KvStoreParams, _P]),
    "g4_attnScore": (_I, [_P, _P, _P, _P, AttnScoreParams]),
    "g4_softmax": (_I, [_P, _P, SoftmaxParams]),
    "g4_attnOutput": (_I, [_P, _P, _P, _P, AttnOutputParams]),
    "g4_attnScore_dev": (_I, [_P, _P, _P, _P, AttnScoreParams, _P]),
    "g4_softmax_dev": (_I, [_P, _P, SoftmaxParams, _P]),
    "g4_attnOutput_dev": (_I, [_P, _P, _P, _P, AttnOutputParams, _P]),
    "g4_attnDecode_workspace_size": (_I, [AttnScoreParams, ctypes.POINTER(_SZ)]),
    "g4_attnDecode": (_I, [_P, _P, _P, _P, _P, AttnScoreParams, _P, _SZ]),
    "g4_attnDecode_dev": (_I, [_P, _P, _P, _P, _P, AttnScoreParams, _P, _SZ, _P]),
    "g4_attnDecode_noalloc": (_I, [_P, _P, _P, _P, _P, AttnScoreParams]),
    "g4_attnDecodeFused_workspace_size": (_I, [AttnFusedParams, ctypes.POINTER(_SZ)]),
    "g4_attnDecodeFused": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, AttnFusedParams, _P, _SZ, _P]),
    "g4_attnDecodeFusedWarm": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, AttnFusedParams, _P, _SZ, _P,
                                    ctypes.POINTER(WarmRegion), _I, _P, _U32]),
    "g4_qkvAttnDecodeFusedWarm": (_I, [_P, _P, _P, _P, _P, _P, _P, ctypes.POINTER(_P), ctypes.POINTER(_P), _I, _U32,
                                       _F, _P, _P, _P, _P, _P, _P, AttnFusedParams, _P, _SZ, _P,
                                       ctypes.POINTER(WarmRegion), _I, _P, _U32]),
    "g4_qkvAttnDecodePartials": (_I, [_P, _P, _P, _P, _P, _P, _P, ctypes.POINTER(_P), ctypes.POINTER(_P), _I, _U32,
                                      _F, _P, _P, _P, _P, _P, AttnFusedParams, _P, _SZ, _P,
                                      ctypes.POINTER(WarmRegion), _I, _P, _U32]),
    "g4_attnHeadsMatmul_q4k": (_I, [_P, _P, _SZ, AttnFusedParams, _P, _P, _P, _U32]),
    "g4_normAddPartsGateUpGeluDigits_q4k": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, MatmulParams, _F]),
    "g4_ropeTable": (_I, [_P, _F, _U32, _P, _U32, _U32, _P]),
    "g4_matmulWarmRegion": (_I, [_P, _I, _U32, _U32, _P, ctypes.POINTER(WarmRegion)]),
    "g4_pagedAttnDecode_workspace_size": (_I, [PagedAttnParams, ctypes.POINTER(_SZ)]),
    "g4_pagedAttnDecode": (_I, [_P, _P, _P, _P, _P, _P, _P, PagedAttnParams, _P, _SZ]),
    "g4_pagedAttnDecodeOps": (_I, [_P, _P, _P, _P, _P, _P, _P, PagedAttnParams, _P, _SZ, _P]),
    "g4_pagedKvStore": (_I, [_P, _P, _P, _P, _P, _P, _P, PagedAttnParams]),
    "g4_pagedAttnDecodeFused_workspace_size": (_I, [PagedAttnFusedParams, ctypes.POINTER(_SZ)]),
    "g4_pagedAttnDecodeFused": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, PagedAttnFusedParams, _P,
                                     _SZ]),
    "g4_advanceSeqLens": (_I, [_P, _P, _U32, _U32]),
    "g4_perHeadRmsNormNoWeight": (_I, [_P, _P, PerHeadNormParams]),
    "g4_fusedPerHeadNormRope": (_I, [_P, _P, _P, NormRopeParams, _P]),
    "g4_fusedPerHeadNormRope_dev": (_I, [_P, _P, _P, NormRopeParams, _P, _P]),
    "g4_rmsNorm": (_I, [_P, _P, _P, _P, RmsNormParams]),
    "g4_fusedNormAdd": (_I, [_P, _P, _P, _P, _P, NormAddParams]),
    "g4_geluMul": (_I, [_P, _P, _P, _P, _U32]),
    "g4_logitSoftcap": (_I, [_P, _P, SoftcapParams]),
    "g4_embeddingLookup": (_I, [_P, _P, _U32, _P, EmbeddingParams]),
    "g4_embeddingLookup_dev": (_I, [_P, _P, _U32, _P, EmbeddingParams, _P]),
    "g4_embeddingLookupBatch": (_I, [_P, _P, _U32, _P, _U32, _P, _U32]),
    "g4_advancePosition": (_I, [_P, _P, _U32]),
    "g4_argmax": (_I, [_P, _P, _P, _U32]),
    "g4_topk256": (_I, [_P, _P, _P, _U32]),
    "g4_argmaxBatch": (_I, [_P, _P, _P, _U32, _U32]),
    "g4_argmaxAdvance": (_I, [_P, _P, _P, _U32, _U32, _P, _U32]),
    "g4_topk256Batch": (_I, [_P, _P, _P, _U32, _U32]),
    "g4_rmsNormMatmul_q4k": (_I, [_P, _P, _P, _P, _P, MatmulParams, _F]),
    "g4_normAddGateUpGelu_q4k": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, MatmulParams, _F]),
    "g4_normAddMatmulSegments": (_I, [_P, _I, _P, _P, _P, _P, _P, ctypes.POINTER(_P),
                                      ctypes.POINTER(_P), ctypes.POINTER(_U32), _I, _U32, _F, _F]),
    "g4_digitsBytes": (_I, [_U32, ctypes.POINTER(_SZ)]),
    "g4_normAddGateUpGeluDigits_q4k": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, MatmulParams, _F]),
    "g4_matmulQuantDigits_q6k": (_I, [_P, _P, _P, _P, MatmulParams]),
    "g4_normAddMatmulArgmax": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _U32, _U32, _F, _F, _P, _P, _U32]),
    "g4_normAddMatmulTopk": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _U32, _U32, _F, _F, _P]),
    "g4_matmulSegmentsBatchPartial": (_I, [_P, _I, _P, _P, ctypes.POINTER(_P), ctypes.POINTER(_P),
                                           ctypes.POINTER(_U32), _I, _U32, _U32, _U32, _F,
                                           ctypes.POINTER(_U32)]),
    "g4_batchOperandBytes": (_I, [_U32, _U32, ctypes.POINTER(_SZ)]),
    "g4_batchPrep": (_I, [_P, _P, _U32, _P, _P, _P, _P, _P, _P, _U32, _U32, _F]),
    "g4_gateUpGeluBatch": (_I, [_P, _P, _P, _P, _P, _P, MatmulParams, _U32]),
    "g4_batchSubOperandBytes": (_I, [_U32, _U32, ctypes.POINTER(_SZ)]),
    "g4_gateUpGeluBatchOps": (_I, [_P, _P, _P, _P, _P, _P, _P, MatmulParams, _U32]),
    "g4_matmulSubBatchPartial": (_I, [_P, _P, _P, _P, _U32, _U32, _U32, _U32, ctypes.POINTER(_U32)]),
    "g4_pagedAttnPrologue": (_I, [_P, _P, _P, _P, _U32, _P, _P, _P, _P, _P, _P, _P, _P, PagedAttnFusedParams,
                                  _P, _U32]),
    "g4_pagedAttnBlock_workspace_size": (_I, [PagedAttnFusedParams, _U32, ctypes.POINTER(_SZ)]),
    "g4_pagedAttnBlock": (_I, [_P, _P, _P, _P, _U32, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, PagedAttnFusedParams,
                               _P, _SZ, _P, _U32]),
    "g4_normAddGateUpGeluBatch": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, MatmulParams, _F, _U32]),
    "g4_normAddMatmulSegmentsBatch": (_I, [_P, _I, _P, _P, _P, _P, _P, ctypes.POINTER(_P),
                                           ctypes.POINTER(_P), ctypes.POINTER(_U32), _I, _U32, _F, _F, _U32]),
    "g4_dequant_q4k": (_I, [_P, _P, _U64, _P]),
    "g4_dequant_q6k": (_I, [_P, _P, _U64, _P]),
    "g4_dequantPath": (_I, [_P, _I, _I, _P, _U64, _P]),
    "g4_dequantF16": (_I, [_P, _I, _P, _U64, _P]),
    "g4_streamRead": (_I, [_P, _P, _U64, _I, _U32, _P]),
    "g4_gguf_open": (_I, [ctypes.c_char_p, _PP]),
    "g4_gguf_open_memory": (_I, [_P, _SZ, _PP]),
    "g4_gguf_close": (_I, [_P]),
    "g4_gguf_info": (_I, [_P, ctypes.POINTER(_U32), ctypes.POINTER(_U64), ctypes.POINTER(_U64),
                          ctypes.POINTER(_U64), ctypes.POINTER(_U32)]),
    "g4_gguf_find_key": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "g4_gguf_kv": (_I, [_P, _U64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U32), ctypes.POINTER(_U32),
                        ctypes.POINTER(_U64)]),
    "g4_gguf_kv_number": (_I, [_P, _U64, _U64, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64),
                               ctypes.POINTER(_U64)]),
    "g4_gguf_kv_string": (_I, [_P, _U64, _U64, _PP, ctypes.POINTER(_U64)]),
    "g4_gguf_find_tensor": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "g4_gguf_tensor": (_I, [_P, _U64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_U32), ctypes.POINTER(_U64),
                            ctypes.POINTER(_U32), ctypes.POINTER(_U64), ctypes.POINTER(_U64)]),
    "g4_gguf_tensor_data": (_I, [_P, _U64, _PP]),
    "g4_gguf_upload": (_I, [_P, _P, _U64, _P, _SZ]),
    "g4_gguf_upload_f16": (_I, [_P, _P, _U64, _P, _SZ]),
    "g4_normAddScaleMatmulSegments": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, ctypes.POINTER(_P), ctypes.POINTER(_P),
                                           ctypes.POINTER(_U32), _I, _U32, _F, _F]),
    "g4_batchPrepScale": (_I, [_P, _P, _U32, _P, _P, _P, _P, _P, _P, _P, _U32, _U32, _F]),
    "g4_pleStage1Fuse": (_I, [_P, _P, _P, _P, _U32, _U32, _P, _P, _U32, _U32, _F, _U32]),
    "g4_pleGeluMul": (_I, [_P, _P, _P, _P, _U32, _U32]),
    "g4_pleSkipScaleAdd": (_I, [_P, _P, _P, _P, _U32]),
    "g4_matmulF16": (_I, [_P, _P, _P, _P, _U32, _U32, _U32]),
    "g4_pleGate": (_I, [_P, _P, _P, _P, _P, _P, _P, _U32, _U32, _P, _U32, _U32, _F, _U32]),
    "g4_fill_q5k": (_I, [_P, _P, _U64, _U64]),
    "g4_splitmix64": (_U64, [_U64, _U64]),
    "g4_fill_q4k": (_I, [_P, _P, _U64, _U64]),
    "g4_fill_q6k": (_I, [_P, _P, _U64, _U64]),
    "g4_fill_normal_f32": (_I, [_P, _P, _U64, _U64, _F, _F]),
    "g4_fill_normal_f16": (_I, [_P, _P, _U64, _U64, _F, _F]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libg4hip.so; raise if it was not built (no fallback path exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C gemma4-webgpu_amd/csrc` "
                "(or __graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int) -> int:
    if rc < 0:
        msg = lib().g4_last_error()
        raise G4Error(rc, msg.decode("utf-8", "replace") if msg else "")
    return rc
