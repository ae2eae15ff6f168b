"""ctypes binding of libindecis_hip.so (include/indecis_hip.h).

The library is built in-tree by indecis_amd.build (or __graft_entry__.build)
and loaded from indecis_amd/libindecis_hip.so. There is no fallback: if it
is missing, or no GPU is visible when a GPU entry point is called, these
functions raise.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
SO_PATH = os.path.join(HERE, "libindecis_hip.so")

# every exported entry point, as declared in include/indecis_hip.h
EXPORTS = [
    "ixh_last_error", "ixh_device_count", "ixh_model_create", "ixh_model_destroy",
    "ixh_model_set_matrix", "ixh_model_set_norm", "ixh_model_set_embeddings_f32",
    "ixh_model_set_embeddings_bf16", "ixh_model_set_embeddings_i8", "ixh_model_set_rope",
    "ixh_model_invalidate", "ixh_encode_seqs", "ixh_encode_tokens", "ixh_encode_device",
    "ixh_head_logits", "ixh_packb8_create", "ixh_packb8_destroy", "ixh_matmul8",
    "ixh_matmul8_outliers", "ixh_linear8", "ixh_model_load_safetensors", "ixh_safetensors_tensor",
    "ixh_tokenizer_load", "ixh_tokenizer_destroy", "ixh_tokenizer_info", "ixh_tokenizer_encode",
    "ixh_tokenizer_encode_pair", "ixh_tokenizer_encode_offsets", "ixh_tokenizer_encode_batch",
    "ixh_embed_texts", "ixh_embed_normalize",
    "ixh_matmul8_tile", "ixh_layernorm_quant", "ixh_ln_matmul8_geglu", "ixh_attend8",
    "ixh_model_set_profiling", "ixh_model_set_profile_filter", "ixh_model_profile",
    "ixh_check_exp255", "ixh_check_gelu", "ixh_check_mfma_rate", "ixh_batcher_create", "ixh_batcher_encode", "ixh_batcher_stats",
    "ixh_batcher_destroy", "ixh_model_set_option", "ixh_model_get_option", "ixh_packb8_set_option",
    "ixh_model_set_heads", "ixh_encode_heads", "ixh_matmul8_noalloc",
]

IXH_OK, IXH_EINVAL, IXH_ERANGE, IXH_ESTATE, IXH_EHIP, IXH_ENOMEM, IXH_EFORMAT = range(7)
POOL_MEAN, POOL_CLS = 0, 1
MAT_QKV, MAT_O, MAT_I, MAT_OMLP = range(4)
NORM_EMB, NORM_ATTN, NORM_MLP, NORM_FINAL = range(4)
LAYOUT_ROWS, LAYOUT_PANELS = 0, 1
OUT_POOLED, OUT_TOKENS = 0, 1
(OPT_PARTS, OPT_PASS_TOKENS, OPT_QKV_FUSED, OPT_QKV_HEADS, OPT_GEMM, OPT_GEMM_TILE,
 OPT_LN_SEG, OPT_FUSE_RES, OPT_FUSE_MLP, OPT_QKV_KBLOCK) = range(10)
OPTIONS = {"parts": OPT_PARTS, "pass_tokens": OPT_PASS_TOKENS, "qkv_fused": OPT_QKV_FUSED,
           "qkv_heads": OPT_QKV_HEADS, "gemm": OPT_GEMM, "gemm_tile": OPT_GEMM_TILE,
           "ln_seg": OPT_LN_SEG, "fuse_res": OPT_FUSE_RES, "fuse_mlp": OPT_FUSE_MLP,
           "qkv_kblock": OPT_QKV_KBLOCK}


class IxhError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


class IxhKernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("launches", C.c_int64), ("ms", C.c_double),
                ("ops", C.c_double), ("bytes", C.c_double)]


class IxhConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_int), ("layers", C.c_int), ("heads", C.c_int),
        ("intermediate", C.c_int), ("vocab", C.c_int), ("norm_eps", C.c_double),
        ("global_every", C.c_int), ("local_attention", C.c_int),
        ("global_theta", C.c_double), ("local_theta", C.c_double),
        ("pooling", C.c_int), ("lanes", C.c_int),
    ]


_lib = None
vp = C.c_void_p


def lib():
    """Loads the library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(SO_PATH):
        raise RuntimeError(
            f"indecis_amd: {SO_PATH} is missing; run __graft_entry__.build() "
            "(the HIP path has no CPU fallback)")
    L = C.CDLL(SO_PATH)
    L.ixh_last_error.restype = C.c_char_p
    L.ixh_last_error.argtypes = []
    sig = {
        "ixh_device_count": [C.POINTER(C.c_int)],
        "ixh_model_create": [C.POINTER(IxhConfig), C.c_int, C.POINTER(vp)],
        "ixh_model_set_matrix": [vp, C.c_int, C.c_int, vp, vp, C.c_int],
        "ixh_model_set_norm": [vp, C.c_int, C.c_int, vp],
        "ixh_model_set_embeddings_f32": [vp, vp],
        "ixh_model_set_embeddings_bf16": [vp, vp, vp, vp, C.c_int],
        "ixh_model_set_embeddings_i8": [vp, vp, vp],
        "ixh_model_set_rope": [vp, C.c_int, vp, vp, C.c_int],
        "ixh_model_invalidate": [vp],
        "ixh_encode_seqs": [vp, vp, vp, C.c_int, vp],
        "ixh_encode_tokens": [vp, vp, vp, C.c_int, vp],
        "ixh_encode_device": [vp, vp, vp, C.c_int, C.c_int, vp, vp],
        "ixh_head_logits": [vp, vp, C.c_int, vp, vp, C.c_int, vp],
        "ixh_packb8_create": [C.c_int, vp, vp, C.c_int, C.c_int, C.c_int, C.POINTER(vp)],
        "ixh_matmul8": [vp, vp, vp, C.c_int, C.c_int],
        "ixh_matmul8_outliers": [vp, vp, vp, C.c_int, C.c_int, C.c_float],
        "ixh_model_load_safetensors": [vp, C.c_char_p],
        "ixh_tokenizer_load": [C.c_char_p, C.POINTER(vp)],
        "ixh_tokenizer_info": [vp, vp, vp, vp, vp],
        "ixh_tokenizer_encode": [vp, C.c_char_p, C.c_int64, C.c_int, vp, C.c_int64, C.POINTER(C.c_int64)],
        "ixh_tokenizer_encode_pair": [vp, C.c_char_p, C.c_int64, C.c_char_p, C.c_int64, C.c_int, vp, C.c_int64,
                                      C.POINTER(C.c_int64)],
        "ixh_tokenizer_encode_offsets": [vp, C.c_char_p, C.c_int64, vp, vp, vp, C.c_int64, C.POINTER(C.c_int64)],
        "ixh_tokenizer_encode_batch": [vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_int64, vp],
        "ixh_embed_texts": [vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp],
        "ixh_embed_normalize": [vp, C.c_int, C.c_int],
        "ixh_safetensors_tensor": [C.c_char_p, C.c_char_p, vp, C.c_int64, C.POINTER(C.c_int64)],
        "ixh_linear8": [vp, vp, vp, C.c_int, vp, C.c_int, C.c_float],
        "ixh_matmul8_tile": [vp, vp, C.c_int, vp, vp, vp],
        "ixh_layernorm_quant": [C.c_int, vp, C.c_int, C.c_int, vp, C.c_double, C.c_int, vp, vp, vp],
        "ixh_ln_matmul8_geglu": [vp, vp, C.c_int, vp, C.c_double, C.c_int, vp, vp],
        "ixh_attend8": [C.c_int, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int],
        "ixh_model_set_profiling": [vp, C.c_int],
        "ixh_model_set_profile_filter": [vp, C.c_char_p],
        "ixh_model_profile": [vp, C.POINTER(IxhKernelStat), C.c_int, C.POINTER(C.c_int)],
        "ixh_check_exp255": [C.c_int, C.POINTER(C.c_int64), C.POINTER(C.c_float),
                             C.POINTER(C.c_int64)],
        "ixh_check_gelu": [C.c_int, C.POINTER(C.c_int64)],
        "ixh_check_mfma_rate": [C.c_int, C.c_int, C.POINTER(C.c_double)],
        "ixh_batcher_create": [vp, C.c_int, C.c_int, C.POINTER(vp)],
        "ixh_batcher_encode": [vp, vp, vp, C.c_int, vp],
        "ixh_batcher_stats": [vp, C.POINTER(C.c_int64), C.POINTER(C.c_int64)],
        "ixh_model_set_option": [vp, C.c_int, C.c_int64],
        "ixh_model_get_option": [vp, C.c_int, C.POINTER(C.c_int64)],
        "ixh_packb8_set_option": [vp, C.c_int, C.c_int64],
        "ixh_model_set_heads": [vp, C.c_int, vp, vp, vp, vp],
        "ixh_encode_heads": [vp, vp, vp, C.c_int, C.c_int, vp, vp],
        "ixh_matmul8_noalloc": [vp, vp, C.c_int, vp, C.c_int, C.c_int, C.c_int, vp],
    }
    for name, args in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = C.c_int
    L.ixh_model_destroy.argtypes = [vp]
    L.ixh_model_destroy.restype = None
    L.ixh_packb8_destroy.argtypes = [vp]
    L.ixh_packb8_destroy.restype = None
    L.ixh_batcher_destroy.argtypes = [vp]
    L.ixh_batcher_destroy.restype = None
    L.ixh_tokenizer_destroy.argtypes = [vp]
    L.ixh_tokenizer_destroy.restype = None
    _lib = L
    return L


def check(rc):
    """Raises IxhError with the library's message for a nonzero code."""
    if rc != IXH_OK:
        msg = lib().ixh_last_error().decode(errors="replace")
        raise IxhError(rc, msg)


def device_count():
    n = C.c_int(0)
    check(lib().ixh_device_count(C.byref(n)))
    return n.value
