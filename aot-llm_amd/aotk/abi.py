"""ctypes mirror of include/aotk.h and the loader of the in-tree libaotk.so.

The structs are byte-compatible with the C header; the loader fails loudly
when the HIP library has not been built (there is no CPU fallback).
"""
import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libaotk.so")

# enum aotk_kind (quant.rs:35-87)
F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = range(9)
NONE = -1
KIND_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", Q4_0: "q4_0", Q5_0: "q5_0",
              Q8_0: "q8_0", Q4_K: "q4_K", Q5_K: "q5_K", Q6_K: "q6_K"}
KIND_BY_NAME = {v.lower(): k for k, v in KIND_NAMES.items()}
BLOCK = {F32: 1, F16: 1, BF16: 1, Q4_0: 32, Q5_0: 32, Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
TYPE_SIZE = {F32: 4, F16: 2, BF16: 2, Q4_0: 18, Q5_0: 22, Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}


def row_bytes(kind, cols):
    """quant.rs:70-73 `Kind::row_bytes`."""
    return cols // BLOCK[kind] * TYPE_SIZE[kind]


def activation(kind):
    """model.rs:85-91: 0 = f32 input, 1 = Q8_0 blocks, 2 = Q8_K blocks."""
    if kind in (Q4_0, Q5_0, Q8_0):
        return 1
    if kind in (Q4_K, Q5_K, Q6_K):
        return 2
    return 0


def act_bytes(kind, cols):
    """Bytes of one quantized input vector for a matrix of `kind`."""
    a = activation(kind)
    if a == 1:
        return cols // 32 * 36
    if a == 2:
        return cols // 256 * 292
    return cols * 4


class Tensor(C.Structure):
    _fields_ = [("kind", C.c_int32), ("reserved", C.c_int32), ("off", C.c_uint64),
                ("len", C.c_uint64), ("rows", C.c_uint64), ("cols", C.c_uint64)]


class Dims(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("dim", "hidden", "n_layer", "n_head", "n_kv_head",
                                          "head_dim", "rot_dim", "vocab", "n_ctx_train")] + [
        ("eps", C.c_float), ("rope_base", C.c_float), ("rope_scale", C.c_float),
        ("swa_window", C.c_uint32), ("rope_base_local", C.c_float), ("rope_scale_local", C.c_float)]


class Flags(C.Structure):
    _fields_ = [(n, C.c_uint8) for n in ("rope_neox", "qkv_bias", "qk_norm", "embd_scale",
                                         "post_norms", "gelu")] + [
        ("reserved", C.c_uint8 * 2), ("swa_pattern", C.c_uint32)]


LAYER_SLOTS = ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "gate", "up", "down",
               "bq", "bk", "bv", "q_norm", "k_norm", "attn_post_norm", "ffn_post_norm")


class Layer(C.Structure):
    _fields_ = [(n, Tensor) for n in LAYER_SLOTS] + [("local_attn", C.c_int32), ("reserved", C.c_int32)]


class ModelSpec(C.Structure):
    _fields_ = [("dims", Dims), ("flags", Flags), ("token_embd", Tensor), ("output_norm", Tensor),
                ("output", Tensor), ("rope_freqs", Tensor), ("layers", C.POINTER(Layer))]


class SamplerConfig(C.Structure):
    """aotk_sampler_config (sampler.rs SamplerConfig)."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("repeat_penalty", C.c_float),
                ("repeat_last_n", C.c_uint32), ("reserved", C.c_uint32), ("seed", C.c_uint64)]


assert C.sizeof(Tensor) == 40
assert C.sizeof(Layer) == 16 * 40 + 8


class AotkError(RuntimeError):
    pass


_lib = None


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args
    return f


def load(path=None):
    """Load libaotk.so (built by aot-llm_amd/build.py). Raises when missing."""
    global _lib
    if _lib is not None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise AotkError(f"{p} is missing: build the HIP library first (python aot-llm_amd/build.py)")
    lib = C.CDLL(p)
    vp, sz, i, u32, u64, fp = C.c_void_p, C.c_size_t, C.c_int, C.c_uint32, C.c_uint64, C.POINTER(C.c_float)
    _sig(lib, "aotk_last_error", C.c_char_p, [])
    _sig(lib, "aotk_init", i, [i])
    _sig(lib, "aotk_dev_alloc", vp, [sz])
    _sig(lib, "aotk_dev_free", i, [vp])
    _sig(lib, "aotk_h2d", i, [vp, vp, sz])
    _sig(lib, "aotk_d2h", i, [vp, vp, sz])
    _sig(lib, "aotk_memset", i, [vp, i, sz])
    _sig(lib, "aotk_d2d", i, [vp, vp, sz])
    _sig(lib, "aotk_sync", i, [])
    _sig(lib, "aotk_row_bytes", sz, [i, sz])
    _sig(lib, "aotk_weight_upload", vp, [i, vp, sz, sz])
    _sig(lib, "aotk_weight_from_dev", vp, [i, vp, sz, sz])
    _sig(lib, "aotk_weight_free", i, [vp])
    _sig(lib, "aotk_dequant_rows", i, [vp, sz, sz, vp])
    _sig(lib, "aotk_quantize_rows", i, [i, vp, sz, sz, vp])
    _sig(lib, "aotk_quantize_q8_0", i, [vp, sz, vp])
    _sig(lib, "aotk_quantize_q8_k", i, [vp, sz, vp])
    _sig(lib, "aotk_matvec", i, [vp, vp, vp])
    _sig(lib, "aotk_matvec_f32", i, [vp, vp, vp])
    _sig(lib, "aotk_matmul", i, [vp, vp, sz, vp])
    _sig(lib, "aotk_matmul_noalloc", i, [vp, vp, sz, vp])
    _sig(lib, "aotk_matvec3", i, [C.POINTER(vp), vp, C.POINTER(vp)])
    _sig(lib, "aotk_matvec2", i, [vp, vp, vp, vp, vp])
    _sig(lib, "aotk_matmul2", i, [vp, vp, vp, sz, vp, vp])
    _sig(lib, "aotk_rmsnorm", i, [vp, vp, vp, sz, sz, C.c_float])
    _sig(lib, "aotk_rmsnorm_heads", i, [vp, vp, sz, sz, C.c_float])
    _sig(lib, "aotk_rope", i, [vp, sz, sz, sz, sz, vp, i])
    _sig(lib, "aotk_softmax", i, [vp, sz])
    _sig(lib, "aotk_silu_mul", i, [vp, vp, sz])
    _sig(lib, "aotk_gelu_mul", i, [vp, vp, sz])
    _sig(lib, "aotk_add", i, [vp, vp, sz])
    _sig(lib, "aotk_attention", i, [vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, sz, sz])
    _sig(lib, "aotk_argmax", i, [vp, sz, C.POINTER(u32)])
    _sig(lib, "aotk_model_load", vp, [C.POINTER(ModelSpec), vp, sz])
    _sig(lib, "aotk_model_synthetic", vp, [C.POINTER(ModelSpec), u64])
    _sig(lib, "aotk_model_download", i, [vp, vp, sz])
    _sig(lib, "aotk_model_free", i, [vp])
    _sig(lib, "aotk_model_weight_bytes", u64, [vp])
    _sig(lib, "aotk_state_new", vp, [vp, sz, sz])
    _sig(lib, "aotk_state_free", i, [vp])
    _sig(lib, "aotk_forward", i, [vp, u32, sz, i])
    _sig(lib, "aotk_forward_batch", i, [vp, C.POINTER(u32), sz, sz, i])
    _sig(lib, "aotk_logits", i, [vp, fp])
    _sig(lib, "aotk_greedy", i, [vp, C.POINTER(u32)])
    _sig(lib, "aotk_generate_greedy", i, [vp, sz, sz, C.POINTER(u32)])
    _sig(lib, "aotk_kv_download", i, [vp, sz, fp, fp])
    _sig(lib, "aotk_kv_upload", i, [vp, sz, fp, fp])
    _sig(lib, "aotk_sampler_new", vp, [C.POINTER(SamplerConfig)])
    _sig(lib, "aotk_sampler_free", i, [vp])
    _sig(lib, "aotk_set_logits", i, [vp, fp])
    _sig(lib, "aotk_sample", i, [vp, vp, C.POINTER(u32), sz, C.POINTER(u32)])
    _sig(lib, "aotk_generate", i, [vp, vp, sz, sz, C.POINTER(u32), sz, C.POINTER(u32)])
    _sig(lib, "aotk_prefix_save", i, [vp, C.POINTER(u32), sz, sz, vp, sz, C.POINTER(sz)])
    _sig(lib, "aotk_prefix_load", i, [vp, vp, sz, C.POINTER(u32), sz, C.POINTER(sz), C.POINTER(sz)])
    _sig(lib, "aotk_stream", vp, [])
    _sig(lib, "aotk_time_matvec", i, [C.POINTER(vp), sz, vp, sz, C.POINTER(C.c_float)])
    _sig(lib, "aotk_time_hbm", i, [C.c_int, C.c_int, C.POINTER(vp), sz, sz, sz, C.POINTER(C.c_float)])
    _sig(lib, "aotk_time_matmul", i, [C.POINTER(vp), sz, vp, sz, sz, C.POINTER(C.c_float)])
    _lib = lib
    return lib


def check(rc):
    """Raise AotkError with aotk_last_error() for a failed call."""
    if rc is None or (isinstance(rc, int) and rc != 0 and rc is not True):
        msg = _lib.aotk_last_error() if _lib is not None else b"library not loaded"
        raise AotkError((msg or b"unknown error").decode())
    return rc


def check_ptr(p):
    if not p:
        msg = _lib.aotk_last_error() if _lib is not None else b"library not loaded"
        raise AotkError((msg or b"unknown error").decode())
    return p
