"""ctypes binding of liblaya_hip.so (declarations in include/laya_hip.h).

The shared library is built in-tree (``make -C laya-cuda_amd/csrc``) and loaded from this
package's directory.  There is no fallback: a missing library raises at first use.
"""
import ctypes as ct
from pathlib import Path

LIBRARY = Path(__file__).with_name("liblaya_hip.so")

OK, EINVAL, EDEVICE, ENOMEM, ESTATE = range(5)
ABI_VERSION = 2  # LAYA_ABI_VERSION of the struct layouts mirrored below
F32, F16, BF16 = 0, 1, 2
NORM_POST, NORM_PRE = 0, 1
POS_LEARNED, POS_ROPE = 0, 1
FFN_GELU, FFN_GEGLU = 0, 1


class LayaConfig(ct.Structure):
    _fields_ = [(name, ct.c_float if name in ("eps", "theta_global", "theta_local") else ct.c_int32) for name in (
        "width", "heads", "layers", "intermediate", "vocab", "max_positions", "type_vocab",
        "norm_order", "pos_kind", "ffn_kind", "bias", "eps", "window", "global_every",
        "head_layers", "n_act", "act_hidden", "max_len", "mfma_dtype", "theta_global", "theta_local")]


class LayaShape(ct.Structure):
    _fields_ = [("rows", ct.c_int32), ("batch", ct.c_int32), ("options", ct.c_int32)]


class LayaMetrics(ct.Structure):
    _fields_ = [("gpu_ms", ct.c_float), ("cache_miss", ct.c_int32), ("graph_capture", ct.c_int32),
                ("graph_replay", ct.c_int32), ("owned_gpu_bytes", ct.c_int64)]


class LayaDevice(ct.Structure):
    _fields_ = [("name", ct.c_char * 256), ("arch", ct.c_char * 64), ("hbm_bytes", ct.c_int64),
                ("free_bytes", ct.c_int64), ("compute_units", ct.c_int32), ("lds_bytes_per_cu", ct.c_int32),
                ("clock_khz", ct.c_int32), ("supported", ct.c_int32)]


_p, _i, _f, _i64 = ct.c_void_p, ct.c_int, ct.c_float, ct.c_int64
_ip = ct.POINTER(ct.c_int32)
_fp = ct.POINTER(ct.c_float)

SIGNATURES = {
    "laya_abi_version": ([], _i),
    "laya_packed_ints": ([ct.POINTER(LayaShape)], _i64),
    "laya_device_count": ([ct.POINTER(ct.c_int)], _i),
    "laya_device_info": ([_i, ct.POINTER(LayaDevice)], _i),
    "laya_create": ([ct.POINTER(LayaConfig), _i, _i, ct.POINTER(_p)], _i),
    "laya_load_weight": ([_p, ct.c_char_p, _p, _i, ct.POINTER(_i64), _i], _i),
    "laya_finalize": ([_p], _i),
    "laya_predict": ([_p, _ip, ct.POINTER(LayaShape), _i, _fp, _fp, ct.POINTER(LayaMetrics)], _i),
    "laya_predict_static": ([_p, _ip, ct.POINTER(LayaShape), _fp, _fp, ct.POINTER(LayaMetrics)], _i),
    "laya_stage_count": ([], _i),
    "laya_stage_name": ([_i], ct.c_char_p),
    "laya_time_stage": ([_p, _ip, ct.POINTER(LayaShape), _i, _i, _i, _fp], _i),
    "laya_stage_launches": ([_p, _i, ct.POINTER(ct.c_int32), ct.POINTER(ct.c_int32)], _i),
    "laya_read_weight": ([_p, ct.c_char_p, _fp, _i64], _i),
    "laya_used_bytes": ([_p], _i64),
    "laya_slot_count": ([_p], _i),
    "laya_destroy": ([_p], _i),
    "laya_last_error": ([_p], ct.c_char_p),
    "laya_attention_tiles": ([_ip, _ip, _i, _i, _i, _ip, _i], _i),
    "laya_attention_block": ([_i, _i], _i),
    "laya_op_embed": ([_p, _p, _p, _p, _p, _p, _p, _f, _p, _p, _i, _i, _i, _i, _i, _p], _i),
    "laya_op_norm": ([_p, _p, _i, _i64, _p, _p, _p, _f, _p, _p, _p, _i, _i, _i, _p], _i),
    "laya_op_linear": ([_p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p], _i),
    "laya_op_qkv": ([_p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p], _i),
    "laya_op_attention": ([_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p], _i),
    "laya_op_gather_rows": ([_p, _p, _p, _p, _i, _p, _p, _i, _i, _p], _i),
    "laya_op_head_gather": ([_p, _p, _p, _p, _p, _p, _p, _p, _f, _p, _p, _i, _i, _p], _i),
}

_lib = None


def load():
    """Load and type the library once; raises if it was not built."""
    global _lib
    if _lib is None:
        if not LIBRARY.is_file():
            raise RuntimeError(f"{LIBRARY} is missing; build it with `make -C laya-cuda_amd/csrc` "
                               "(or __graft_entry__.build()).  There is no CPU fallback.")
        lib = ct.CDLL(str(LIBRARY))
        # The version first: a library of another ABI may lack or rename the other exports.
        version = getattr(lib, "laya_abi_version", None)
        if version is None:
            raise RuntimeError(f"{LIBRARY} exports no laya_abi_version; rebuild the library")
        version.argtypes, version.restype = [], ct.c_int
        if version() != ABI_VERSION:
            raise RuntimeError(f"{LIBRARY} has ABI version {version()}, this binding "
                               f"mirrors version {ABI_VERSION}; rebuild the library")
        for name, (args, ret) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, ret
        _lib = lib
    return _lib


def error(handle=None):
    message = load().laya_last_error(handle)
    return message.decode() if message else "unknown error"


def check(code, handle=None):
    if code != OK:
        raise RuntimeError(f"liblaya_hip: {error(handle)}")
