"""ctypes binding of libpk_gpu.so (include/pk_gpu.h) for Python callers.

The library is C; this module only declares argument types and turns error
codes into exceptions.  Device memory and streams may come from PyTorch
(tensor.data_ptr(), torch.cuda.current_stream().cuda_stream); host-pointer
calls take numpy arrays.  Importing this module never falls back to the CPU:
if the shared library is missing, load() raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
# PK_GPU_LIB selects another build of the library (e.g. to compare two builds).
LIB_PATH = os.environ.get("PK_GPU_LIB") or os.path.join(LIB_DIR, "libpk_gpu.so")
SHIM_PATH = os.path.join(LIB_DIR, "libpk_gpu_cblas.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "pk_gpu.h")

NOTRANS = 111

_i, _f, _p = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
_ll, _sz = ctypes.c_longlong, ctypes.c_size_t

_PROTOS = {
    "pk_gpu_init": (_i, [_i]),
    "pk_gpu_shutdown": (None, []),
    "pk_gpu_last_error": (ctypes.c_char_p, []),
    "pk_gpu_register_weight": (_i, [_p, _sz]),
    "pk_gpu_unregister_weight": (_i, [_p]),
    "pk_gpu_device_ptr": (_p, [_p]),
    "pk_gpu_resident_bytes": (_sz, []),
    "pk_gpu_gemm_i8": (_i, [_i, _i, _i, _f, _p, _i, _p, _f, _i, _f, _p, _i]),
    "pk_gpu_gemm_i8_noalloc": (_i, [_i, _i, _i, _f, _p, _i, _p, _f, _i, _f, _p, _i, _p]),
    "pk_gpu_gemm_i4": (_i, [_i, _i, _i, _f, _p, _i, _p, _p, _i, _f, _p, _i]),
    "pk_gpu_sgemm": (_i, [_i, _i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i]),
    "pk_gpu_gemm_i8_dev": (_i, [_i, _i, _i, _f, _p, _i, _p, _f, _i, _f, _p, _i, _p]),
    "pk_gpu_gemm_i4_dev": (_i, [_i, _i, _i, _f, _p, _i, _p, _p, _i, _f, _p, _i, _p]),
    "pk_gpu_sgemm_dev": (_i, [_i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i, _p]),
    "pk_gpu_gemm_i8_ex_dev": (_i, [_i, _i, _i, _f, _p, _i, _p, _f, _i, _f, _p, _i, _p, _i, _p]),
    "pk_gpu_gemm_i4_ex_dev": (_i, [_i, _i, _i, _f, _p, _i, _p, _p, _i, _f, _p, _i, _p, _i, _p]),
    "pk_gpu_sgemm_ex_dev": (_i, [_i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i, _p, _i, _p]),
    "pk_gpu_swish_dev": (_i, [_p, _p, _ll, _p]),
    "pk_gpu_num_configs": (_i, []),
    "pk_gpu_config_info": (_i, [_i, _p, _p, _p, _p, _p, _p]),
    "pk_gpu_pick_config": (_i, [_i, _i, _i]),
    "pk_gpu_pick_config_bits": (_i, [_i, _i, _i, _i]),
    "pk_gpu_force_config": (_i, [_i]),
    "pk_gpu_set_numerics": (_i, [_i]),
    "pk_gpu_get_numerics": (_i, []),
    "pk_gpu_uses_small_m": (_i, [_i, _i, _i, _i]),
    "pk_gpu_uses_split": (_i, [_i, _i, _i, _i]),
    "pk_gpu_set_workspace": (_i, [_p, _sz]),
    "pk_gpu_split_k_segments": (_i, [_i, _i, _i, _i]),
    "pk_gpu_force_small_tile": (_i, [_i, _i]),
    "pk_gpu_pack_weight_dev": (_i, [_i, _i, _i, _p, _i, _p, _p]),
    "pk_gpu_unpack_weight_dev": (_i, [_p]),
    "pk_gpu_panel_bytes": (_sz, []),
    "pk_gpu_presplit_weight_dev": (_i, [_i, _i, _i, _p, _i, _p, _p]),
    "pk_gpu_unsplit_weight_dev": (_i, [_p]),
    "pk_gpu_presplit_bytes": (_sz, []),
    "pk_gpu_uses_panel": (_i, [_i, _i, _i, _i, _p, _i, _p]),
    "pk_gpu_panel_segments": (_i, [_i, _i, _i]),
    "pk_gpu_panel_decode_dev": (_i, [_i, _i, _i, _p, _i, _p, _f, _p, _p]),
    "pk_gpu_force_panel_tile": (_i, [_i, _i]),
    "pk_gpu_dequant_dev": (_i, [_i, _i, _i, _p, _i, _f, _p, _i, _p, _p]),
    "pk_gpu_layer_norm_dev": (_i, [_p, _p, _p, _p, _i, _i, _p]),
    "pk_gpu_attention_dev": (_i, [_p, _i, _p, _i, _p, _p, _p, _i, _i, _i, _p]),
    "pk_gpu_attention_ws_floats": (ctypes.c_size_t, [_i, _i]),
    "pk_gpu_attention_ws_dev": (_i, [_p, _i, _p, _i, _p, _p, _p, _i, _i, _i, _p, ctypes.c_size_t, _p]),
    "pk_gpu_glu_dev": (_i, [_p, _p, _i, _i, _p]),
    "pk_gpu_depthwise_dev": (_i, [_p, _i, _p, _p, _p, _i, _i, _i, _i, _i, _p]),
    "pk_gpu_encoder_create": (_i, [_p, _p, _i, _p, _i, _i]),
    "pk_gpu_encoder_run": (_i, [_p, _p, _i, _i, _i, _p]),
    "pk_gpu_encoder_run_dev": (_i, [_p, _p, _i, _i, _i, _p, _p]),
    "pk_gpu_encoder_bytes": (_sz, [_p]),
    "pk_gpu_encoder_destroy": (None, [_p]),
    "pk_gpu_encoder_profile": (_i, [_p, _i]),
    "pk_gpu_encoder_set_groups": (_i, [_p, _i]),
    "pk_gpu_encoder_set_group_lag": (_i, [_p, _i]),
    "pk_gpu_encoder_set_numerics": (_i, [_p, _i]),
    "pk_gpu_encoder_get_numerics": (_i, [_p]),
    "pk_gpu_encoder_set_pre_encode": (_i, [_p, _p]),
    "pk_gpu_encoder_frames": (_i, [_i]),
    "pk_gpu_encoder_pre_encode_dev": (_i, [_p, _p, _i, _p, _p]),
    "pk_gpu_encoder_run_mel": (_i, [_p, _p, _i, _i, _i, _p]),
    "pk_gpu_encoder_profile_read": (_i, [_p, _i, _p, _p, _p, _p]),
}

EPI_NONE, EPI_SWISH, EPI_HALF_RESIDUAL, EPI_RESIDUAL = 0, 1, 2, 3
NUMERICS_DEFAULT, NUMERICS_EXACT, NUMERICS_FAST = 0, 1, 2
# PK_GPU_STAGE_*: pk_gpu_encoder_profile_read's stages
STAGE_GEMM_I4, STAGE_GEMM_I8, STAGE_GEMM_F32, STAGE_ATTENTION, STAGE_LAYER_NORM, STAGE_CONV, STAGE_COPY = range(7)
NOALLOC_BYTES = 64 << 20          # PK_GPU_NOALLOC_BYTES
SPLIT_WORKSPACE_BYTES = 32 << 20  # PK_GPU_SPLIT_WORKSPACE_BYTES


class Weight(ctypes.Structure):
    """pk_gpu_weight (include/pk_gpu.h; the reference's Weight, parakeet.h:42-57)."""
    _fields_ = [("data", _p), ("scale", _f), ("scales", _p), ("bits", _i)]


_BLOCK_FIELDS = [
    ("norm_ff1_w", _p), ("norm_ff1_b", _p),
    ("ff1_linear1_w", Weight), ("ff1_linear1_b", _p),
    ("ff1_linear2_w", Weight), ("ff1_linear2_b", _p),
    ("norm_sa_w", _p), ("norm_sa_b", _p),
    ("linear_qkv_w", Weight), ("linear_qkv_b", _p),
    ("linear_pos_w", Weight),
    ("linear_out_w", Weight), ("linear_out_b", _p),
    ("pos_bias_u", _p), ("pos_bias_v", _p),
    ("norm_conv_w", _p), ("norm_conv_b", _p),
    ("conv_pw1_w", _p), ("conv_pw1_b", _p),
    ("conv_dw_w", _p), ("conv_dw_b", _p),
    ("conv_pw2_w", _p), ("conv_pw2_b", _p),
    ("norm_ff2_w", _p), ("norm_ff2_b", _p),
    ("ff2_linear1_w", Weight), ("ff2_linear1_b", _p),
    ("ff2_linear2_w", Weight), ("ff2_linear2_b", _p),
    ("norm_out_w", _p), ("norm_out_b", _p),
]


class BlockWeights(ctypes.Structure):
    """pk_gpu_block_weights (include/pk_gpu.h): one conformer block, host pointers."""
    _fields_ = _BLOCK_FIELDS


class PreEncodeWeights(ctypes.Structure):
    """pk_gpu_pre_encode_weights (include/pk_gpu.h; PreEncodeWeights, parakeet.h)."""
    _fields_ = [("conv0_w", _p), ("conv0_b", _p), ("conv2_w", _p), ("conv2_b", _p),
                ("conv3_w", _p), ("conv3_b", _p), ("conv5_w", _p), ("conv5_b", _p),
                ("conv6_w", _p), ("conv6_b", _p), ("out_w", Weight), ("out_b", _p)]

STATUS = {0: "OK", -1: "EINVAL", -2: "ENOTSUP", -3: "ENOMEM", -4: "EHIP", -5: "ENODEV", -6: "EBUSY"}


class PkGpuError(RuntimeError):
    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} -> {STATUS.get(code, code)}: {msg}")
        self.code = code


_lib = None


def load():
    """Load libpk_gpu.so (raises if it was not built).

    PyTorch ships its own libamdhip64.so with the same SONAME as ROCm's
    (libamdhip64.so.7).  Importing torch first lets the library's HIP
    dependency bind to that copy, so the process holds one HIP runtime and
    torch's device pointers, streams and events are valid here; loading the
    library first would bring in a second runtime."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built; run __graft_entry__.build()")
        try:
            import torch  # noqa: F401  (one HIP runtime per process, see above)
        except ImportError:
            pass
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(fn_name, rc):
    if rc != 0:
        msg = load().pk_gpu_last_error()
        raise PkGpuError(fn_name, rc, msg.decode() if msg else "")
    return rc


def call(fn_name, *args):
    """Call an int-returning entry point and raise on a non-zero status."""
    return check(fn_name, getattr(load(), fn_name)(*args))


def configs():
    lib = load()
    out = []
    for i in range(lib.pk_gpu_num_configs()):
        v = [ctypes.c_int() for _ in range(6)]
        check("pk_gpu_config_info", lib.pk_gpu_config_info(i, *[ctypes.byref(x) for x in v]))
        fam, mf, cw, wgm, wgn, kt = (x.value for x in v)
        out.append((chr(fam), mf, cw, wgm, wgn, kt))
    return out


def header_functions(path=HEADER):
    """Function names declared in include/pk_gpu.h."""
    import re
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pk_gpu_\w+)\s*\(", text)))
