"""ctypes binding of libcoopt_amd.so (the C ABI declared in include/coopt_amd.h).

The library must be loaded after `import torch`: torch ships its own libamdhip64.so, and a
library whose NEEDED entry names the same soname then binds to that already-loaded runtime,
so stream handles and device pointers from torch are valid inside the kernels.  There is no
CPU fallback: if the library is missing or its HIP runtime differs from torch's, every entry
point raises.
"""
import ctypes
import os
import re
import threading

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcoopt_amd.so")

COOPT_OK, COOPT_EINVAL, COOPT_EHIP, COOPT_EWORKSPACE = 0, -1, -2, -3
DT_F32, DT_BF16, DT_F16, DT_I8 = 0, 1, 2, 3

_i, _i64, _f, _p, _sz = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# (name, restype, argtypes) for every symbol of include/coopt_amd.h
SIGNATURES = {
    "coopt_last_error": (ctypes.c_char_p, []),
    "coopt_hip_runtime_version": (_i, [ctypes.POINTER(_i)]),
    "coopt_kv_write": (_i, [_i, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p,
                            _i64, _i64, _i64, _p, _i, _i, _i, _i, _i64, _p]),
    "coopt_quantize": (_i, [_i, _i, _p, _i64, _i, _p, _p, _p]),
    "coopt_kv_swap_out": (_i, [_i, _i, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i, _i, _i,
                               _i, _i64, _p, _p, _p]),
    "coopt_kv_swap_in": (_i, [_i, _i, _p, _p, _p, _i, _i, _i, _i, _i64, _p, _i64, _i64, _i64, _p,
                              _i64, _i64, _i64, _p]),
    "coopt_kv_swap_out_caches": (_i, [_i, _i, _i, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p,
                                      _i, _i, _i, _i, _i64, _p, _p, _p]),
    "coopt_kv_swap_in_caches": (_i, [_i, _i, _i, _p, _p, _p, _i, _i, _i, _i, _i64, _p, _p, _i64,
                                     _i64, _i64, _i64, _i64, _i64, _p]),
    "coopt_dequantize": (_i, [_i, _p, _p, _i64, _i, _i, _p, _p]),
    "coopt_kv_copy_blocks": (_i, [_p, _i, _p, _p, _i, _i64, _p]),
    "coopt_linear_workspace": (_sz, [_i, _i, _i]),
    "coopt_linear": (_i, [_p, _i64, _p, _i64, _i, _i, _i, _p, _i64, _p, _sz, _p]),
    "coopt_linear_split": (_i, [_i, _i, _i, _p, _p]),
    "coopt_linear_partials": (_i, [_p, _i64, _p, _i64, _i, _i, _i, _p, _sz, _p]),
    "coopt_linear_pack_weight": (_i, [_p, _i64, _i, _i, _p, _p]),
    "coopt_row_slots": (_i, [_p, _i64, _i, _p, _p, _i, _i, _i, _p, _p, _p, _p]),
    "coopt_spec_step_begin": (_i, [_p, _i64, _i, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i, _i,
                                   _i, _i, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p]),
    "coopt_spec_step_verify_tokens": (_i, [_p, _i64, _i, _i, _p, _p, _p]),
    "coopt_spec_step_commit": (_i, [_p, _p, _p, _i, _p, _p, _p, _p, _p, _i64, _i64, _p, _p, _p, _i,
                                    _p]),
    "coopt_linear_pack_gate_up": (_i, [_p, _i64, _i, _i, _p, _p]),
    "coopt_linear_silu_supported": (_i, [_i, _i, _i]),
    "coopt_linear_silu_packed": (_i, [_p, _i64, _p, _i, _i, _i, _p, _i64, _p]),
    "coopt_linear_packed": (_i, [_p, _i64, _p, _i, _i, _i, _p, _i64, _p, _sz, _p]),
    "coopt_linear_partials_packed": (_i, [_p, _i64, _p, _i, _i, _i, _p, _sz, _p]),
    "coopt_rms_norm_partials": (_i, [_p, _i, _i64, _p, _p, _p, _i64, _i, _f, _p]),
    "coopt_silu_mul_partials": (_i, [_p, _i, _i64, _p, _i64, _i, _p]),
    "coopt_qkv_epilogue": (_i, [_i, _p, _i64, _p, _i, _i64, _p, _p, _p, _i64, _i, _p, _i64, _i64,
                                _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i, _i, _i,
                                _i, _i, _i64, _p]),
    "coopt_verify_attention_workspace": (_sz, [_i, _i, _i, _i, _i, _i]),
    "coopt_verify_attention_qkv_supported": (_i, [_i, _i, _i, _i, _i, _i, _i]),
    "coopt_verify_attention_qkv": (_i, [_i, _p, _i64, _p, _i, _i64, _p, _p, _p, _i64, _i, _p,
                                        _p, _p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64,
                                        _p, _i64, _p, _p, _i, _i, _i, _i, _i, _i64, _i, _i, _f,
                                        _p, _i64, _i64, _p, _sz, _p]),
    "coopt_verify_attention": (_i, [_i, _p, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _p, _i64,
                                    _i64, _i64, _p, _i64, _p, _p, _i, _i, _i, _i, _i, _i64, _i,
                                    _i, _f, _p, _i64, _i64, _p, _sz, _p]),
    "coopt_accept_sample_workspace": (_sz, [_i, _i, _i]),
    "coopt_accept_sample": (_i, [_i, _p, _i64, _p, _i, _p, _i64, _p, _p, _p, _p, _p, _f, _i, _i,
                                 _i, _p, _p, _p, _p, _sz, _p]),
    "coopt_accept_sample_noalloc_max_bytes": (_sz, []),
    "coopt_accept_sample_noalloc": (_i, [_i, _p, _i64, _p, _i, _p, _i64, _p, _p, _p, _p, _p, _f,
                                         _i, _i, _i, _p, _p, _p, _p]),
    "coopt_softmax": (_i, [_i, _p, _i64, _i64, _i, _f, _p, _i64, _p]),
    "coopt_sample_probs": (_i, [_i, _p, _i64, _i, _i, _f, _p, _sz, _p, _i64, _p]),
    "coopt_sample": (_i, [_i, _p, _i64, _i, _i, _f, _p, _p, _p, _p, _i64, _p, _sz, _p]),
    "coopt_rms_norm": (_i, [_p, _p, _p, _p, _i64, _i, _f, _p]),
    "coopt_rope": (_i, [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _p, _i64, _i, _i, _i, _i, _i, _p]),
    "coopt_silu_mul": (_i, [_p, _p, _i64, _i, _p]),
}

_lock = threading.Lock()
_lib = None


class CooptError(RuntimeError):
    """A libcoopt_amd.so entry point returned an error code."""


def _hip_libs_mapped():
    try:
        maps = open("/proc/self/maps").read()
    except OSError:
        return []
    return sorted(set(re.findall(r"\S*libamdhip64\.so\S*", maps)))


def load(path: str = LIB_PATH):
    """Loads (once) and returns the ctypes handle; raises if the library is unusable."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise CooptError(
                f"{path} is missing: build it with __graft_entry__.build() "
                "(python -m iitj_llm_coopt_amd.build). There is no CPU fallback.")
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        hip = _hip_libs_mapped()
        if len(hip) > 1:
            raise CooptError(f"two HIP runtimes are mapped ({hip}); libcoopt_amd.so must bind "
                             "to torch's: import torch before loading it")
        _lib = lib
        return lib


def last_error() -> str:
    return load().coopt_last_error().decode(errors="replace")


def check(rc: int, what: str):
    if rc != COOPT_OK:
        raise CooptError(f"{what} failed ({rc}): {last_error()}")


def runtime_version() -> int:
    v = ctypes.c_int(0)
    check(load().coopt_hip_runtime_version(ctypes.byref(v)), "coopt_hip_runtime_version")
    return v.value


def stream_handle(device=None) -> int:
    """hipStream_t of torch's current stream on `device` (the stream every call uses)."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


_DT = {torch.float32: DT_F32, torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.int8: DT_I8}


def dt_code(dtype) -> int:
    try:
        return _DT[dtype]
    except KeyError:
        raise CooptError(f"unsupported dtype {dtype}") from None


def require_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise CooptError("libcoopt_amd.so kernels take device tensors; got a CPU tensor "
                             "(there is no CPU fallback)")


class WorkspaceCache:
    """Device scratch buffers, grown on demand and reused (the kernels need no initialised
    workspace).  One buffer per (device, stream): calls that overlap in time must not share
    a workspace, and stream order keeps calls on one stream from overlapping.  An outgrown
    buffer is kept alive, not freed: a HIP graph captured with it keeps its address."""

    def __init__(self):
        self._bufs = {}
        self._retired = []

    def get(self, nbytes: int, device) -> torch.Tensor:
        dev = torch.device(device)
        key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
        buf = self._bufs.get(key)
        if buf is None or buf.numel() < nbytes:
            if buf is not None:
                self._retired.append(buf)
            buf = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=dev)
            self._bufs[key] = buf
        return buf
