"""CPU: libcoopt_amd.so loads, binds torch's HIP runtime, exports every symbol of
include/coopt_amd.h, and rejects bad arguments with an error code + message before any launch.
No kernel is launched here."""
import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (must precede the library load)

from iitj_llm_coopt_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "coopt_amd.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(coopt_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_single_hip_runtime_is_mapped(lib):
    hip = _lib._hip_libs_mapped()
    assert len(hip) == 1 and "torch" in hip[0], hip


def test_runtime_version_matches_torch(lib):
    v = _lib.runtime_version()
    major, minor = v // 10000000, (v // 100000) % 100
    assert f"{major}.{minor}" == ".".join(torch.version.hip.split(".")[:2]), (v, torch.version.hip)


def test_workspace_sizes_are_positive_and_monotone(lib):
    a = lib.coopt_verify_attention_workspace(32, 32, 8, 128, 5, 4101)
    b = lib.coopt_verify_attention_workspace(64, 32, 8, 128, 9, 16393)
    assert 0 < a < b
    assert lib.coopt_verify_attention_workspace(0, 32, 8, 128, 5, 100) == 0
    c = lib.coopt_accept_sample_workspace(8, 4, 128256)
    d = lib.coopt_accept_sample_workspace(32, 4, 128256)
    assert 0 < c < d


def _err(rc):
    assert rc == _lib.COOPT_EINVAL, rc
    msg = _lib.last_error()
    assert msg
    return msg


def test_kv_write_rejects_bad_arguments(lib):
    msg = _err(lib.coopt_kv_write(99, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 8,
                                  128, 16, 16, None))
    assert "cache_dtype" in msg
    assert "D must be" in _err(lib.coopt_kv_write(_lib.DT_BF16, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                                                  0, 0, 0, 0, 0, 0, 1, 8, 96, 16, 16, None))
    assert "null" in _err(lib.coopt_kv_write(_lib.DT_BF16, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                                             0, 0, 0, 0, 1, 8, 128, 16, 16, None))
    # misaligned k/v rows (pointer not 16-byte aligned): rejected before launch
    assert "aligned" in _err(lib.coopt_kv_write(_lib.DT_BF16, 8, 8, 1024, 128, 1024, 128, 16, 16,
                                                0, 0, 0, 0, 0, 0, 0, 0, 16, 1, 8, 128, 16, 16,
                                                None))
    # T == 0 is a no-op
    assert lib.coopt_kv_write(_lib.DT_BF16, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                              8, 128, 16, 16, None) == 0


def test_verify_attention_rejects_unsupported_shapes(lib):
    args = dict(kv=_lib.DT_BF16, B=2, Hq=32, Hkv=8, D=128, bs=16, mq=5, mk=100, bt=16)

    def call(**kw):
        a = {**args, **kw}
        return lib.coopt_verify_attention(a["kv"], 16, 4096, 128, 16, 16, 0, 0, 0, 0, 0, 0, 0, 0,
                                          16, a["bt"], 16, 16, a["B"], a["Hq"], a["Hkv"], a["D"],
                                          a["bs"], 64, a["mq"], a["mk"], 0.088, 16, 4096, 128, 16,
                                          1 << 30, None)
    assert "head_dim" in _err(call(D=96))
    assert "multiple of Hkv" in _err(call(Hq=30))
    assert "<= 64" in _err(call(Hq=130, Hkv=2))   # more query heads per KV head than rows
    assert "power of two" in _err(call(bs=24))
    assert ">= 16" in _err(call(bs=8))
    assert "narrower" in _err(call(bt=3))
    assert "kv_dtype" in _err(call(kv=7))
    # INT8 without scales
    assert "scale" in _err(call(kv=_lib.DT_I8))


def test_verify_attention_reports_small_workspace(lib):
    rc = lib.coopt_verify_attention(_lib.DT_BF16, 16, 4096, 128, 16, 16, 0, 0, 0, 0, 0, 0, 0, 0,
                                    16, 16, 16, 16, 2, 32, 8, 128, 16, 64, 5, 100, 0.088, 16,
                                    4096, 128, 16, 8, None)
    assert rc == _lib.COOPT_EWORKSPACE and "workspace" in _lib.last_error()


def test_accept_sample_rejects_bad_arguments(lib):
    assert "logits_dtype" in _err(lib.coopt_accept_sample(5, 16, 100, 0, 0, 16, 100, 0, 16, 0,
                                                          16, 16, 1.0, 2, 4, 100, 16, 16, 0, 16,
                                                          1 << 20, None))
    assert "null" in _err(lib.coopt_accept_sample(_lib.DT_F32, 0, 100, 0, 0, 16, 100, 0, 16, 0,
                                                  16, 16, 1.0, 2, 4, 100, 16, 16, 0, 16, 1 << 20,
                                                  None))
    assert "stride" in _err(lib.coopt_accept_sample(_lib.DT_F32, 16, 50, 0, 0, 16, 100, 0, 16, 0,
                                                    16, 16, 1.0, 2, 4, 100, 16, 16, 0, 16,
                                                    1 << 20, None))
    rc = lib.coopt_accept_sample(_lib.DT_F32, 16, 100, 0, 0, 16, 100, 0, 16, 0, 16, 16, 1.0, 2, 4,
                                 100, 16, 16, 0, 16, 8, None)
    assert rc == _lib.COOPT_EWORKSPACE


def test_codec_rejects_bad_arguments(lib):
    assert "bits" in _err(lib.coopt_quantize(6, _lib.DT_BF16, 16, 4, 128, 16, 16, None))
    assert "even" in _err(lib.coopt_quantize(8, _lib.DT_BF16, 16, 4, 127, 16, 16, None))
    assert "out_dtype" in _err(lib.coopt_dequantize(8, 16, 16, 4, 128, _lib.DT_I8, 16, None))


def test_python_wrappers_refuse_cpu_tensors():
    import iitj_llm_coopt_amd as M

    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises(_lib.CooptError, match="no CPU fallback"):
        M.quantize(x, 8)
    with pytest.raises(_lib.CooptError, match="no CPU fallback"):
        M.sample(torch.zeros(2, 10), 1.0)


def test_accept_noalloc_rejects_sizes_beyond_its_scratch(lib):
    """The static-scratch accept entry point checks its size before touching the device."""
    cap = lib.coopt_accept_sample_noalloc_max_bytes()
    assert cap == 2 << 20
    assert lib.coopt_accept_sample_workspace(512, 8, 128256) <= cap
    need = lib.coopt_accept_sample_workspace(4096, 8, 262144)
    assert need > cap
    rc = lib.coopt_accept_sample_noalloc(_lib.DT_F32, 16, 262144, None, 0, 16, 262144, None, 16,
                                         None, 16, 16, 1.0, 4096, 8, 262144, 16, 16, 16, None)
    assert rc == _lib.COOPT_EWORKSPACE
    msg = _lib.last_error()
    assert "scratch" in msg and str(need) in msg and str(cap) in msg, msg
    assert lib.coopt_accept_sample_noalloc(_lib.DT_F32, 0, 1, None, 0, 0, 1, None, 0, None, 0, 0,
                                           1.0, 0, 4, 100, 0, 0, 0, None) == _lib.COOPT_OK
