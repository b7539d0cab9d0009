"""CPU: pins oracle.codec (restating engine/kv_tier_manager.py:21-41)."""
import numpy as np
import pytest
import torch

from oracle import codec


def bf16_values(rng, shape, outliers=0.01, scale=20.0):
    x = rng.standard_normal(shape).astype(np.float32)
    x = np.where(rng.random(shape) < outliers, x * scale, x)
    return codec.bf16_round(x)


def test_amax_maps_to_qmax_and_signs():
    x = np.array([[0.5, -2.0, 1.0, 2.0], [-3.0, 1.5, 0.0, 0.75]], np.float32)
    q, s = codec.quantize(x, 8)
    assert q[0, 3] == 127 and q[0, 1] == -127 and q[1, 0] == -127
    assert s.dtype == np.float16
    assert np.isclose(float(s[0]), 2.0 / 127, rtol=1e-3)
    q4, s4 = codec.quantize(x, 4)
    lo = (q4 & 0xF).astype(int) - 8
    hi = (q4 >> 4).astype(int) - 8
    assert hi[0, 1] == 7 and hi[0, 0] == -7  # x[0,3]=2 (amax) -> +7 ; x[0,1]=-2 -> -7
    assert lo[0, 0] == 2  # x[0,0]=0.5 -> round(1.75) = 2


def test_zero_vector_has_zero_fp16_scale_and_codes():
    q, s = codec.quantize(np.zeros((3, 128), np.float32), 8)
    assert (q == 0).all()
    # fp32 scale 1e-8/127 ~ 7.9e-11 underflows fp16 to 0 (round to nearest)
    assert (s == 0).all() and not np.signbit(s).any()


def test_half_ties_round_to_even():
    # amax 127 -> s32 = 127 * fl(1/127) = 1.0 exactly, so codes are round(x)
    assert np.float32(127) * (np.float32(1) / np.float32(127)) == np.float32(1.0)
    x = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]], np.float32)
    q, _ = codec.quantize(x, 8)
    assert q.tolist() == [[127, 0, 2, 2, 0, -2, -2, 4]]


def test_outlier_crushes_other_codes():
    x = np.full((1, 128), 0.01, np.float32)
    x[0, 7] = 50.0
    q, s = codec.quantize(x, 8)
    assert q[0, 7] == 127 and (np.delete(q[0], 7) == 0).all()


@pytest.mark.parametrize("bits", [8, 4])
def test_cpu_mode_matches_reference_lines_run_by_torch_cpu(bits):
    rng = np.random.default_rng(0)
    x = bf16_values(rng, (512, 128))
    qt, st = codec.quantize_torch_cpu(torch.from_numpy(x).to(torch.bfloat16), bits)
    qo, so = codec.quantize(x, bits, mode="cpu")
    assert np.array_equal(qt.numpy(), qo)
    assert np.array_equal(st.numpy(), so)


def test_device_and_cpu_division_differ_only_in_last_bit_of_fp32_scale():
    rng = np.random.default_rng(1)
    amax = codec.bf16_round(np.abs(rng.standard_normal(200000)).astype(np.float32) * 4 + 1e-3)
    dev = np.maximum(amax, np.float32(1e-8)) * (np.float32(1) / np.float32(127))
    cpu = np.maximum(amax, np.float32(1e-8)) / np.float32(127)
    ulps = np.abs(dev.view(np.int32).astype(np.int64) - cpu.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1  # the two modes are one fp32 rounding apart at most
    assert (ulps == 1).any()  # ...and they do differ, so the mode matters for bit-exactness


@pytest.mark.parametrize("bits,qmax", [(8, 127), (4, 7)])
def test_round_trip_error_bound(bits, qmax):
    rng = np.random.default_rng(2)
    x = bf16_values(rng, (256, 128))
    q, s = codec.quantize(x, bits)
    y = codec.dequantize(q, s, bits)
    amax = np.abs(x).max(-1, keepdims=True)
    # half a code step, plus the fp16 rounding of the scale applied to |code| <= qmax
    bound = amax / qmax * (0.5 + qmax * 2.0 ** -10) + 1e-6
    assert (np.abs(y - x) <= bound).all()


def test_int4_pack_layout_even_low_odd_high():
    x = np.array([[7.0, -7.0, 1.0, -1.0]], np.float32)  # amax 7 -> scale 1, codes = x
    q, _ = codec.quantize(x, 4)
    assert q.tolist() == [[(7 + 8) | ((-7 + 8) << 4), (1 + 8) | ((-1 + 8) << 4)]]
    assert np.array_equal(codec.dequantize(q, np.float16([1.0]), 4), x)


def test_bf16_round_ties_to_even():
    # 1 + 2^-8 is halfway between bf16 neighbours 1 and 1 + 2^-7: ties to even (1.0)
    assert codec.bf16_round(np.float32(1 + 2 ** -8)) == np.float32(1.0)
    assert codec.bf16_round(np.float32(1 + 3 * 2 ** -8)) == np.float32(1 + 2 ** -6)
    t = torch.randn(4096)
    assert np.array_equal(codec.bf16_round(t.numpy()), t.to(torch.bfloat16).float().numpy())
