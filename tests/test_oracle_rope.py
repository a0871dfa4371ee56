"""Pins of the CPU oracle's rotary embedding and Q/K epilogue (CPU only).

The oracle restates the reference's fused_rope kernel (src/optimized.cu:77).
It is checked here against:
  - the reference's own known answer: zero positions give x back
    (tests/optimized_test.cpp:139-141);
  - an independent restatement in torch.  The axis choice uses the slices of
    the published interleaved mRoPE (HF Qwen3.5 `apply_interleaved_mrope`,
    references/modeling_qwen3_5.py).  The inverse frequencies come from
    float64 pow.  The rotation is rotate_half, with the BF16 tensor rounding
    points of the reference's unoptimized branch (src/engine.cpp:253-256,
    :286-297);
  - planted mistakes (a flipped sign, interleaved pairs, every pair on the
    temporal axis) that the same comparison must reject.
"""
import numpy as np
import pytest
import torch

from parity import bf16_to_f32, ulp_distance


def bf16_bits(t):
    return t.to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(b):
    return torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).view(torch.bfloat16)


def rand_bits(rng, shape):
    return bf16_bits(torch.from_numpy(rng.standard_normal(shape).astype(np.float32)))


def torch_rope(x_bits, pos, rotary, theta, hs, ws, sign=1.0, interleaved=False, axes=True):
    """Interleaved multi-axis RoPE written from the published definition, not
    from the reference kernel: freqs[a] = pos[a] * inv_freq, the temporal row
    overwritten at f = 1, 4, ... < 3*hs by the height row and at
    f = 2, 5, ... < 3*ws by the width row; then x*cos + rotate_half(x)*sin in
    BF16 tensor arithmetic.  sign / interleaved / axes plant mistakes."""
    x = from_bits(x_bits)  # [T, H, D]
    half = rotary // 2
    inv = torch.tensor([theta ** (-2.0 * j / rotary) for j in range(half)], dtype=torch.float64).float()
    freqs = torch.from_numpy(pos).float()[:, :, None] * inv[None, None, :]  # [3, T, half]
    f = freqs[0].clone()
    if axes:
        f[..., 1:hs * 3:3] = freqs[1][..., 1:hs * 3:3]
        f[..., 2:ws * 3:3] = freqs[2][..., 2:ws * 3:3]
    angle = torch.cat([f, f], -1)  # [T, rotary]
    cos = angle.cos().to(torch.bfloat16).unsqueeze(1)
    sin = angle.sin().to(torch.bfloat16).unsqueeze(1)
    a, rest = x[..., :rotary], x[..., rotary:]
    if interleaved:
        rot = torch.stack([-a[..., 1::2], a[..., 0::2]], -1).flatten(-2)
    else:
        rot = torch.cat([-a[..., half:], a[..., :half]], -1)
    if sign < 0:
        rot = -rot
    return bf16_bits(torch.cat([a * cos + rot * sin, rest], -1))


def close(got, ref, min_exact, max_ulp):
    u = ulp_distance(got, ref)
    return (u == 0).mean() >= min_exact and u.max() <= max_ulp


def test_zero_positions_identity(oracle):
    """tests/optimized_test.cpp:139-141: x [3, 2, 64], zero positions,
    rotary 32, theta 1e4, sections 4 and 4 -> x bit for bit."""
    rng = np.random.default_rng(141)
    x = rand_bits(rng, (3, 2, 64))
    y = oracle.rope(x, np.zeros((3, 3), np.int64), 32, 1e4, 4, 4)
    assert np.array_equal(bf16_to_f32(y), bf16_to_f32(x))


@pytest.mark.parametrize("shape,rotary,theta,hs,ws", [
    ((5, 12, 256), 64, 1e7, 11, 10),   # the model's layer (TP=2 rank), sections [11, 11, 10]
    ((9, 2, 128), 128, 1e4, 4, 2),    # full rotation, section bounds inside the pairs
    ((4, 3, 100), 30, 5e5, 2, 5),     # ragged head and rotary sizes
])
def test_rope_against_published_mrope(oracle, shape, rotary, theta, hs, ws):
    """The oracle agrees with the independent torch restatement: the
    pass-through part bit for bit, the rotated part exactly on >= 99% of the
    values and within 2 BF16 ulps everywhere.  Differences come from 1-ulp
    differences of the FP32 inverse frequency (powf here, float64 pow there),
    which move cos/sin across a BF16 rounding point at large angles.  Each
    planted mistake fails the same bar."""
    rng = np.random.default_rng(sum(shape) + rotary)
    T = shape[0]
    x = rand_bits(rng, shape)
    pos = rng.integers(0, 4096, size=(3, T), dtype=np.int64)
    y = oracle.rope(x, pos, rotary, theta, hs, ws)
    ref = torch_rope(x, pos, rotary, theta, hs, ws)
    assert np.array_equal(y[..., rotary:], x[..., rotary:])
    assert close(y, ref, 0.99, 2), (ulp_distance(y, ref) == 0).mean()
    for mistake in (dict(sign=-1.0), dict(interleaved=True), dict(axes=False)):
        assert not close(y, torch_rope(x, pos, rotary, theta, hs, ws, **mistake), 0.99, 2), mistake


def test_rope_position_closed_forms(oracle):
    """Rotary pairs at angle 0 (position 0 on every axis) pass through.  With
    theta = 1 every frequency is 1, so every pair f rotates by the angle of
    its axis's position, whatever f is."""
    rng = np.random.default_rng(7)
    x = rand_bits(rng, (2, 1, 16))
    pos = np.array([[0, 3], [0, 5], [0, 7]], np.int64)
    y = oracle.rope(x, pos, 16, 1.0, 8, 8)
    assert np.array_equal(y[0], x[0])
    xf = bf16_to_f32(x[1, 0]).astype(np.float64)
    for f in range(8):
        p = pos[1 if f % 3 == 1 else (2 if f % 3 == 2 else 0), 1]
        c = bf16_to_f32(bf16_bits(torch.tensor([np.cos(np.float32(p))], dtype=torch.float32)))[0]
        s = bf16_to_f32(bf16_bits(torch.tensor([np.sin(np.float32(p))], dtype=torch.float32)))[0]
        want0 = xf[f] * c - xf[f + 8] * s
        want1 = xf[f + 8] * c + xf[f] * s
        got = bf16_to_f32(y[1, 0])
        assert abs(got[f] - want0) <= 0.02 * max(1.0, abs(want0)), (f, got[f], want0)
        assert abs(got[f + 8] - want1) <= 0.02 * max(1.0, abs(want1)), (f, got[f + 8], want1)


def test_qk_norm_rope_layout(oracle):
    """The Q/K epilogue reads the QKV-gate output as the reference slices it
    (src/engine.cpp:279-282): per token H blocks [query D | gate D], then HK
    key heads, then HK value heads.  Built from separate query, gate, key and
    value arrays, its q and k match the torch restatement of the unoptimized
    branch: the centered norm of src/engine.cpp:245-247, then the rotation
    above.  Gate and value columns must not leak in."""
    rng = np.random.default_rng(279)
    T, H, HK, D, R = 3, 4, 2, 64, 16
    qh, gh = rand_bits(rng, (T, H, D)), rand_bits(rng, (T, H, D))
    kh, vh = rand_bits(rng, (T, HK, D)), rand_bits(rng, (T, HK, D))
    projected = np.concatenate([np.concatenate([qh, gh], -1).reshape(T, -1), kh.reshape(T, -1),
                                vh.reshape(T, -1)], -1)
    qw, kw = rand_bits(rng, (D,)), rand_bits(rng, (D,))
    pos = rng.integers(0, 512, size=(3, T), dtype=np.int64)
    q, k = oracle.qk_norm_rope(projected, qw, kw, pos, H, HK, D, R, 1e6, 3, 2, 1e-6)

    def torch_norm(h, w):
        f = from_bits(h).float()
        n = f * torch.rsqrt((f * f).mean(-1, keepdim=True) + 1e-6)
        return bf16_bits(n * (from_bits(w).float() + 1))

    for got, heads, w in ((q, qh, qw), (k, kh, kw)):
        want = torch_rope(torch_norm(heads, w), pos, R, 1e6, 3, 2)
        assert close(got, want, 0.99, 2), (ulp_distance(got, want) == 0).mean()
    swapped, _ = oracle.qk_norm_rope(np.concatenate([np.concatenate([gh, qh], -1).reshape(T, -1),
                                                     kh.reshape(T, -1), vh.reshape(T, -1)], -1),
                                     qw, kw, pos, H, HK, D, R, 1e6, 3, 2, 1e-6)
    assert not close(swapped, q, 0.5, 4)


@pytest.mark.parametrize("theta,rotary", [(1e7, 64), (1e4, 128), (5e5, 30), (1e4, 4096), (1e4, 30)])
def test_frequency_exp2_form_is_powf(theta, rotary):
    """The device computes the inverse frequency theta^(-2f/R) as
    float(exp2(double(e) * log2(double(float(theta))))) with e = -2f/R in
    FP32 and log2 from the host.  For every pair of the tested (theta, R)
    combinations that equals the FP32 powf the oracle uses (glibc's, correctly
    rounded), so the device and the oracle rotate by the same angles."""
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    t32 = np.float32(theta)
    log2t = np.log2(np.float64(t32))
    bad = []
    for f in range(1, rotary // 2):
        e = np.float32(np.float32(-2.0) * np.float32(f)) / np.float32(rotary)
        dev = np.float32(np.exp2(np.float64(e) * log2t))
        ref = np.float32(libm.powf(float(t32), float(e)))
        if dev != ref:
            bad.append((f, float(dev), float(ref)))
    assert not bad, bad
