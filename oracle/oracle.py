"""ctypes binding of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker: the product library never calls it and
has no CPU fallback.  The C functions it binds cite the reference file:line
they restate (oracle/fp8lin_oracle.h).

All arrays are numpy; BF16 tensors are carried as uint16 bit patterns.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "liboracle.so")

_lib = None

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_f32p = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.c_int64
_f64p = ctypes.POINTER(ctypes.c_double)
_i64p = ctypes.POINTER(ctypes.c_int64)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("CPU oracle not built: run `python oracle/build_oracle.py` "
                               "(or __graft_entry__.build())")
        _lib = ctypes.CDLL(LIB_PATH)
        L = _lib
        L.oracle_fp8_e4m3_value.restype = ctypes.c_float
        L.oracle_fp8_e4m3_value.argtypes = [ctypes.c_uint8]
        L.oracle_bf16_rne.restype = ctypes.c_uint16
        L.oracle_bf16_rne.argtypes = [ctypes.c_float]
        L.oracle_e4m3_from_float.restype = ctypes.c_uint8
        L.oracle_e4m3_from_float.argtypes = [ctypes.c_float]
        L.oracle_decode_table.argtypes = [_f32p]
        L.oracle_bf16_rne_array.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.oracle_e4m3_from_float_array.argtypes = [_f32p, _u8p, ctypes.c_size_t]
        L.oracle_expand_block_scales.argtypes = [_f32p, _f32p, _i64, _i64]
        L.oracle_dequant.argtypes = [_u8p, _f32p, _i64, _u16p, _i64, _i64]
        L.oracle_linear.restype = ctypes.c_int
        L.oracle_linear.argtypes = [_u16p, _u8p, _f32p, _i64, _u16p, _i64, _i64, _i64,
                                    _i64, _i64, ctypes.c_int]
        L.oracle_linear_bf16w.restype = ctypes.c_int
        L.oracle_linear_bf16w.argtypes = [_u16p, _u16p, _u16p, _i64, _i64, _i64, ctypes.c_int]
        L.oracle_swiglu.argtypes = [_u16p, _u16p, _i64, _i64]
        L.oracle_philox4x32_10.argtypes = [_u32p, _u32p, _u32p]
        L.oracle_normal.restype = ctypes.c_float
        L.oracle_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64]
        L.oracle_normal_array.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint64,
                                          _f32p, ctypes.c_size_t]
        L.oracle_gen_weights.argtypes = [ctypes.c_uint64, ctypes.c_uint32, _i64, _i64,
                                         ctypes.c_float, _u8p, _f32p, _f32p]
        L.oracle_gen_activations.argtypes = [ctypes.c_uint64, ctypes.c_uint32, _i64, _i64, _u16p]
        L.oracle_max_threads.restype = ctypes.c_int
        L.oracle_rms.argtypes = [_u16p, _u16p, _u16p, _i64, _i64, ctypes.c_float, ctypes.c_int]
        L.oracle_residual_rms.argtypes = [_u16p, _u16p, _u16p, _u16p, _u16p, _i64, _i64, ctypes.c_float,
                                          ctypes.c_int]
        L.oracle_rope.argtypes = [_u16p, _i64p, _u16p, _i64, _i64, _i64, _i64, ctypes.c_float, _i64, _i64]
        L.oracle_vocab_candidates.argtypes = [_u16p, _i64, _i64, _i64, _f64p]
        L.oracle_merge_candidates.argtypes = [_f64p, _i64, _i64, _i64p]
    return _lib


def _p(a, t):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(t)


# ---- scalar codecs ----
def decode_table():
    out = np.empty(256, np.float32)
    lib().oracle_decode_table(_p(out, _f32p))
    return out


def fp8_decode_values(codes):
    return decode_table()[np.asarray(codes, np.uint8)]


def bf16_rne(values):
    v = np.ascontiguousarray(values, np.float32)
    out = np.empty(v.shape, np.uint16)
    lib().oracle_bf16_rne_array(_p(v, _f32p), _p(out, _u16p), v.size)
    return out


def bf16_to_float(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_from_float(values):
    v = np.ascontiguousarray(values, np.float32)
    out = np.empty(v.shape, np.uint8)
    lib().oracle_e4m3_from_float_array(_p(v, _f32p), _p(out, _u8p), v.size)
    return out


def expand_block_scales(block, n):
    block = np.ascontiguousarray(block, np.float32)
    kb = block.shape[1]
    out = np.empty((n, kb), np.float32)
    lib().oracle_expand_block_scales(_p(block, _f32p), _p(out, _f32p), n, kb)
    return out


# ---- linear-path functions ----
def _scale_cols(scales, n, k):
    s = np.ascontiguousarray(scales, np.float32)
    if s.ndim == 1:
        assert s.shape[0] == n
        return s, 1
    assert s.shape == (n, (k + 127) // 128), s.shape
    return s, s.shape[1]


def dequant(codes, scales):
    codes = np.ascontiguousarray(codes, np.uint8)
    n, k = codes.shape
    s, sc = _scale_cols(scales, n, k)
    out = np.empty((n, k), np.uint16)
    lib().oracle_dequant(_p(codes, _u8p), _p(s, _f32p), sc, _p(out, _u16p), n, k)
    return out


def linear(x_bits, codes, scales, rows=None, threads=0):
    """FP64 oracle of fp8_linear: x [M,K] bf16 bits, codes [N,K] u8, scales
    [N] or [N,ceil(K/128)] -> y [M,N] bf16 bits.  `rows` = (begin, end)
    restricts the computed output columns (others are zero)."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    codes = np.ascontiguousarray(codes, np.uint8)
    m, k = x.shape
    n = codes.shape[0]
    assert codes.shape[1] == k
    s, sc = _scale_cols(scales, n, k)
    y = np.zeros((m, n), np.uint16)
    b, e = rows if rows is not None else (0, n)
    rc = lib().oracle_linear(_p(x, _u16p), _p(codes, _u8p), _p(s, _f32p), sc, _p(y, _u16p),
                             m, n, k, b, e, threads)
    assert rc == 0, "oracle_linear rejected its arguments"
    return y


def linear_bf16w(x_bits, w_bits, threads=0):
    x = np.ascontiguousarray(x_bits, np.uint16)
    w = np.ascontiguousarray(w_bits, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), np.uint16)
    rc = lib().oracle_linear_bf16w(_p(x, _u16p), _p(w, _u16p), _p(y, _u16p), m, n, k, threads)
    assert rc == 0
    return y


def swiglu(gate_up_bits):
    g = np.ascontiguousarray(gate_up_bits, np.uint16)
    m, d2 = g.shape
    assert d2 % 2 == 0
    y = np.empty((m, d2 // 2), np.uint16)
    lib().oracle_swiglu(_p(g, _u16p), _p(y, _u16p), m, d2 // 2)
    return y


# ---- decode epilogue and output head ----
def rms(x_bits, w_bits, eps=1e-6, centered=True):
    x = np.ascontiguousarray(x_bits, np.uint16)
    w = np.ascontiguousarray(w_bits, np.uint16)
    m, d = x.shape
    y = np.empty_like(x)
    lib().oracle_rms(_p(x, _u16p), _p(w, _u16p), _p(y, _u16p), m, d, eps, int(centered))
    return y


def rope(x_bits, positions, rotary, theta, height_section, width_section):
    """x_bits [T, H, D] uint16 (BF16), positions [3, T] int64; theta is used
    in FP32 as the reference's kernel parameter is."""
    x = np.ascontiguousarray(x_bits, np.uint16)
    pos = np.ascontiguousarray(positions, np.int64)
    t, h, d = x.shape
    assert pos.shape == (3, t) and 0 < rotary <= d and rotary % 2 == 0
    y = np.empty_like(x)
    lib().oracle_rope(_p(x, _u16p), _p(pos, _i64p), _p(y, _u16p), t, h, d, rotary, float(theta),
                      height_section, width_section)
    return y


def qk_norm_rope(projected_bits, q_norm_bits, k_norm_bits, positions, heads, kv_heads, head_dim, rotary, theta,
                 height_section, width_section, eps=1e-6):
    """The optimized branch of src/engine.cpp:279-287 on the QKV-gate output
    [T, H*2D + 2*HK*D]: q = rope(rms(q rows)), k = rope(rms(k rows)) with the
    centered norm of src/engine.cpp:243-244 (one_center defaults to true,
    include/avi/engine.h:50)."""
    p = np.ascontiguousarray(projected_bits, np.uint16)
    t = p.shape[0]
    hd, kd = heads * head_dim, kv_heads * head_dim
    assert p.shape[1] == 2 * hd + 2 * kd
    q = p[:, :2 * hd].reshape(t, heads, 2 * head_dim)[:, :, :head_dim].reshape(t * heads, head_dim)
    k = p[:, 2 * hd:2 * hd + kd].reshape(t * kv_heads, head_dim)
    q = rms(q, q_norm_bits, eps, True).reshape(t, heads, head_dim)
    k = rms(k, k_norm_bits, eps, True).reshape(t, kv_heads, head_dim)
    args = (positions, rotary, theta, height_section, width_section)
    return rope(q, *args), rope(k, *args)


def residual_rms(x_bits, u_bits, w_bits, eps=1e-6, centered=True):
    x = np.ascontiguousarray(x_bits, np.uint16)
    u = np.ascontiguousarray(u_bits, np.uint16)
    w = np.ascontiguousarray(w_bits, np.uint16)
    m, d = x.shape
    res, y = np.empty_like(x), np.empty_like(x)
    lib().oracle_residual_rms(_p(x, _u16p), _p(u, _u16p), _p(w, _u16p), _p(res, _u16p), _p(y, _u16p), m, d,
                              eps, int(centered))
    return res, y


def vocab_candidates(logit_bits, offset=0):
    lg = np.ascontiguousarray(logit_bits, np.uint16)
    m, n = lg.shape
    out = np.empty((m, 2), np.float64)
    lib().oracle_vocab_candidates(_p(lg, _u16p), m, n, offset, _p(out, _f64p))
    return out


def merge_candidates(gathered):
    g = np.ascontiguousarray(gathered, np.float64)
    ranks, rows, two = g.shape
    assert two == 2
    out = np.empty(rows, np.int64)
    lib().oracle_merge_candidates(_p(g, _f64p), ranks, rows, _p(out, _i64p))
    return out


# ---- synthetic inputs ----
def philox(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.empty(4, np.uint32)
    lib().oracle_philox4x32_10(_p(c, _u32p), _p(k, _u32p), _p(out, _u32p))
    return out


def normal(seed, tag, first, n):
    out = np.empty(n, np.float32)
    lib().oracle_normal_array(seed, tag, first, _p(out, _f32p), n)
    return out


def gen_weights(seed, tag, n, k, std=0.02, want_w=False):
    codes = np.empty((n, k), np.uint8)
    scales = np.empty((n, (k + 127) // 128), np.float32)
    w = np.empty((n, k), np.float32) if want_w else None
    lib().oracle_gen_weights(seed, tag, n, k, std, _p(codes, _u8p), _p(scales, _f32p),
                             _p(w, _f32p) if want_w else None)
    return (codes, scales, w) if want_w else (codes, scales)


def gen_activations(seed, tag, m, k):
    x = np.empty((m, k), np.uint16)
    lib().oracle_gen_activations(seed, tag, m, k, _p(x, _u16p))
    return x


def max_threads():
    return lib().oracle_max_threads()
