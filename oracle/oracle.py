"""ctypes view of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the
benchmark's CPU-baseline leg, never by the product.  See vxm_oracle.c for
the reference citations of each function.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
BASE_LIB = os.path.join(HERE, "libcpubase.so")

QUANT_REF = 0
QUANT_X86 = 1

_P = C.c_void_p
_I64 = C.c_int64
_I = C.c_int
_F = C.c_float


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class Cfg(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32), ("n_heads", C.c_int32), ("n_kv_heads", C.c_int32),
        ("head_dim", C.c_int32), ("ffn", C.c_int32), ("eps", C.c_float),
        ("rope_theta", C.c_float), ("no_rope", C.c_int32), ("scale", C.c_float),
        ("rope_ff", C.c_void_p), ("quant_variant", C.c_int32),
    ]


class Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "g_in", "g_post")] + [
        ("wtype", C.c_int32)]


class LocDiT(C.Structure):
    _fields_ = [
        ("layers", C.c_void_p), ("n_layers", C.c_int32),
        ("in_proj", C.c_void_p), ("in_bias", C.c_void_p),
        ("cond_proj", C.c_void_p), ("cond_bias", C.c_void_p),
        ("out_proj", C.c_void_p), ("out_bias", C.c_void_p),
        ("norm", C.c_void_p),
        ("t_w1", C.c_void_p), ("t_w2", C.c_void_p), ("dt_w1", C.c_void_p), ("dt_w2", C.c_void_p),
        ("t_b1", C.c_void_p), ("t_b2", C.c_void_p), ("dt_b1", C.c_void_p), ("dt_b2", C.c_void_p),
        ("feat", C.c_int32),
    ]


class LocEnc(C.Structure):
    _fields_ = [
        ("layers", C.c_void_p), ("n_layers", C.c_int32),
        ("in_proj", C.c_void_p), ("in_bias", C.c_void_p),
        ("special", C.c_void_p), ("norm", C.c_void_p),
        ("feat", C.c_int32),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = C.CDLL(LIB)
        L.orc_fp32_to_fp16.restype = C.c_uint16
        L.orc_fp32_to_fp16.argtypes = [_F]
        L.orc_fp16_to_fp32.restype = _F
        L.orc_fp16_to_fp32.argtypes = [C.c_uint16]
        L.orc_bf16_round.restype = _F
        L.orc_bf16_round.argtypes = [_F]
        L.orc_fp32_to_fp16_n.argtypes = [_P, _P, _I64]
        L.orc_fp16_to_fp32_n.argtypes = [_P, _P, _I64]
        L.orc_bf16_round_n.argtypes = [_P, _P, _I64]
        L.orc_quantize_row_q8_0.argtypes = [_P, _P, _I64, _I]
        L.orc_quantize_rows_q8_0.argtypes = [_P, _P, _I64, _I64, _I]
        L.orc_dequantize_row_q8_0.argtypes = [_P, _P, _I64]
        L.orc_block_dots_q8_0.argtypes = [_P, _P, _I64, _I64, _I64, _P]
        L.orc_mul_mat_q8_0.argtypes = [_P, _P, _I64, _I64, _I64, _P]
        L.orc_mul_mat_q8_0_f64.argtypes = [_P, _P, _I64, _I64, _I64, _P]
        L.orc_rms_norm.argtypes = [_P, _P, _I64, _I64, _F, _P]
        L.orc_rope_neox.argtypes = [_P, _I64, _I64, C.c_int32, _F, _P]
        L.orc_silu.restype = _F
        L.orc_silu.argtypes = [_F]
        L.orc_minicpm4_block.argtypes = [C.POINTER(Cfg), C.POINTER(Layer), _P, _I64, _P, _P, _I64,
                                         C.c_int32, _I]
        L.orc_attention.argtypes = [C.POINTER(Cfg), C.POINTER(Layer), _P, _I64, _P, _P, _I64, C.c_int32, _I, _P]
        L.orc_mlp.argtypes = [C.POINTER(Cfg), C.POINTER(Layer), _P, _I64, _P]
        L.orc_minicpm4_forward.argtypes = [C.POINTER(Cfg), _P, C.c_int32, _P, _P, _I64, _P, _P, _I64,
                                           C.c_int32]
        L.orc_sinusoid_embed.argtypes = [_F, C.c_int32, _P]
        L.orc_locdit_forward.argtypes = [C.POINTER(Cfg), C.POINTER(LocDiT), _P, _P, C.c_int32, C.c_int32,
                                         _F, _F, _P, _P]
        L.orc_locdit_forward_states.argtypes = [C.POINTER(Cfg), C.POINTER(LocDiT), _P, _P, C.c_int32, C.c_int32,
                                                _F, _F, _P, _P, _P]
        L.orc_cfm_sway_t_bf16.restype = _F
        L.orc_cfm_sway_t_bf16.argtypes = [_I, _I]
        L.orc_cfm_uniform_t_bf16.restype = _F
        L.orc_cfm_uniform_t_bf16.argtypes = [_I, _I]
        L.orc_cfm_cfg_zero_star.restype = _F
        L.orc_cfm_cfg_zero_star.argtypes = [_P, _P, _I, _F]
        L.orc_cfm_zero_star_steps.argtypes = [_I]
        L.orc_cfm_step_dt.restype = _F
        L.orc_cfm_step_dt.argtypes = [_I, _I, _I]
        L.orc_cfm_euler_update.argtypes = [_P, _P, _I, _F]
        L.orc_cfm_solve.argtypes = [C.POINTER(Cfg), C.POINTER(LocDiT), _P, _P, C.c_int32, C.c_int32, _P,
                                    _I, _F, _I, _I]
        L.orc_locenc_forward.argtypes = [C.POINTER(Cfg), C.POINTER(LocEnc), _P, C.c_int32, _P, _P]
        L.orc_fsq_quantize.argtypes = [_P, _I64, _F, _P]
        _lib = L
    return _lib


# ---- number formats ----

def fp32_to_fp16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_fp32_to_fp16_n(_p(x), _p(out), x.size)
    return out


def fp16_bits_to_fp32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_fp16_to_fp32_n(_p(h), _p(out), h.size)
    return out


def bf16_round(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.float32)
    lib().orc_bf16_round_n(_p(x), _p(out), x.size)
    return out


# ---- Q8_0 ----

def quantize_rows(x, variant):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    out = np.empty(rows * (k // 32) * 34, dtype=np.uint8)
    lib().orc_quantize_rows_q8_0(_p(x), _p(out), rows, k, variant)
    return out


def dequantize_rows(q, rows, k):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty((rows, k), dtype=np.float32)
    rb = k // 32 * 34
    for r in range(rows):
        lib().orc_dequantize_row_q8_0(_p(q[r * rb:(r + 1) * rb]), _p(out[r]), k)
    return out


def split_q8(q, rows, k):
    """GGUF rows -> (qs int8 [rows][k], d fp16 bits [rows][k/32])."""
    b = np.ascontiguousarray(q, dtype=np.uint8).reshape(rows, k // 32, 34)
    d = b[:, :, :2].copy().view(np.uint16).reshape(rows, k // 32)
    qs = b[:, :, 2:].copy().view(np.int8).reshape(rows, k)
    return qs, d


def join_q8(qs, d):
    rows, k = qs.shape
    b = np.empty((rows, k // 32, 34), dtype=np.uint8)
    b[:, :, :2] = np.ascontiguousarray(d, dtype=np.uint16).reshape(rows, k // 32, 1).view(np.uint8)
    b[:, :, 2:] = np.ascontiguousarray(qs, dtype=np.int8).reshape(rows, k // 32, 32).view(np.uint8)
    return b.reshape(-1)


def block_dots(w, xq, N, K, M):
    out = np.empty((M, N, K // 32), dtype=np.int32)
    lib().orc_block_dots_q8_0(_p(w), _p(xq), N, K, M, _p(out))
    return out


def mul_mat(w, xq, N, K, M):
    y = np.empty((M, N), dtype=np.float32)
    lib().orc_mul_mat_q8_0(_p(w), _p(xq), N, K, M, _p(y))
    return y


def mul_mat_f64(w, xq, N, K, M):
    y = np.empty((M, N), dtype=np.float64)
    lib().orc_mul_mat_q8_0_f64(_p(w), _p(xq), N, K, M, _p(y))
    return y


def rms_norm(x, g, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, n = x.shape
    y = np.empty_like(x)
    gg = None if g is None else np.ascontiguousarray(g, dtype=np.float32)
    lib().orc_rms_norm(_p(x), _p(gg), rows, n, eps, _p(y))
    return y


def rope_neox(x, n_heads, head_dim, pos, theta, ff=None):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    f = None if ff is None else np.ascontiguousarray(ff, dtype=np.float32)
    lib().orc_rope_neox(_p(x), n_heads, head_dim, pos, theta, _p(f))
    return x


# ---- MiniCPM4 ----

# LongRoPE short factors of the VoxCPM2 lm_config (src/minicpm4.c:49-66):
# model constants, one per rotary pair when head_dim == 128.
ROPE_SHORT_FACTORS = np.array([
    0.9977997200, 1.0146582960, 1.0349680405, 1.0594292461,
    1.0888815017, 1.1243301355, 1.1669771036, 1.2182568067,
    1.2798772354, 1.3538666752, 1.4426259040, 1.5489853360,
    1.6762658237, 1.8283407612, 2.0096956086, 2.2254789275,
    2.4815363797, 2.7844159346, 3.1413289096, 3.5600478448,
    4.0487193801, 4.6155695421, 5.2684819497, 6.0144385919,
    6.8588300492, 7.8046682500, 8.8517684937, 9.9960050583,
    11.2287664413, 12.5367574692, 13.9022579193, 15.3038854599,
    16.7178382874, 18.1194648743, 19.4849643707, 20.7929573059,
    22.0257186890, 23.1699542999, 24.2170543671, 25.1628932953,
    26.0072841644, 26.7532405853, 27.4061527252, 27.9730033875,
    28.4616756439, 28.8803939819, 29.2373065948, 29.5401859283,
    29.7962436676, 30.0120277405, 30.1933822632, 30.3454570770,
    30.4727382660, 30.5790977478, 30.6678562164, 30.7418460846,
    30.8034667969, 30.8547458649, 30.8973922729, 30.9328403473,
    30.9622936249, 30.9867553711, 31.0070648193, 31.0239238739,
], dtype=np.float32)


def make_cfg(hidden, n_heads, n_kv_heads, head_dim, ffn, eps=1e-6, rope_theta=10000.0, no_rope=0,
             scale=1.0, rope_ff=None, quant_variant=QUANT_X86):
    c = Cfg(hidden, n_heads, n_kv_heads, head_dim, ffn, eps, rope_theta, no_rope, scale, None, quant_variant)
    c._keep = None
    if rope_ff is not None:
        ff = np.ascontiguousarray(rope_ff, dtype=np.float32)
        c._keep = ff
        c.rope_ff = ff.ctypes.data
    return c


class LayerW:
    """Host copy of one block's weights: GGUF Q8_0 byte arrays + F32 gains."""

    names = ("wq", "wk", "wv", "wo", "wg", "wu", "wd", "g_in", "g_post")

    def __init__(self, wtype=0, **kw):
        self.wtype = wtype
        for n in self.names:
            v = kw.get(n)
            setattr(self, n, None if v is None else np.ascontiguousarray(v))

    def struct(self):
        return Layer(*[(None if getattr(self, n) is None else getattr(self, n).ctypes.data) for n in self.names],
                     self.wtype)


def minicpm4_block(cfg, lw, x, k_cache=None, v_cache=None, capacity=0, pos=0, no_causal=0):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    M = x.shape[0]
    s = lw.struct()
    rc = lib().orc_minicpm4_block(C.byref(cfg), C.byref(s), _p(x), M, _p(k_cache), _p(v_cache), capacity, pos,
                                  no_causal)
    assert rc == 0
    return x


def attention(cfg, lw, xn, k_cache=None, v_cache=None, capacity=0, pos=0, no_causal=0):
    xn = np.ascontiguousarray(xn, dtype=np.float32)
    M = xn.shape[0]
    out = np.empty((M, cfg.hidden), dtype=np.float32)
    s = lw.struct()
    rc = lib().orc_attention(C.byref(cfg), C.byref(s), _p(xn), M, _p(k_cache), _p(v_cache), capacity, pos,
                             no_causal, _p(out))
    assert rc == 0
    return out


def mlp(cfg, lw, xn):
    xn = np.ascontiguousarray(xn, dtype=np.float32)
    M = xn.shape[0]
    out = np.empty((M, cfg.hidden), dtype=np.float32)
    s = lw.struct()
    lib().orc_mlp(C.byref(cfg), C.byref(s), _p(xn), M, _p(out))
    return out


def minicpm4_forward(cfg, layers, final_norm, x, k_caches, v_caches, capacity, pos):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    M = x.shape[0]
    arr = (Layer * len(layers))(*[l.struct() for l in layers])
    kp = (C.c_void_p * len(layers))(*[k.ctypes.data for k in k_caches])
    vp = (C.c_void_p * len(layers))(*[v.ctypes.data for v in v_caches])
    fn = None if final_norm is None else np.ascontiguousarray(final_norm, dtype=np.float32)
    rc = lib().orc_minicpm4_forward(C.byref(cfg), C.cast(arr, C.c_void_p), len(layers), _p(fn), _p(x), M,
                                    C.cast(kp, C.c_void_p), C.cast(vp, C.c_void_p), capacity, pos)
    assert rc == 0
    return x


# ---- CFM ----

def sway_t(step, n):
    return lib().orc_cfm_sway_t_bf16(step, n)


def uniform_t(step, n):
    return lib().orc_cfm_uniform_t_bf16(step, n)


def cfg_zero_star(negative, positive, cfg_value):
    neg = np.ascontiguousarray(negative, dtype=np.float32).copy()
    pos = np.ascontiguousarray(positive, dtype=np.float32)
    st = lib().orc_cfm_cfg_zero_star(_p(neg), _p(pos), neg.size, cfg_value)
    return st, neg


def zero_star_steps(n):
    return lib().orc_cfm_zero_star_steps(n)


def cfm_step_dt(step, n, schedule=0):
    return lib().orc_cfm_step_dt(step, n, schedule)


def cfm_euler_update(x, v, dt):
    """orc_cfm_euler_update: bf16(x + bf16(dt * v)), returned as a new array."""
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    v = np.ascontiguousarray(v, dtype=np.float32)
    assert x.size == v.size
    lib().orc_cfm_euler_update(_p(x), _p(v), x.size, dt)
    return x


def sinusoid(t, dim):
    out = np.empty(dim, dtype=np.float32)
    lib().orc_sinusoid_embed(t, dim, _p(out))
    return out


# ---- LocDiT / CFM ----

class LocDiTW:
    """Host copy of LocDiT weights: GGUF Q8_0 rows + F32 vectors (biases may be None)."""

    names = ("in_proj", "in_bias", "cond_proj", "cond_bias", "out_proj", "out_bias", "norm",
             "t_w1", "t_w2", "dt_w1", "dt_w2", "t_b1", "t_b2", "dt_b1", "dt_b2")

    def __init__(self, layers, feat, **kw):
        self.layers = layers
        self.feat = feat
        for n in self.names:
            v = kw.get(n)
            setattr(self, n, None if v is None else np.ascontiguousarray(v))

    def struct(self):
        self._arr = (Layer * max(1, len(self.layers)))(*[l.struct() for l in self.layers])
        g = {n: (None if getattr(self, n) is None else getattr(self, n).ctypes.data) for n in self.names}
        return LocDiT(C.cast(self._arr, C.c_void_p).value, len(self.layers), g["in_proj"], g["in_bias"],
                      g["cond_proj"], g["cond_bias"], g["out_proj"], g["out_bias"], g["norm"], g["t_w1"],
                      g["t_w2"], g["dt_w1"], g["dt_w2"], g["t_b1"], g["t_b2"], g["dt_b1"], g["dt_b2"], self.feat)


def locdit_forward(cfg, w, x, cond, t, dt=0.0, mu=None):
    """orc_locdit_forward: velocity [P][feat] of x [P][feat] with cond [Pc][feat], mu [2][hidden] or None."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cond = np.ascontiguousarray(cond, dtype=np.float32)
    mu = None if mu is None else np.ascontiguousarray(mu, dtype=np.float32)
    P, Pc = x.shape[0], cond.shape[0]
    out = np.empty((P, w.feat), dtype=np.float32)
    s = w.struct()
    rc = lib().orc_locdit_forward(C.byref(cfg), C.byref(s), _p(x), _p(cond), P, Pc, t, dt, _p(mu), _p(out))
    assert rc == 0
    return out


def locdit_states(cfg, w, x, cond, t, dt=0.0, mu=None):
    """orc_locdit_forward_states: (velocity, sequence entering each block + after the last)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    cond = np.ascontiguousarray(cond, dtype=np.float32)
    mu = None if mu is None else np.ascontiguousarray(mu, dtype=np.float32)
    P, Pc = x.shape[0], cond.shape[0]
    S, H = 3 + Pc + P, cfg.hidden
    out = np.empty((P, w.feat), dtype=np.float32)
    states = np.empty((len(w.layers) + 1, S, H), dtype=np.float32)
    s = w.struct()
    rc = lib().orc_locdit_forward_states(C.byref(cfg), C.byref(s), _p(x), _p(cond), P, Pc, t, dt, _p(mu), _p(out),
                                         _p(states))
    assert rc == 0
    return out, states


def cfm_solve(cfg, w, x, cond, mu, n_steps, cfg_value, schedule=0, use_zero_star=1):
    """orc_cfm_solve: the CFM Euler loop (schedule 0 sway, 1 uniform); returns the final x."""
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    cond = np.ascontiguousarray(cond, dtype=np.float32)
    mu = None if mu is None else np.ascontiguousarray(mu, dtype=np.float32)
    s = w.struct()
    rc = lib().orc_cfm_solve(C.byref(cfg), C.byref(s), _p(x), _p(cond), x.shape[0], cond.shape[0], _p(mu),
                             n_steps, cfg_value, schedule, use_zero_star)
    assert rc == 0
    return x


# ---- LocEnc / FSQ / LM update ----

class LocEncW:
    """Host copy of LocEnc weights: GGUF Q8_0 rows of in_proj + F32 vectors (in_bias / special may be None)."""

    names = ("in_proj", "in_bias", "special", "norm")

    def __init__(self, layers, feat, **kw):
        self.layers = layers
        self.feat = feat
        for n in self.names:
            v = kw.get(n)
            setattr(self, n, None if v is None else np.ascontiguousarray(v))

    def struct(self):
        self._arr = (Layer * max(1, len(self.layers)))(*[l.struct() for l in self.layers])
        g = {n: (None if getattr(self, n) is None else getattr(self, n).ctypes.data) for n in self.names}
        return LocEnc(C.cast(self._arr, C.c_void_p).value, len(self.layers), g["in_proj"], g["in_bias"],
                      g["special"], g["norm"], self.feat)


def locenc_forward(cfg, w, x, states=False):
    """orc_locenc_forward: [hidden] (special-token row) or [P][hidden]; with states=True also the
    sequence entering each block and leaving the last."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    P, H = x.shape[0], cfg.hidden
    S = P + (w.special is not None)
    out = np.empty((1 if w.special is not None else P, H), dtype=np.float32)
    st = np.empty((len(w.layers) + 1, S, H), dtype=np.float32) if states else None
    s = w.struct()
    rc = lib().orc_locenc_forward(C.byref(cfg), C.byref(s), _p(x), P, _p(out), _p(st))
    assert rc == 0
    out = out[0] if w.special is not None else out
    return (out, st) if states else out


def fsq_quantize(x, quant_scale):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_fsq_quantize(_p(x), x.size, quant_scale, _p(y))
    return y


def linear(w, x, N, K, bias=None, variant=QUANT_X86):
    """ggml_mul_mat of Q8_0 rows w [N][K] with F32 x [M][K] (x quantized to Q8_0), plus an F32 bias."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    y = mul_mat(w, quantize_rows(x, variant), N, K, x.shape[0])
    if bias is not None:
        y = (y + np.asarray(bias, np.float32)).astype(np.float32)
    return y


def lm_update(enc_cfg, enc_w, tslm, ralm, pw, prev_patch, pos, fsq_scale=9.0, variant=QUANT_X86):
    """gen_lm_update (src/gen_step.c:712-927) composed from the oracle pieces.

    tslm / ralm: dicts with cfg, layers, norm, k, v (per-layer f16 caches, updated in place), cap.
    pw: dict of the projections (enc_to_lm, enc_to_lm_bias, fsq_in, fsq_in_bias, fsq_out, fsq_out_bias,
    fusion) as GGUF Q8_0 rows / F32 vectors, with widths L (lm hidden), E, Fq, R.
    Returns (audio_embed, base_hidden, fsq, ralm_hidden)."""
    L, E, R = pw["L"], pw["E"], pw["R"]
    fe = locenc_forward(enc_cfg, enc_w, prev_patch)
    audio = linear(pw["enc_to_lm"], fe, L, E, pw.get("enc_to_lm_bias"), variant)[0]
    base = minicpm4_forward(tslm["cfg"], tslm["layers"], tslm["norm"], audio[None], tslm["k"], tslm["v"],
                            tslm["cap"], pos)[0]
    if pw.get("fsq_in") is not None:
        Fq = pw["Fq"]
        h = linear(pw["fsq_in"], base, Fq, L, pw.get("fsq_in_bias"), variant)[0]
        q = fsq_quantize(h, fsq_scale)
        fsq = linear(pw["fsq_out"], q, L, Fq, pw.get("fsq_out_bias"), variant)[0]
    else:
        fsq = base.copy()
    cat = np.concatenate([fsq, audio]).astype(np.float32)
    ralm_in = linear(pw["fusion"], cat, R, 2 * L, None, variant)[0]
    ralm_h = minicpm4_forward(ralm["cfg"], ralm["layers"], ralm["norm"], ralm_in[None], ralm["k"], ralm["v"],
                              ralm["cap"], pos)[0]
    return audio, base, fsq, ralm_h


def prompt_prefill(tslm, ralm, pw, x, pos, variant=QUANT_X86):
    """gen_prompt_eval_range (src/gen_prompt.c:186-272) composed from the oracle pieces: the base LM over
    the n text embeddings x [n][L] at positions [pos, pos + n) (:197-200), the RALM input
    fusion_concat([base ; 0]) with a zero second half for every prompt row (:204-217), and the RALM over
    the same positions (:219-223).  tslm / ralm as in lm_update (caches updated in place).
    Returns (base_hidden [n][L], ralm_hidden [n][R])."""
    L, R = pw["L"], pw["R"]
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[0]
    base = minicpm4_forward(tslm["cfg"], tslm["layers"], tslm["norm"], x, tslm["k"], tslm["v"], tslm["cap"], pos)
    cat = np.concatenate([base, np.zeros((n, L), np.float32)], axis=1)
    ralm_in = linear(pw["fusion"], cat, R, 2 * L, None, variant)
    ralm_h = minicpm4_forward(ralm["cfg"], ralm["layers"], ralm["norm"], ralm_in, ralm["k"], ralm["v"],
                              ralm["cap"], pos)
    return base, ralm_h


def embed_rows_q8_0(table, n_rows, k, ids):
    """The Q8_0 branch of gen_forward_text's embedding rows (src/gen_prompt.c:106-125): row ids[i] of the
    GGUF Q8_0 table dequantized; an id outside [0, n_rows) reads row 0 (:113-114)."""
    ids = np.asarray(ids, np.int64)
    rb = k // 32 * 34
    out = np.empty((ids.size, k), np.float32)
    for i, r in enumerate(ids):
        r = int(r) if 0 <= r < n_rows else 0
        out[i] = dequantize_rows(table[r * rb:(r + 1) * rb], 1, k)[0]
    return out
