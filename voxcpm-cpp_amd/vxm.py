"""Python host mirror of the gfx950 Q8_0 library (libvxm_q8.so).

This module binds the C ABI declared in include/vxm_q8.h with ctypes and
offers the reference's operator vocabulary on top of it: ``mul_mat`` is
ggml_mul_mat(W_q8_0, x) (src/projections.h:24-29), ``rms_norm`` is
vcpm_rms_norm (src/minicpm4.c:132-152), and so on.  Device memory is
torch's (tensors on ``cuda:N``); torch is plumbing here, every computation
runs in the library's HIP kernels.  Nothing in this module falls back to a
CPU path: a missing library or a failed call raises ``VxmError``.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
# the in-tree library; VXM_LIB names another build of it (the profiling build, libvxm_q8_trace.so)
LIB_PATH = os.environ.get("VXM_LIB") or os.path.join(HERE, "libvxm_q8.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "vxm_q8.h")

QUANT_REF = 0
QUANT_X86 = 1
PATH_AUTO = 0
PATH_GEMV = 1
PATH_MFMA = 2
PATH_MFMA_TILED = 3
DECODE_AUTO = 0          # block strategies (vxm_minicpm4_set_decode_mode, vxm_locdit_set_block_mode)
DECODE_KERNELS = 1
DECODE_PERSISTENT = 2

STATUS = {
    0: "VXM_OK",
    1: "VXM_ERR_INVALID_ARG",
    2: "VXM_ERR_IO",
    3: "VXM_ERR_MODEL_FORMAT",
    4: "VXM_ERR_UNSUPPORTED_ARCH",
    5: "VXM_ERR_BACKEND",
    6: "VXM_ERR_OOM",
    7: "VXM_ERR_NOT_IMPLEMENTED",
}


class VxmError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code


_lib = None

_P = C.c_void_p
_I64 = C.c_int64
_I = C.c_int
_F = C.c_float
_U64 = C.c_uint64

# name -> (restype, argtypes)
_SIGS = {
    "vxm_open": (_I, [_I, C.POINTER(_P)]),
    "vxm_close": (_I, [_P]),
    "vxm_sync": (_I, [_P]),
    "vxm_get_stream": (_P, [_P]),
    "vxm_last_error": (C.c_char_p, [_P]),
    "vxm_set_quant_variant": (_I, [_P, _I]),
    "vxm_set_path": (_I, [_P, _I]),
    "vxm_capture_begin": (_I, [_P]),
    "vxm_capture_end": (_I, [_P, C.POINTER(_P)]),
    "vxm_graph_launch": (_I, [_P, _P]),
    "vxm_graph_free": (_I, [_P]),
    "vxm_malloc": (_I, [_P, C.c_size_t, C.POINTER(_P)]),
    "vxm_free": (_I, [_P, _P]),
    "vxm_memcpy_h2d": (_I, [_P, _P, _P, C.c_size_t]),
    "vxm_memcpy_d2h": (_I, [_P, _P, _P, C.c_size_t]),
    "vxm_upload_q8_0": (_I, [_P, _P, _I64, _I64, C.POINTER(_P)]),
    "vxm_download_q8_0": (_I, [_P, _P, _P]),
    "vxm_weight_free": (_I, [_P, _P]),
    "vxm_weight_rows": (_I64, [_P]),
    "vxm_weight_cols": (_I64, [_P]),
    "vxm_quantize_q8_0": (_I, [_P, _P, _I64, _I64, _I, _P, _P]),
    "vxm_mul_mat_q8_0": (_I, [_P, _P, _P, _I64, _P]),
    "vxm_mul_mat_q8_0_q8_0": (_I, [_P, _P, _P, _P, _I64, _P]),
    "vxm_mul_mat_q8_0_noalloc": (_I, [_P, _P, _P, _I64, _P]),
    "vxm_noalloc_scratch_bytes": (C.c_size_t, []),
    "vxm_mul_mat_q8_0_q8_0_multi": (_I, [_P, C.c_int32, _P, _P, _P, _I64, _P]),
    "vxm_stream_read": (_I, [_P, C.c_int32, _P, _P, _P]),
    "vxm_stream_read_sink_words": (_I64, [C.c_int32, _P]),
    "vxm_block_dots_q8_0": (_I, [_P, _P, _P, _P, _I64, _P]),
    "vxm_rms_norm": (_I, [_P, _P, _P, _I64, _I64, _F, _P, _P, _P]),
    "vxm_minicpm4_create": (_I, [_P, _P, _P, _P, C.POINTER(_P)]),
    "vxm_minicpm4_free": (_I, [_P]),
    "vxm_kv_cache_create": (_I, [_P, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.POINTER(_P)]),
    "vxm_kv_cache_free": (_I, [_P]),
    "vxm_kv_cache_reset": (_I, [_P]),
    "vxm_kv_cache_set_used": (_I, [_P, C.c_int32]),
    "vxm_kv_cache_used": (C.c_int32, [_P]),
    "vxm_kv_cache_layer": (_I, [_P, C.c_int32, C.POINTER(_P), C.POINTER(_P)]),
    "vxm_minicpm4_block": (_I, [_P, _P, C.c_int32, _P, _I64, C.c_int32, _I]),
    "vxm_minicpm4_forward": (_I, [_P, _P, _P, _I64, C.c_int32]),
    "vxm_minicpm4_set_decode_mode": (_I, [_P, _I]),
    "vxm_minicpm4_check": (_I, [_P]),
    "vxm_minicpm4_set_layer_dump": (_I, [_P, _P]),
    "vxm_minicpm4_set_decode_epoch": (_I, [_P, C.c_uint32]),
    "vxm_minicpm4_decode_epoch": (_I, [_P, C.POINTER(C.c_uint32)]),
    "vxm_locdit_set_block_dump": (_I, [_P, _P]),
    "vxm_locenc_set_block_dump": (_I, [_P, _P]),
    "vxm_host_quantize_q8_0": (_I, [_P, _I64, _I64, _P]),
    "vxm_host_randn": (_I, [_U64, _U64, _I64, _F, _F, _P]),
    "vxm_locdit_create": (_I, [_P, _P, _P, C.POINTER(_P)]),
    "vxm_locdit_free": (_I, [_P]),
    "vxm_locdit_forward": (_I, [_P, _P, _P, C.c_int32, C.c_int32, _F, _F, _P, _P]),
    "vxm_cfm_solve": (_I, [_P, _P, _P, C.c_int32, C.c_int32, _P, C.c_int32, _F, C.c_int32, C.c_int32]),
    "vxm_locdit_set_block_mode": (_I, [_P, _I]),
    "vxm_locdit_check": (_I, [_P]),
    "vxm_host_sinusoid_embed": (_I, [_F, C.c_int32, _P]),
    "vxm_host_cfm_t": (_F, [C.c_int32, C.c_int32, C.c_int32]),
    "vxm_host_cfm_zero_star_steps": (C.c_int32, [C.c_int32]),
    "vxm_host_rope_cache": (_I, [_F, C.c_int32, _P, C.c_int32, C.c_int32, _P]),
    "vxm_locenc_create": (_I, [_P, _P, _P, C.POINTER(_P)]),
    "vxm_locenc_free": (_I, [_P]),
    "vxm_locenc_forward": (_I, [_P, _P, C.c_int32, _P]),
    "vxm_locenc_set_block_mode": (_I, [_P, _I]),
    "vxm_locenc_check": (_I, [_P]),
    "vxm_fsq_quantize": (_I, [_P, _P, _I64, _F, _P]),
    "vxm_lm_update_create": (_I, [_P, _P, _P, _P, _P, _P, C.POINTER(_P)]),
    "vxm_lm_update_free": (_I, [_P]),
    "vxm_lm_update_step": (_I, [_P, _P, _P, _P, C.c_int32, C.c_int32, _P, _P, _P, _P]),
    "vxm_prompt_prefill": (_I, [_P, _P, _P, _P, C.c_int32, C.c_int32, _P]),
    "vxm_embed_rows_q8_0": (_I, [_P, _P, _P, C.c_int32, _P]),
    "vxm_gguf_open": (_I, [C.c_char_p, C.POINTER(_P), C.c_char_p, C.c_size_t]),
    "vxm_gguf_close": (_I, [_P]),
    "vxm_gguf_last_error": (C.c_char_p, [_P]),
    "vxm_gguf_version": (C.c_int32, [_P]),
    "vxm_gguf_n_tensors": (_I64, [_P]),
    "vxm_gguf_find_tensor": (_I64, [_P, C.c_char_p]),
    "vxm_gguf_tensor": (_I, [_P, _I64, _P]),
    "vxm_gguf_get_i32": (C.c_int32, [_P, C.c_char_p, C.c_int32]),
    "vxm_gguf_get_f32": (_F, [_P, C.c_char_p, _F]),
    "vxm_gguf_get_str": (C.c_char_p, [_P, C.c_char_p, C.c_char_p]),
    "vxm_gguf_tensor_f32": (_I, [_P, _I64, _P, _I64]),
    "vxm_gguf_layer_q8_0": (_I, [_P, C.c_char_p, C.c_int32, _I64, _I64, _I64, _I64, _P, _P]),
    "vxm_gguf_minicpm4_config": (_I, [_P, C.c_int32, _P]),
}

CFM_SWAY = 0
CFM_UNIFORM = 1


def header_functions(path=HEADER):
    """Names of every function the public header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vxm_[a-z0-9_]+)\s*\(", text)))


def lib():
    """Load libvxm_q8.so (built in-tree); raise if it is missing."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise VxmError(5, f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(t):
    """Device (or host numpy) pointer of a tensor/array, None for None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return C.c_void_p(t.data_ptr())
    if hasattr(t, "ctypes"):
        return t.ctypes.data_as(C.c_void_p)
    return C.c_void_p(int(t))


class Graph:
    """A recorded sequence of calls on a context (vxm_capture_end)."""

    def __init__(self, ctx, h):
        self.ctx, self.h = ctx, h

    def launch(self):
        self.ctx.check(lib().vxm_graph_launch(self.ctx.h, self.h))

    def free(self):
        if self.h:
            lib().vxm_graph_free(self.h)
            self.h = None


class Context:
    """One device + one stream (vxm_open); closes on ``close()``."""

    def __init__(self, device=0):
        L = lib()
        h = C.c_void_p()
        rc = L.vxm_open(device, C.byref(h))
        if rc:
            raise VxmError(rc, L.vxm_last_error(None).decode())
        self.h = h
        self.device = device
        self._stream = None

    def check(self, rc):
        if rc:
            raise VxmError(rc, lib().vxm_last_error(self.h).decode())

    def close(self):
        if self.h:
            self.check(lib().vxm_close(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def sync(self):
        self.check(lib().vxm_sync(self.h))

    @property
    def stream_handle(self):
        return lib().vxm_get_stream(self.h)

    def torch_stream(self):
        """The context's HIP stream as a torch ExternalStream (for events)."""
        import torch

        if self._stream is None:
            self._stream = torch.cuda.ExternalStream(self.stream_handle, device=f"cuda:{self.device}")
        return self._stream

    def set_quant_variant(self, v):
        self.check(lib().vxm_set_quant_variant(self.h, v))

    # ---- HIP graph capture of the context's stream ----
    def capture_begin(self):
        self.check(lib().vxm_capture_begin(self.h))

    def capture_end(self):
        """End the capture; returns a Graph that replays the recorded calls."""
        h = C.c_void_p()
        self.check(lib().vxm_capture_end(self.h, C.byref(h)))
        return Graph(self, h)

    def set_path(self, p):
        self.check(lib().vxm_set_path(self.h, p))

    # ---- weights ----
    def upload_q8_0(self, gguf_rows, n_rows, k):
        """gguf_rows: host numpy uint8 array of n_rows*(k/32)*34 bytes."""
        import numpy as np

        buf = np.ascontiguousarray(gguf_rows, dtype=np.uint8)
        if buf.size != n_rows * (k // 32) * 34:
            raise VxmError(1, f"expected {n_rows * (k // 32) * 34} bytes, got {buf.size}")
        h = C.c_void_p()
        self.check(lib().vxm_upload_q8_0(self.h, _ptr(buf), n_rows, k, C.byref(h)))
        return Q8Weight(self, h, n_rows, k)

    # ---- ops (device tensors) ----
    def quantize_q8_0(self, x, variant=QUANT_X86, xq=None, xd=None):
        import torch

        M, K = x.shape
        xq = torch.empty((M, K), dtype=torch.int8, device=x.device) if xq is None else xq
        xd = torch.empty((M, K // 32), dtype=torch.int16, device=x.device) if xd is None else xd
        self.check(lib().vxm_quantize_q8_0(self.h, _ptr(x), M, K, variant, _ptr(xq), _ptr(xd)))
        return xq, xd

    def mul_mat(self, w, x, y=None):
        """ggml_mul_mat(W, x): x fp32 [M][K] -> y fp32 [M][N]."""
        import torch

        M = x.shape[0]
        y = torch.empty((M, w.n), dtype=torch.float32, device=x.device) if y is None else y
        self.check(lib().vxm_mul_mat_q8_0(self.h, w.h, _ptr(x), M, _ptr(y)))
        return y

    def mul_mat_noalloc(self, w, x, y):
        """ggml_mul_mat(W, x) through the allocation-free entry: y must be given."""
        self.check(lib().vxm_mul_mat_q8_0_noalloc(self.h, w.h, _ptr(x), x.shape[0], _ptr(y)))
        return y

    def mul_mat_q8_multi(self, ws, xqs, xds, ys):
        """y_i = W_i . x_i for quantized x_i (M rows each, one K) in one launch per 64."""
        n = len(ws)
        M = xqs[0].shape[0] if n else 0

        def arr(ptrs):
            return (C.c_void_p * max(n, 1))(*[p.value for p in ptrs])

        self.check(lib().vxm_mul_mat_q8_0_q8_0_multi(
            self.h, n, arr([C.c_void_p(w.h.value) for w in ws]), arr([_ptr(t) for t in xqs]),
            arr([_ptr(t) for t in xds]), M, arr([_ptr(t) for t in ys])))
        return ys

    def stream_read(self, tensors):
        """Read every tensor once in one launch; returns the device words (one per wave) whose XOR
        is the XOR of all 32-bit words read."""
        import torch

        n = len(tensors)
        ptrs = (C.c_void_p * max(n, 1))(*[_ptr(t).value for t in tensors])
        sizes = (C.c_int64 * max(n, 1))(*[t.numel() * t.element_size() for t in tensors])
        words = lib().vxm_stream_read_sink_words(n, sizes)
        sink = torch.zeros(max(words, 1), dtype=torch.int32, device=f"cuda:{self.device}")
        self.check(lib().vxm_stream_read(self.h, n, ptrs, sizes, _ptr(sink)))
        return sink

    def embed_rows_q8_0(self, table, ids, out=None):
        """Dequantized Q8_0 rows ids (int32 device tensor) of table -> [n][cols] F32."""
        import torch

        n = ids.shape[0]
        out = torch.empty((n, table.k), dtype=torch.float32, device=ids.device) if out is None else out
        self.check(lib().vxm_embed_rows_q8_0(self.h, table.h, _ptr(ids), n, _ptr(out)))
        return out

    def mul_mat_q8(self, w, xq, xd, y=None):
        import torch

        M = xq.shape[0]
        y = torch.empty((M, w.n), dtype=torch.float32, device=xq.device) if y is None else y
        self.check(lib().vxm_mul_mat_q8_0_q8_0(self.h, w.h, _ptr(xq), _ptr(xd), M, _ptr(y)))
        return y

    def rms_norm(self, x, gain, eps, quantize=False):
        """vcpm_rms_norm on device rows; returns y (and Q8_0 (xq, xd) if asked)."""
        import torch

        rows, n = x.shape
        y = torch.empty_like(x)
        xq = xd = None
        if quantize:
            xq = torch.empty((rows, n), dtype=torch.int8, device=x.device)
            xd = torch.empty((rows, n // 32), dtype=torch.int16, device=x.device)
        self.check(lib().vxm_rms_norm(self.h, _ptr(x), _ptr(gain), rows, n, eps, _ptr(y), _ptr(xq), _ptr(xd)))
        return (y, xq, xd) if quantize else y

    def fsq_quantize(self, x, quant_scale, y=None):
        """vcpm_fsq_quantize on a device tensor: round(tanh(x) * s) / s."""
        import torch

        if y is None:
            y = torch.empty_like(x)
        self.check(lib().vxm_fsq_quantize(self.h, _ptr(x), x.numel(), quant_scale, _ptr(y)))
        return y

    def block_dots(self, w, xq, xd):
        import torch

        M = xq.shape[0]
        out = torch.empty((M, w.n, w.k // 32), dtype=torch.int32, device=xq.device)
        self.check(lib().vxm_block_dots_q8_0(self.h, w.h, _ptr(xq), _ptr(xd), M, _ptr(out)))
        return out


class MiniCPM4Config(C.Structure):
    """Mirror of vxm_minicpm4_config (vcpm_minicpm4_config, src/minicpm4.h:14-27)."""

    _fields_ = [
        ("hidden_size", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("intermediate_size", C.c_int32), ("head_dim", C.c_int32),
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_int32), ("no_rope", C.c_int32),
        ("scale_depth", C.c_float), ("rope_freq_factors", C.c_void_p),
    ]


class LayerWeightsQ8(C.Structure):
    """Mirror of vxm_layer_weights_q8_0 (host pointers)."""

    _fields_ = [(n, C.c_void_p) for n in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj",
                                          "down_proj", "input_layernorm", "post_attention_layernorm")]


class KVCache:
    """f16 KV cache: per layer K, V [n_kv_heads][capacity][head_dim]."""

    def __init__(self, ctx, n_layers, n_kv_heads, head_dim, capacity):
        h = C.c_void_p()
        ctx.check(lib().vxm_kv_cache_create(ctx.h, n_layers, n_kv_heads, head_dim, capacity, C.byref(h)))
        self.ctx, self.h = ctx, h
        self.n_layers, self.nkv, self.hd, self.cap = n_layers, n_kv_heads, head_dim, capacity

    def layer(self, l):
        k, v = C.c_void_p(), C.c_void_p()
        self.ctx.check(lib().vxm_kv_cache_layer(self.h, l, C.byref(k), C.byref(v)))
        return k.value, v.value

    def upload(self, l, k_host, v_host):
        """Copy host f16 bits [nkv][cap][hd] into layer l (a host-boundary copy)."""
        import numpy as np

        k, v = self.layer(l)
        n = self.nkv * self.cap * self.hd * 2
        for dst, src in ((k, k_host), (v, v_host)):
            a = np.ascontiguousarray(src, dtype=np.uint16)
            assert a.nbytes == n
            self.ctx.check(lib().vxm_memcpy_h2d(self.ctx.h, C.c_void_p(dst), _ptr(a), n))

    def download(self, l):
        import numpy as np

        k, v = self.layer(l)
        out = []
        for src in (k, v):
            a = np.empty((self.nkv, self.cap, self.hd), dtype=np.uint16)
            self.ctx.check(lib().vxm_memcpy_d2h(self.ctx.h, _ptr(a), C.c_void_p(src), a.nbytes))
            out.append(a)
        return out

    @property
    def used(self):
        return lib().vxm_kv_cache_used(self.h)

    def set_used(self, n):
        self.ctx.check(lib().vxm_kv_cache_set_used(self.h, n))

    def reset(self):
        self.ctx.check(lib().vxm_kv_cache_reset(self.h))

    def free(self):
        if self.h:
            self.ctx.check(lib().vxm_kv_cache_free(self.h))
            self.h = None


class MiniCPM4:
    """vcpm_minicpm4 on the device: n_layers blocks of GGUF Q8_0 weights."""

    def __init__(self, ctx, cfg: dict, layers, final_norm=None):
        import numpy as np

        self.ctx = ctx
        self._keep = []
        ff = cfg.get("rope_freq_factors")
        if ff is not None:
            ff = np.ascontiguousarray(ff, dtype=np.float32)
            self._keep.append(ff)
        c = MiniCPM4Config(cfg["hidden_size"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                           cfg["intermediate_size"], cfg["head_dim"], cfg.get("rms_norm_eps", 1e-6),
                           int(cfg.get("rope_theta", 10000)), int(cfg.get("no_rope", 0)),
                           float(cfg.get("scale_depth", 0.0)), None if ff is None else ff.ctypes.data)
        self.cfg = cfg
        arr = (LayerWeightsQ8 * len(layers))()
        names = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj",
                 "input_layernorm", "post_attention_layernorm")
        for i, lw in enumerate(layers):
            if isinstance(lw, LayerWeightsQ8):   # pointers already set (e.g. into a GGUF mapping)
                arr[i] = lw
                continue
            for n in names:
                a = np.ascontiguousarray(lw[n])
                self._keep.append(a)
                setattr(arr[i], n, a.ctypes.data)
        fn = None
        if final_norm is not None:
            fn = np.ascontiguousarray(final_norm, dtype=np.float32)
            self._keep.append(fn)
        h = C.c_void_p()
        ctx.check(lib().vxm_minicpm4_create(ctx.h, C.byref(c), C.cast(arr, C.c_void_p),
                                            None if fn is None else fn.ctypes.data_as(C.c_void_p), C.byref(h)))
        self.h = h
        self._keep = []

    def block(self, kv, layer, x, pos, no_causal=0):
        """In place on x (fp32 [n_tokens][hidden] device tensor)."""
        self.ctx.check(lib().vxm_minicpm4_block(self.h, None if kv is None else kv.h, layer, _ptr(x), x.shape[0],
                                                pos, no_causal))
        return x

    def set_decode_mode(self, mode):
        """0 auto, 1 one kernel per op, 2 persistent whole-stack launch."""
        self.ctx.check(lib().vxm_minicpm4_set_decode_mode(self.h, mode))

    def check(self):
        """Sync and raise if a persistent decode launch failed on the device."""
        self.ctx.check(lib().vxm_minicpm4_check(self.h))

    def set_layer_dump(self, dump):
        """Debug: every forward writes each layer's input and the last layer's output
        (before the final norm) to dump, fp32 [n_layers + 1][n_tokens][hidden]; None: off."""
        self.ctx.check(lib().vxm_minicpm4_set_layer_dump(self.h, _ptr(dump)))

    def set_decode_epoch(self, epoch):
        """Test hook: the tag epoch of the next single-launch decode (1 .. 2^20 - 1)."""
        self.ctx.check(lib().vxm_minicpm4_set_decode_epoch(self.h, epoch))

    def decode_epoch(self):
        e = C.c_uint32()
        self.ctx.check(lib().vxm_minicpm4_decode_epoch(self.h, C.byref(e)))
        return e.value

    def forward(self, kv, x, pos):
        self.ctx.check(lib().vxm_minicpm4_forward(self.h, kv.h, _ptr(x), x.shape[0], pos))
        return x

    def free(self):
        if self.h:
            self.ctx.check(lib().vxm_minicpm4_free(self.h))
            self.h = None


class LocDiTConfig(C.Structure):
    """Mirror of vxm_locdit_config (vcpm_locdit_config, src/locdit.h:26-34)."""

    _fields_ = [
        ("hidden_size", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("intermediate_size", C.c_int32), ("head_dim", C.c_int32),
        ("feat_dim", C.c_int32), ("cond_dim", C.c_int32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_int32), ("rope_freq_factors", C.c_void_p),
    ]


LOCDIT_TENSORS = ("in_proj", "in_bias", "cond_proj", "cond_bias", "out_proj", "out_bias", "norm",
                  "t_w1", "t_w2", "dt_w1", "dt_w2", "t_b1", "t_b2", "dt_b1", "dt_b2")


class LocDiTWeightsQ8(C.Structure):
    """Mirror of vxm_locdit_weights_q8_0 (vcpm_locdit_weights, src/locdit.h:41-68)."""

    _fields_ = [("layers", C.c_void_p)] + [(n, C.c_void_p) for n in LOCDIT_TENSORS]


class LocDiT:
    """vcpm_locdit on the device, plus the CFM solver that drives it.

    ``weights``: dict with GGUF Q8_0 rows for in_proj [hidden][feat], cond_proj
    [hidden][cond], out_proj [feat][hidden], t_w1/t_w2/dt_w1/dt_w2 [hidden][hidden],
    F32 biases / norm (biases may be None) and ``layers`` (MiniCPM4 block dicts)."""

    def __init__(self, ctx, cfg: dict, weights: dict):
        import numpy as np

        self.ctx = ctx
        keep = []
        ff = cfg.get("rope_freq_factors")
        if ff is not None:
            ff = np.ascontiguousarray(ff, dtype=np.float32)
            keep.append(ff)
        c = LocDiTConfig(cfg["hidden_size"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                         cfg["intermediate_size"], cfg["head_dim"], cfg["feat_dim"], cfg.get("cond_dim", cfg["feat_dim"]),
                         cfg.get("rms_norm_eps", 1e-6), int(cfg.get("rope_theta", 10000)),
                         None if ff is None else ff.ctypes.data)
        self.cfg = cfg
        layers = weights.get("layers", [])
        arr = (LayerWeightsQ8 * max(1, len(layers)))()
        names = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj",
                 "input_layernorm", "post_attention_layernorm")
        for i, lw in enumerate(layers):
            for n in names:
                a = np.ascontiguousarray(lw[n])
                keep.append(a)
                setattr(arr[i], n, a.ctypes.data)
        w = LocDiTWeightsQ8()
        w.layers = C.cast(arr, C.c_void_p).value
        for n in LOCDIT_TENSORS:
            v = weights.get(n)
            if v is not None:
                a = np.ascontiguousarray(v)
                keep.append(a)
                setattr(w, n, a.ctypes.data)
        h = C.c_void_p()
        ctx.check(lib().vxm_locdit_create(ctx.h, C.byref(c), C.byref(w), C.byref(h)))
        self.h = h

    def forward(self, x, cond, t, dt=0.0, mu=None, out=None):
        """Velocity [P][feat] of x [P][feat] (device tensors); mu [2][hidden] or None."""
        import torch

        P = x.shape[0]
        Pc = 0 if cond is None else cond.shape[0]
        if out is None:
            out = torch.empty((P, self.cfg["feat_dim"]), dtype=torch.float32, device=x.device)
        self.ctx.check(lib().vxm_locdit_forward(self.h, _ptr(x), _ptr(cond), P, Pc, t, dt, _ptr(mu), _ptr(out)))
        return out

    def cfm_solve(self, x, cond, mu, n_steps, cfg_value=2.0, schedule=CFM_SWAY, use_zero_star=True):
        """The Euler loop, in place on x [P][feat] (device tensor)."""
        P = x.shape[0]
        Pc = 0 if cond is None else cond.shape[0]
        self.ctx.check(lib().vxm_cfm_solve(self.h, _ptr(x), _ptr(cond), P, Pc, _ptr(mu), n_steps, cfg_value,
                                           schedule, int(use_zero_star)))
        return x

    def set_block_mode(self, mode):
        """DECODE_AUTO / DECODE_KERNELS / DECODE_PERSISTENT: how the blocks of an evaluation launch."""
        self.ctx.check(lib().vxm_locdit_set_block_mode(self.h, mode))

    def check(self):
        """Synchronise; raise if a persistent block launch timed out on the device."""
        self.ctx.check(lib().vxm_locdit_check(self.h))

    def set_block_dump(self, dump):
        """Debug: each evaluation writes the rows entering every block and the last block's
        output to dump, fp32 [n_layers + 1][rows][hidden]; None: off."""
        self.ctx.check(lib().vxm_locdit_set_block_dump(self.h, _ptr(dump)))

    def free(self):
        if self.h:
            self.ctx.check(lib().vxm_locdit_free(self.h))
            self.h = None


class Q8Weight:
    def __init__(self, ctx, h, n, k):
        self.ctx, self.h, self.n, self.k = ctx, h, n, k

    def download(self):
        import numpy as np

        out = np.empty(self.n * (self.k // 32) * 34, dtype=np.uint8)
        self.ctx.check(lib().vxm_download_q8_0(self.ctx.h, self.h, _ptr(out)))
        return out

    def free(self):
        if self.h:
            self.ctx.check(lib().vxm_weight_free(self.ctx.h, self.h))
            self.h = None


# ---- host helpers (no device work) ----

def host_randn(seed, n, mean=0.0, std=1.0, offset=0):
    import numpy as np

    out = np.empty(n, dtype=np.float32)
    rc = lib().vxm_host_randn(seed, offset, n, mean, std, _ptr(out))
    if rc:
        raise VxmError(rc, "vxm_host_randn")
    return out


def host_quantize_q8_0(x):
    """GGUF Q8_0 rows of a float32 [rows][k] array (weight rule)."""
    import numpy as np

    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    out = np.empty(rows * (k // 32) * 34, dtype=np.uint8)
    rc = lib().vxm_host_quantize_q8_0(_ptr(x), rows, k, _ptr(out))
    if rc:
        raise VxmError(rc, "vxm_host_quantize_q8_0")
    return out


def host_sinusoid_embed(t, dim):
    import numpy as np

    out = np.empty(dim, dtype=np.float32)
    rc = lib().vxm_host_sinusoid_embed(t, dim, _ptr(out))
    if rc:
        raise VxmError(rc, "vxm_host_sinusoid_embed")
    return out


def host_cfm_t(step, n_steps, schedule=CFM_SWAY):
    return lib().vxm_host_cfm_t(step, n_steps, schedule)


def host_cfm_zero_star_steps(n_steps):
    return lib().vxm_host_cfm_zero_star_steps(n_steps)


def host_rope_cache(base, head_dim, ff, pos0, n_pos):
    """(cos, sin) rope table [n_pos][head_dim/2][2] of ggml_rope_ext's NEOX angles."""
    import numpy as np

    out = np.empty((n_pos, head_dim // 2, 2), dtype=np.float32)
    ffa = None if ff is None else np.ascontiguousarray(ff, dtype=np.float32)
    rc = lib().vxm_host_rope_cache(base, head_dim, _ptr(ffa), pos0, n_pos, _ptr(out))
    if rc:
        raise VxmError(rc, "vxm_host_rope_cache")
    return out


class LocEncConfig(C.Structure):
    """Mirror of vxm_locenc_config (vcpm_locenc_config, src/locenc.h:49-60)."""

    _fields_ = [
        ("hidden_size", C.c_int32), ("n_layers", C.c_int32), ("n_heads", C.c_int32),
        ("n_kv_heads", C.c_int32), ("intermediate_size", C.c_int32), ("head_dim", C.c_int32),
        ("feat_dim", C.c_int32), ("rms_norm_eps", C.c_float), ("rope_theta", C.c_int32),
        ("rope_freq_factors", C.c_void_p),
    ]


LOCENC_TENSORS = ("in_proj", "in_bias", "special_token", "norm")


class LocEncWeightsQ8(C.Structure):
    """Mirror of vxm_locenc_weights_q8_0 (vcpm_locenc_weights, src/locenc.h:67-73)."""

    _fields_ = [("layers", C.c_void_p)] + [(n, C.c_void_p) for n in LOCENC_TENSORS]


def _layer_array(layers, keep):
    import numpy as np

    arr = (LayerWeightsQ8 * max(1, len(layers)))()
    names = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj",
             "input_layernorm", "post_attention_layernorm")
    for i, lw in enumerate(layers):
        for n in names:
            a = np.ascontiguousarray(lw[n])
            keep.append(a)
            setattr(arr[i], n, a.ctypes.data)
    keep.append(arr)
    return C.cast(arr, C.c_void_p).value


class LocEnc:
    """vcpm_locenc (the feature encoder) on the device.

    ``weights``: in_proj GGUF Q8_0 rows [hidden][feat], F32 in_bias / special_token /
    norm (in_bias and special_token may be None) and ``layers`` (MiniCPM4 block dicts)."""

    def __init__(self, ctx, cfg: dict, weights: dict):
        import numpy as np

        self.ctx = ctx
        keep = []
        ff = cfg.get("rope_freq_factors")
        if ff is not None:
            ff = np.ascontiguousarray(ff, dtype=np.float32)
            keep.append(ff)
        c = LocEncConfig(cfg["hidden_size"], cfg["n_layers"], cfg["n_heads"], cfg["n_kv_heads"],
                         cfg["intermediate_size"], cfg["head_dim"], cfg["feat_dim"], cfg.get("rms_norm_eps", 1e-6),
                         int(cfg.get("rope_theta", 10000)), None if ff is None else ff.ctypes.data)
        self.cfg = cfg
        self.has_special = weights.get("special_token") is not None
        w = LocEncWeightsQ8()
        w.layers = _layer_array(weights.get("layers", []), keep)
        for n in LOCENC_TENSORS:
            v = weights.get(n)
            if v is not None:
                a = np.ascontiguousarray(v)
                keep.append(a)
                setattr(w, n, a.ctypes.data)
        h = C.c_void_p()
        ctx.check(lib().vxm_locenc_create(ctx.h, C.byref(c), C.byref(w), C.byref(h)))
        self.h = h

    def forward(self, x, out=None):
        """x [P][feat] device tensor -> [hidden] (special-token row) or [P][hidden]."""
        import torch

        P, H = x.shape[0], self.cfg["hidden_size"]
        if out is None:
            shape = (H,) if self.has_special else (P, H)
            out = torch.empty(shape, dtype=torch.float32, device=x.device)
        self.ctx.check(lib().vxm_locenc_forward(self.h, _ptr(x), P, _ptr(out)))
        return out

    def set_block_mode(self, mode):
        """DECODE_AUTO / DECODE_KERNELS / DECODE_PERSISTENT: how the blocks launch."""
        self.ctx.check(lib().vxm_locenc_set_block_mode(self.h, mode))

    def check(self):
        """Synchronise; raise if a persistent block launch timed out on the device."""
        self.ctx.check(lib().vxm_locenc_check(self.h))

    def set_block_dump(self, dump):
        """Debug: as LocDiT.set_block_dump for the P + 1 encoder rows."""
        self.ctx.check(lib().vxm_locenc_set_block_dump(self.h, _ptr(dump)))

    def free(self):
        if self.h:
            self.ctx.check(lib().vxm_locenc_free(self.h))
            self.h = None


class LMUpdateConfig(C.Structure):
    """Mirror of vxm_lm_update_config."""

    _fields_ = [("lm_hidden", C.c_int32), ("enc_hidden", C.c_int32), ("fsq_dim", C.c_int32),
                ("res_hidden", C.c_int32), ("fsq_quant_scale", C.c_float)]


LM_UPDATE_TENSORS = ("enc_to_lm", "enc_to_lm_bias", "fsq_in", "fsq_in_bias", "fsq_out", "fsq_out_bias",
                     "fusion_concat")


class LMUpdateWeightsQ8(C.Structure):
    """Mirror of vxm_lm_update_weights_q8_0."""

    _fields_ = [(n, C.c_void_p) for n in LM_UPDATE_TENSORS]


class LMUpdate:
    """gen_lm_update on the device: LocEnc -> enc_to_lm -> TSLM step -> FSQ -> fusion -> RALM step.
    Borrows enc / tslm / ralm (keeps Python references to them)."""

    def __init__(self, ctx, cfg: dict, weights: dict, enc, tslm, ralm):
        import numpy as np

        self.ctx, self.cfg = ctx, cfg
        self._owners = (enc, tslm, ralm)
        keep = []
        w = LMUpdateWeightsQ8()
        for n in LM_UPDATE_TENSORS:
            v = weights.get(n)
            if v is not None:
                a = np.ascontiguousarray(v)
                keep.append(a)
                setattr(w, n, a.ctypes.data)
        c = LMUpdateConfig(cfg["lm_hidden"], cfg["enc_hidden"], cfg.get("fsq_dim", 0), cfg["res_hidden"],
                           cfg.get("fsq_quant_scale", 9.0))
        h = C.c_void_p()
        ctx.check(lib().vxm_lm_update_create(ctx.h, C.byref(c), C.byref(w), enc.h, tslm.h, ralm.h, C.byref(h)))
        self.h = h

    def step(self, tslm_kv, ralm_kv, prev_patch, pos, audio_embed=None, base_hidden=None, fsq=None,
             ralm_hidden=None):
        """Returns (audio_embed, base_hidden, fsq, ralm_hidden) device tensors."""
        import torch

        dev = prev_patch.device
        L, R = self.cfg["lm_hidden"], self.cfg["res_hidden"]

        def new(t, n):
            return torch.empty(n, dtype=torch.float32, device=dev) if t is None else t

        audio_embed, base_hidden, fsq, ralm_hidden = (new(audio_embed, L), new(base_hidden, L), new(fsq, L),
                                                      new(ralm_hidden, R))
        self.ctx.check(lib().vxm_lm_update_step(self.h, tslm_kv.h, ralm_kv.h, _ptr(prev_patch), prev_patch.shape[0],
                                                pos, _ptr(audio_embed), _ptr(base_hidden), _ptr(fsq),
                                                _ptr(ralm_hidden)))
        return audio_embed, base_hidden, fsq, ralm_hidden

    def prompt_prefill(self, tslm_kv, ralm_kv, x, pos, ralm_hidden=None):
        """gen_prompt_eval_range: x [n][lm_hidden] text embeddings (device) -> base_hidden in place;
        returns (x, ralm_hidden [n][res_hidden])."""
        import torch

        n = x.shape[0]
        if ralm_hidden is None:
            ralm_hidden = torch.empty((n, self.cfg["res_hidden"]), dtype=torch.float32, device=x.device)
        self.ctx.check(lib().vxm_prompt_prefill(self.h, tslm_kv.h, ralm_kv.h, _ptr(x), n, pos, _ptr(ralm_hidden)))
        return x, ralm_hidden

    def free(self):
        if self.h:
            self.ctx.check(lib().vxm_lm_update_free(self.h))
            self.h = None


GGML_F32, GGML_F16, GGML_Q8_0, GGML_BF16 = 0, 1, 8, 30


class GGUFTensorInfo(C.Structure):
    """Mirror of vxm_gguf_tensor_info."""

    _fields_ = [("name", C.c_char_p), ("type", C.c_int32), ("n_dims", C.c_int32), ("ne", C.c_int64 * 4),
                ("n_elements", C.c_int64), ("offset", C.c_uint64), ("data", C.c_void_p), ("nbytes", C.c_uint64)]


class GGUF:
    """A memory-mapped GGUF file (host only): tensors by name as numpy views, metadata getters, F32
    copies and per-block Q8_0 weights as the reference names them."""

    def __init__(self, path):
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        rc = lib().vxm_gguf_open(str(path).encode(), C.byref(h), err, len(err))
        if rc:
            raise VxmError(rc, err.value.decode())
        self.h = h
        self._norms = []

    def close(self):
        if self.h:
            lib().vxm_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc):
        if rc:
            raise VxmError(rc, (lib().vxm_gguf_last_error(self.h) or b"").decode())

    @property
    def version(self):
        return lib().vxm_gguf_version(self.h)

    def __len__(self):
        return lib().vxm_gguf_n_tensors(self.h)

    def find(self, name):
        return lib().vxm_gguf_find_tensor(self.h, name.encode())

    def info(self, idx_or_name):
        idx = self.find(idx_or_name) if isinstance(idx_or_name, str) else idx_or_name
        if idx < 0:
            raise KeyError(idx_or_name)
        ti = GGUFTensorInfo()
        self._check(lib().vxm_gguf_tensor(self.h, idx, C.byref(ti)))
        return ti

    def raw(self, name):
        """The tensor's bytes (a copy) as uint8."""
        import numpy as np

        ti = self.info(name)
        return np.ctypeslib.as_array((C.c_uint8 * ti.nbytes).from_address(ti.data)).copy()

    def f32(self, name):
        import numpy as np

        idx = self.find(name)
        if idx < 0:
            raise KeyError(name)
        ti = self.info(idx)
        out = np.empty(ti.n_elements, dtype=np.float32)
        self._check(lib().vxm_gguf_tensor_f32(self.h, idx, out.ctypes.data_as(C.c_void_p), out.size))
        return out

    def get_i32(self, key, default=0):
        return lib().vxm_gguf_get_i32(self.h, key.encode(), default)

    def get_f32(self, key, default=0.0):
        return lib().vxm_gguf_get_f32(self.h, key.encode(), default)

    def get_str(self, key, default=None):
        v = lib().vxm_gguf_get_str(self.h, key.encode(), None if default is None else default.encode())
        return None if v is None else v.decode()

    def layer_q8_0(self, prefix, layer, cfg):
        """LayerWeightsQ8 pointing into the mapping; the F32 norms live as long as this object.
        cfg: a MiniCPM4 config dict (hidden_size, n_heads, n_kv_heads, head_dim,
        intermediate_size); every projection's shape is checked against it."""
        import numpy as np

        hidden = cfg["hidden_size"]
        norms = np.empty(2 * hidden, dtype=np.float32)
        self._norms.append(norms)
        w = LayerWeightsQ8()
        self._check(lib().vxm_gguf_layer_q8_0(self.h, prefix.encode(), layer, hidden,
                                              cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"],
                                              cfg["intermediate_size"], norms.ctypes.data_as(C.c_void_p),
                                              C.byref(w)))
        return w

    def minicpm4_config(self, residual=False):
        c = MiniCPM4Config()
        self._check(lib().vxm_gguf_minicpm4_config(self.h, int(residual), C.byref(c)))
        return {f: getattr(c, f) for f, _ in MiniCPM4Config._fields_}
