"""ctypes binding of the oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

The oracle restates gemma4-rs's CPU attention path in C (g4_oracle.c).  It is
what results are compared against: only the test suite, the smoke check and
the CPU-baseline leg of the benchmark load it.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# G4_ORACLE_LIB selects a rebuilt variant (the planted-mistake test uses it).
LIB_PATH = os.environ.get("G4_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

OR_OK = 0
OR_ERR_COMPUTE = 1
OR_ERR_CONTEXT_TOO_LONG = 2
OR_ERR_MISSING_LAYER = 3
OR_ERR_KV_LAYER_OUT_OF_RANGE = 10
OR_ERR_KV_TOO_MANY_SHARED = 11
OR_ERR_KV_NO_EARLIER_SAME_KIND = 12

_lib = None
c_size = ctypes.c_size_t
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p
P_f32 = ctypes.POINTER(ctypes.c_float)


class OracleError(RuntimeError):
    def __init__(self, code, message):
        self.code = code
        self.message = message
        super().__init__(f"oracle status {code}: {message}")


class Hparams(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_size), ("n_heads", c_size), ("n_kv_heads", c_size), ("head_dim_local", c_size),
        ("head_dim_global", c_size), ("sliding_window", c_size), ("shared_kv_layers", c_size),
        ("local_rope_base", c_f32), ("global_rope_base", c_f32), ("rms_norm_eps", c_f32),
    ]

    @classmethod
    def e2b(cls):
        return cls(35, 8, 1, 256, 512, 512, 20, 10000.0, 1000000.0, 1e-6)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "or_last_error": (ctypes.c_char_p, []),
            "or_dot_f32": (c_f32, [c_vp, c_vp, c_size]),
            "or_softmax_f32": (ctypes.c_int, [c_vp, c_size, c_vp]),
            "or_rms_norm": (ctypes.c_int, [c_vp, c_size, c_vp, c_size, c_f32, c_vp]),
            "or_rope_neox": (ctypes.c_int, [c_vp, c_size, c_size, c_f32, c_size, c_vp, c_size]),
            "or_attend_head": (ctypes.c_int, [c_vp, c_vp, c_vp, c_size, c_size, c_size, c_size, c_size, c_f32,
                                              c_size, c_vp]),
            "or_attend": (ctypes.c_int, [c_vp, c_size, c_vp, c_vp, c_size, c_size, c_size, c_f32, c_vp]),
            "or_attend_rows": (ctypes.c_int, [c_vp, c_size, c_vp, c_vp, c_size, c_size, c_size, c_f32, c_size,
                                              c_vp]),
            "or_attend_prefill": (ctypes.c_int, [c_vp, c_size, c_size, c_vp, c_vp, c_size, c_size, c_size, c_size,
                                                 c_f32, c_size, c_vp, c_vp]),
            "or_attend_prefill_blocked": (ctypes.c_int, [c_vp, c_size, c_size, c_vp, c_vp, c_vp, c_size, c_size,
                                                         c_size, c_size, c_f32, c_size, c_vp, c_vp]),
            "or_attend_f64": (ctypes.c_int, [c_vp, c_size, c_vp, c_vp, c_size, c_size, c_size, ctypes.c_double,
                                             c_vp]),
            "or_norm_heads": (ctypes.c_int, [c_vp, c_size, c_size, c_vp, c_f32]),
            "or_rope_heads": (ctypes.c_int, [c_vp, c_size, c_size, c_size, c_f32, c_vp, c_size]),
            "or_layer_attention_kind": (ctypes.c_int, [c_size, c_size]),
            "or_head_dim": (c_size, [c_size, c_size, c_size, c_size]),
            "or_proportional_rope_freq_factors": (None, [c_size, c_f32, c_vp]),
            "or_windowed_len": (None, [c_size, c_size, ctypes.POINTER(c_size), ctypes.POINTER(c_size)]),
            "or_kv_source_layer": (ctypes.c_int, [c_size, c_size, c_size, ctypes.POINTER(c_size)]),
            "or_kv_new": (c_vp, []),
            "or_kv_free": (None, [c_vp]),
            "or_kv_append": (ctypes.c_int, [c_vp, c_size, c_vp, c_vp, c_size]),
            "or_kv_view": (ctypes.c_int, [c_vp, c_size, c_size, ctypes.POINTER(c_vp), ctypes.POINTER(c_vp),
                                          ctypes.POINTER(c_size)]),
            "or_kv_clear": (None, [c_vp]),
            "or_layer_attention": (ctypes.c_int, [c_vp, ctypes.POINTER(Hparams), c_size, c_size, c_vp, c_vp, c_vp,
                                                  c_vp, c_vp, c_vp, c_size, c_vp, ctypes.POINTER(c_size),
                                                  ctypes.POINTER(c_size), ctypes.POINTER(c_size)]),
            "or_pool_threads": (c_size, []),
            "or_f16_to_f32": (c_f32, [ctypes.c_uint16]),
            "or_f32_to_f16": (ctypes.c_uint16, [c_f32]),
            "or_bf16_to_f32": (c_f32, [ctypes.c_uint16]),
            "or_f32_to_bf16": (ctypes.c_uint16, [c_f32]),
            "or_quantize_q8_0": (ctypes.c_int, [c_vp, c_size, c_vp, c_vp]),
            "or_dequant_q8_0": (ctypes.c_int, [c_vp, c_size, c_vp]),
            "or_matvec_q8_0": (ctypes.c_int, [c_vp, c_size, c_size, c_size, c_vp, c_vp, c_vp]),
            "or_matvec_q8_0_softcap": (ctypes.c_int, [c_vp, c_size, c_size, c_size, c_vp, c_vp, c_f32, c_vp]),
            "or_geglu_q8_0": (ctypes.c_int, [c_vp, c_vp, c_size, c_size, c_size, c_vp, c_vp, ctypes.c_int, c_vp]),
            "or_matvec_q8_0_f32": (ctypes.c_int, [c_vp, c_size, c_size, c_size, c_vp, ctypes.c_int, c_vp]),
            "or_matvec_bf16": (ctypes.c_int, [c_vp, c_size, c_size, c_size, c_vp, c_vp]),
            "or_matvec_f32": (ctypes.c_int, [c_vp, c_size, c_size, c_size, c_vp, c_vp]),
            "or_softcap": (c_f32, [c_f32, c_f32]),
            "or_gelu_tanh": (c_f32, [c_f32]),
            "or_gelu_tanh_fp16_table": (c_f32, [c_f32]),
            "or_prepare_rows": (ctypes.c_int, [c_vp, c_size, c_size, c_size, c_vp, c_f32, c_size, c_f32, c_vp,
                                               c_size]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(rc):
    if rc != OR_OK:
        raise OracleError(rc, lib().or_last_error().decode())


def dot_f32(a, b):
    a, b = _f32(a), _f32(b)
    return lib().or_dot_f32(a.ctypes.data, b.ctypes.data, a.size)


def softmax_f32(x):
    x = _f32(x)
    out = np.empty_like(x)
    _check(lib().or_softmax_f32(x.ctypes.data, x.size, out.ctypes.data))
    return out


def rms_norm(x, weight, eps):
    x = _f32(x)
    out = np.empty_like(x)
    w = None if weight is None else _f32(weight)
    _check(lib().or_rms_norm(x.ctypes.data, x.size, None if w is None else w.ctypes.data,
                             0 if w is None else w.size, eps, out.ctypes.data))
    return out


def rope_neox(x, position, base, n_rot, freq_factors=None):
    x = _f32(x).copy()
    f = None if freq_factors is None else _f32(freq_factors)
    _check(lib().or_rope_neox(x.ctypes.data, x.size, position, base, n_rot,
                              None if f is None else f.ctypes.data, 0 if f is None else f.size))
    return x


def norm_heads(x, head_dim, weight, eps):
    x = _f32(x).copy()
    w = None if weight is None else _f32(weight)
    _check(lib().or_norm_heads(x.ctypes.data, x.size, head_dim, None if w is None else w.ctypes.data, eps))
    return x


def rope_heads(x, head_dim, position, base, freq_factors=None):
    x = _f32(x).copy()
    f = None if freq_factors is None else _f32(freq_factors)
    _check(lib().or_rope_heads(x.ctypes.data, x.size, head_dim, position, base,
                               None if f is None else f.ctypes.data, 0 if f is None else f.size))
    return x


def attend(q, keys, values, n_heads, n_kv_heads, scale=1.0):
    """attend over a contiguous [T][n_kv*head_dim] image (model.rs:348-366)."""
    q, keys, values = _f32(q), _f32(keys), _f32(values)
    head_dim = q.size // n_heads
    T = keys.size // (n_kv_heads * head_dim) if head_dim else 0
    out = np.zeros(q.size, dtype=np.float32)
    _check(lib().or_attend(q.ctypes.data, q.size, keys.ctypes.data, values.ctypes.data, T, n_heads, n_kv_heads,
                           scale, out.ctypes.data))
    return out


def attend_rows(q, keys, values, n_heads, n_kv_heads, scale=1.0, threads=0):
    """attend with the reference's per-row `concat` copy and head pool."""
    q, keys, values = _f32(q), _f32(keys), _f32(values)
    T = keys.shape[0]
    kr = (c_vp * T)(*[keys[t].ctypes.data for t in range(T)])
    vr = (c_vp * T)(*[values[t].ctypes.data for t in range(T)])
    out = np.zeros(q.size, dtype=np.float32)
    _check(lib().or_attend_rows(q.ctypes.data, q.size, kr, vr, T, n_heads, n_kv_heads, scale, threads,
                                out.ctypes.data))
    return out


def attend_prefill(q, keys, values, pos0, window, n_heads, n_kv_heads, scale=1.0, threads=None, blocked=True,
                   positions=None):
    """The token-at-a-time prompt loop (generate.rs:37-41): row i of q
    [N, n_heads*head_dim] at position pos0 + i attends rows [b, pos0+i+1) of
    the contiguous keys/values image (row t = position t; b from the window,
    0 = global).  Returns (out [N, q_len], status [N]): status[i] is 0 or the
    oracle's error code for that query; queries run on `threads` OS threads
    (default: all CPUs).  blocked: the same arithmetic with groups of queries
    walking the keys together (or_attend_prefill_blocked, bit-identical to
    the plain loop and faster on long contexts).  positions: the rows of q
    are queries at these positions instead of pos0 + i (a sample of a
    chunk; blocked form only)."""
    q, keys, values = _f32(q), _f32(keys), _f32(values)
    N, q_len = q.shape
    last = int(np.max(positions)) + 1 if positions is not None and N else pos0 + N
    if keys.shape[0] < last or values.shape[0] < last:
        raise ValueError("keys/values must hold rows up to the last query's position")
    threads = threads or os.cpu_count() or 1
    out = np.zeros((N, q_len), dtype=np.float32)
    status = np.zeros(N, dtype=np.int32)
    if positions is not None or (blocked and n_heads <= 64):
        pos = None if positions is None else np.ascontiguousarray(positions, dtype=np.uint64)
        if pos is not None and pos.shape != (N,):
            raise ValueError("one position per query row")
        lib().or_attend_prefill_blocked(q.ctypes.data, q_len, N, None if pos is None else pos.ctypes.data,
                                        keys.ctypes.data, values.ctypes.data, pos0, window, n_heads, n_kv_heads,
                                        scale, threads, status.ctypes.data, out.ctypes.data)
    else:
        lib().or_attend_prefill(q.ctypes.data, q_len, N, keys.ctypes.data, values.ctypes.data, pos0, window,
                                n_heads, n_kv_heads, scale, threads, status.ctypes.data, out.ctypes.data)
    return out, status


class RowPointers:
    """Row pointer arrays for or_attend_rows over a large contiguous cache,
    built once so that timing loops measure only the attention call."""

    def __init__(self, keys, values):
        self.keys, self.values = keys, values
        T, w = keys.shape
        kb, vb = keys.ctypes.data, values.ctypes.data
        self.k = (c_vp * T)(*[kb + 4 * w * t for t in range(T)])
        self.v = (c_vp * T)(*[vb + 4 * w * t for t in range(T)])
        self.T = T

    def attend(self, q, begin, end, n_heads, n_kv_heads, out, scale=1.0, threads=0):
        kp = ctypes.cast(ctypes.byref(self.k, 8 * begin), ctypes.c_void_p)
        vp = ctypes.cast(ctypes.byref(self.v, 8 * begin), ctypes.c_void_p)
        _check(lib().or_attend_rows(q.ctypes.data, q.size, kp, vp, end - begin, n_heads, n_kv_heads, scale,
                                    threads, out.ctypes.data))
        return out


def attend_f64(q, keys, values, n_heads, n_kv_heads, scale=1.0):
    q, keys, values = _f32(q), _f32(keys), _f32(values)
    head_dim = q.size // n_heads
    T = keys.size // (n_kv_heads * head_dim)
    out = np.zeros(q.size, dtype=np.float64)
    _check(lib().or_attend_f64(q.ctypes.data, q.size, keys.ctypes.data, values.ctypes.data, T, n_heads,
                               n_kv_heads, scale, out.ctypes.data))
    return out


def layer_attention_kind(n_layers, layer):
    return "global" if lib().or_layer_attention_kind(n_layers, layer) else "local"


def head_dim(n_layers, layer, local, glob):
    return lib().or_head_dim(n_layers, layer, local, glob)


def proportional_rope_freq_factors(hd, p):
    out = np.zeros(hd // 2, dtype=np.float32)
    lib().or_proportional_rope_freq_factors(hd, p, out.ctypes.data)
    return out


def windowed_len(seq_len, window):
    b, e = c_size(0), c_size(0)
    lib().or_windowed_len(seq_len, window, ctypes.byref(b), ctypes.byref(e))
    return range(b.value, e.value)


def kv_source_layer(n_layers, shared, layer):
    out = c_size(0)
    _check(lib().or_kv_source_layer(n_layers, shared, layer, ctypes.byref(out)))
    return out.value


class KvCache:
    """The oracle's ContextMemory (context_memory.rs:21-86)."""

    def __init__(self):
        self.h = lib().or_kv_new()

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_kv_free(self.h)
            self.h = None

    def append(self, layer, k, v):
        k, v = _f32(k), _f32(v)
        _check(lib().or_kv_append(self.h, layer, k.ctypes.data, v.ctypes.data, k.size))

    def view(self, layer, length):
        kp, vp, w = c_vp(), c_vp(), c_size(0)
        _check(lib().or_kv_view(self.h, layer, length, ctypes.byref(kp), ctypes.byref(vp), ctypes.byref(w)))
        if length == 0:
            return np.zeros((0, w.value), np.float32), np.zeros((0, w.value), np.float32)
        n = length * w.value
        k = np.ctypeslib.as_array(ctypes.cast(kp, P_f32), shape=(n,)).reshape(length, w.value).copy()
        v = np.ctypeslib.as_array(ctypes.cast(vp, P_f32), shape=(n,)).reshape(length, w.value).copy()
        return k, v

    def clear(self):
        lib().or_kv_clear(self.h)

    def layer_attention(self, hp, layer, position, q, k, v, q_norm_w, k_norm_w, rope_freqs):
        """Returns (out, source_layer, range) and leaves q/k/v normalised+rotated."""
        q, k, v = _f32(q).copy(), _f32(k).copy(), _f32(v).copy()
        qn = None if q_norm_w is None else _f32(q_norm_w)
        kn = None if k_norm_w is None else _f32(k_norm_w)
        rf = None if rope_freqs is None else _f32(rope_freqs)
        out = np.zeros(q.size, np.float32)
        src, b, e = c_size(0), c_size(0), c_size(0)
        _check(lib().or_layer_attention(self.h, ctypes.byref(hp), layer, position, q.ctypes.data, k.ctypes.data,
                                        v.ctypes.data, None if qn is None else qn.ctypes.data,
                                        None if kn is None else kn.ctypes.data,
                                        None if rf is None else rf.ctypes.data, 0 if rf is None else rf.size,
                                        out.ctypes.data, ctypes.byref(src), ctypes.byref(b), ctypes.byref(e)))
        return out, src.value, range(b.value, e.value), q, k, v


def pool_threads():
    return lib().or_pool_threads()


def prepare_rows(x, head_dim, weight=None, eps=1e-6, pos0=0, base=0.0, freq_factors=None):
    """In place on a C-contiguous float32 [n_rows, row_width] array: per-head
    RMS norm, then (base > 0) NEOX RoPE at position pos0 + row."""
    assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
    w = None if weight is None else _f32(weight)
    f = None if freq_factors is None else _f32(freq_factors)
    _check(lib().or_prepare_rows(x.ctypes.data, x.shape[0], x.shape[1], head_dim,
                                 None if w is None else w.ctypes.data, eps, pos0, base,
                                 None if f is None else f.ctypes.data, 0 if f is None else f.size))
    return x


# ---------------------------------------------- mat-vecs over GGUF weight formats
def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def f16_to_f32(h):
    return lib().or_f16_to_f32(int(h))


def f32_to_f16(x):
    return lib().or_f32_to_f16(float(x))


def bf16_to_f32(b):
    return lib().or_bf16_to_f32(int(b))


def f32_to_bf16(x):
    return lib().or_f32_to_bf16(float(x))


def quantize_q8_0(x):
    """quantize_q8_0 (matvec.rs:35-53): (scales f32 [n/32], quants int8 [n])."""
    x = _f32(x)
    scales = np.zeros(max(x.size // 32, 1), np.float32)
    quants = np.zeros(max(x.size, 1), np.int8)
    _check(lib().or_quantize_q8_0(x.ctypes.data, x.size, scales.ctypes.data, quants.ctypes.data))
    return scales[: x.size // 32], quants[: x.size]


def dequant_q8_0(data):
    data = _u8(data)
    out = np.zeros(max(data.size // 34 * 32, 1), np.float32)
    _check(lib().or_dequant_q8_0(data.ctypes.data, data.size, out.ctypes.data))
    return out[: data.size // 34 * 32]


def matvec_q8_0(w, rows, cols, xs, xq, softcap=None):
    w, xs, xq = _u8(w), _f32(xs), np.ascontiguousarray(xq, np.int8)
    out = np.zeros(max(rows, 1), np.float32)
    if softcap is None:
        _check(lib().or_matvec_q8_0(w.ctypes.data, w.size, rows, cols, xs.ctypes.data, xq.ctypes.data,
                                    out.ctypes.data))
    else:
        _check(lib().or_matvec_q8_0_softcap(w.ctypes.data, w.size, rows, cols, xs.ctypes.data, xq.ctypes.data,
                                            softcap, out.ctypes.data))
    return out[:rows]


def geglu_q8_0(gate, up, rows, cols, xs, xq, fp16_gelu=False):
    gate, up, xs, xq = _u8(gate), _u8(up), _f32(xs), np.ascontiguousarray(xq, np.int8)
    assert gate.size == up.size
    out = np.zeros(max(rows, 1), np.float32)
    _check(lib().or_geglu_q8_0(gate.ctypes.data, up.ctypes.data, gate.size, rows, cols, xs.ctypes.data,
                               xq.ctypes.data, int(fp16_gelu), out.ctypes.data))
    return out[:rows]


def matvec_q8_0_f32(w, rows, cols, x, f64_sums=False):
    w, x = _u8(w), _f32(x)
    out = np.zeros(max(rows, 1), np.float32)
    _check(lib().or_matvec_q8_0_f32(w.ctypes.data, w.size, rows, cols, x.ctypes.data, int(f64_sums),
                                    out.ctypes.data))
    return out[:rows]


def matvec_bf16(w, rows, cols, x):
    w, x = np.ascontiguousarray(w, np.uint16), _f32(x)
    out = np.zeros(max(rows, 1), np.float32)
    _check(lib().or_matvec_bf16(w.ctypes.data, w.size, rows, cols, x.ctypes.data, out.ctypes.data))
    return out[:rows]


def matvec_f32(w, rows, cols, x):
    w, x = _f32(w), _f32(x)
    out = np.zeros(max(rows, 1), np.float32)
    _check(lib().or_matvec_f32(w.ctypes.data, w.size, rows, cols, x.ctypes.data, out.ctypes.data))
    return out[:rows]


def softcap(v, cap):
    return lib().or_softcap(float(v), float(cap))


def gelu_tanh(x):
    return lib().or_gelu_tanh(float(x))


def gelu_tanh_fp16_table(x):
    return lib().or_gelu_tanh_fp16_table(float(x))
