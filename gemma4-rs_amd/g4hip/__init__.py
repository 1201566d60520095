"""Python binding of libg4attn.so, the MI355X attention backend for gemma4-rs.

The names mirror the engine's attention path (crates/llm-gemma4/src/impl_/model.rs,
crates/llm-backend-cpu/src/ops.rs, crates/llm-eng/src/context_memory.rs) so callers
and tests read like the reference's own.  Device buffers are torch tensors on
the GPU (torch provides allocation and streams only); every computation runs in
the HIP kernels of libg4attn.so.  There is no CPU fallback: without the built
library or without a GPU the calls raise.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libg4attn.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(_HERE)), "include", "g4attn.h")

G4_OK = 0
G4_ERR_CONTEXT_TOO_LONG = 1
G4_ERR_MISSING_LAYER = 2
G4_ERR_MISSING_WEIGHT = 3
G4_ERR_COMPUTE = 4
G4_ERR_MSG = 5

_ERR_NAMES = {
    G4_ERR_CONTEXT_TOO_LONG: "ContextTooLong",
    G4_ERR_MISSING_LAYER: "MissingLayer",
    G4_ERR_MISSING_WEIGHT: "MissingWeight",
    G4_ERR_COMPUTE: "Compute",
    G4_ERR_MSG: "Msg",
}


class EngError(RuntimeError):
    """An EngError variant (crates/llm-eng/src/error.rs:3-15) raised by the backend."""

    def __init__(self, code, message, fields=(0, 0)):
        self.code = code
        self.kind = _ERR_NAMES.get(code, f"status {code}")
        self.message = message
        self.fields = fields
        super().__init__(f"{self.kind}: {message}")


_lib = None

c_i64 = ctypes.c_int64
c_f32 = ctypes.c_float
c_int = ctypes.c_int
c_vp = ctypes.c_void_p
c_size = ctypes.c_size_t

_SIGS = {
    "g4_last_error": (ctypes.c_char_p, []),
    "g4_last_error_fields": (None, [ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "g4_init": (c_int, [c_int, ctypes.POINTER(c_vp)]),
    "g4_release": (c_int, [c_vp]),
    "g4_check_status": (c_int, [c_vp, c_vp]),
    "g4_set_decode_chunk": (c_int, [c_vp, c_i64]),
    "g4_set_prefill_exact": (c_int, [c_vp, c_int]),
    "g4_alloc": (c_int, [c_vp, c_size, ctypes.POINTER(c_vp)]),
    "g4_free": (c_int, [c_vp, c_vp]),
    "g4_copy_to_device": (c_int, [c_vp, c_vp, c_vp, c_size]),
    "g4_copy_to_host": (c_int, [c_vp, c_vp, c_vp, c_size]),
    "g4_copy_on_device": (c_int, [c_vp, c_vp, c_vp, c_size]),
    "g4_sync": (c_int, [c_vp, c_vp]),
    "g4_activate": (c_int, [c_vp]),
    "g4_attend": (c_int, [c_vp, c_vp, c_size, c_vp, c_vp, c_size, c_size, c_size, c_f32, c_vp]),
    "g4_attend_decode": (c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_f32, c_vp, c_vp]),
    "g4_attend_decode_noalloc": (c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_f32, c_vp,
                                         c_vp]),
    "g4_attend_decode_batch": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_int, c_int,
                                       c_int, c_f32, c_vp, c_vp]),
    "g4_attend_prefill": (c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_int, c_int, c_int, c_f32,
                                  c_vp, c_vp]),
    "g4_rms_norm_rows": (c_int, [c_vp, c_vp, c_i64, c_i64, c_vp, c_f32, c_vp, c_vp]),
    "g4_rope_neox_rows": (c_int, [c_vp, c_vp, c_i64, c_int, c_int, c_int, c_i64, c_f32, c_vp, c_i64, c_vp]),
    "g4_kv_create": (c_int, [c_vp, c_int, ctypes.POINTER(c_i64), c_i64, ctypes.POINTER(c_vp)]),
    "g4_kv_destroy": (c_int, [c_vp]),
    "g4_kv_append": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp]),
    "g4_kv_append_rows": (c_int, [c_vp, c_int, c_vp, c_vp, c_i64, c_vp]),
    "g4_kv_view": (c_int, [c_vp, c_int, c_i64, ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), ctypes.POINTER(c_i64)]),
    "g4_kv_view_rows": (c_int, [c_vp, c_int, c_i64, c_i64, ctypes.POINTER(c_vp), ctypes.POINTER(c_vp),
                                ctypes.POINTER(c_i64)]),
    "g4_kv_create_ring": (c_int, [c_vp, c_int, ctypes.POINTER(c_i64), c_i64, ctypes.POINTER(c_i64),
                                  ctypes.POINTER(c_vp)]),
    "g4_kv_len": (c_i64, [c_vp, c_int]),
    "g4_kv_clear": (None, [c_vp]),
    "g4_layer_attention": (c_int, [c_vp, c_vp, c_vp, c_int, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                   ctypes.POINTER(c_int), ctypes.POINTER(c_i64), ctypes.POINTER(c_i64), c_vp]),
    "g4_prepare_qkv": (c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_int, c_int, c_int, c_vp, c_vp, c_f32, c_f32,
                               c_vp, c_vp, c_vp, c_i64, c_vp]),
    "g4_decode_step_fused": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_f32, c_f32, c_vp, c_i64, c_vp, c_vp,
                                     c_i64, c_i64, c_vp, c_vp, c_int, c_int, c_int, c_f32, c_vp, c_vp]),
    "g4_layer_prefill": (c_int, [c_vp, c_vp, c_vp, c_int, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp,
                                 ctypes.POINTER(c_int), c_vp]),
    "g4_quantize_q8_0": (c_int, [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp]),
    "g4_matvec_q8_0": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp]),
    "g4_matvec_q8_0_softcap": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_f32, c_vp, c_vp]),
    "g4_geglu_q8_0": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_int, c_vp, c_vp]),
    "g4_matvec_q8_0_f32": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_vp, c_vp]),
    "g4_project_q8_0": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "g4_gated_ffn_q8_0": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_int, c_vp, c_vp]),
    "g4_logits_q8_0": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_f32, c_vp, c_vp]),
    "g4_matvec_bf16": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "g4_matvec_f32": (c_int, [c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "g4_prefill_schedule": (c_int, [c_i64, c_i64, c_i64, c_int, c_int, c_int, c_vp, c_i64, c_vp, c_i64, c_vp]),
    "g4_layer_is_global": (c_int, [c_int, c_int]),
    "g4_kv_source_layer": (c_int, [c_int, c_int, c_int, ctypes.POINTER(c_int)]),
    "g4_windowed_len": (None, [c_i64, c_i64, ctypes.POINTER(c_i64), ctypes.POINTER(c_i64)]),
    "g4_proportional_rope_freq_factors": (None, [c_int, c_f32, ctypes.POINTER(c_f32)]),
    "g4_port_matmul": (c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_vp, c_vp]),
    "g4_port_rms_norm": (c_int, [c_vp, c_vp, c_vp, c_i64, c_f32, c_vp, c_vp]),
    "g4_port_softmax": (c_int, [c_vp, c_vp, c_i64, c_vp, c_vp]),
    "g4_port_rope": (c_int, [c_vp, c_vp, c_i64, c_i64, c_f32, c_i64, c_vp]),
    "g4_port_add": (c_int, [c_vp, c_vp, c_vp, c_i64, c_vp, c_vp]),
}


class G4Hparams(ctypes.Structure):
    """g4_hparams: the Gemma4HyperParams fields attention reads (idea/mod.rs:15-34)."""

    _fields_ = [
        ("n_layers", c_int), ("n_heads", c_int), ("n_kv_heads", c_int),
        ("head_dim_local", c_int), ("head_dim_global", c_int), ("sliding_window", c_i64),
        ("shared_kv_layers", c_int), ("local_rope_base", c_f32), ("global_rope_base", c_f32),
        ("rms_norm_eps", c_f32),
    ]

    @classmethod
    def e2b(cls):
        """Gemma4HyperParams::e2b() (crates/llm-gemma4/src/idea/mod.rs:48-68)."""
        return cls(35, 8, 1, 256, 512, 512, 20, 10000.0, 1000000.0, 1e-6)


def lib():
    """The loaded libg4attn.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _raise(code):
    if code == G4_OK:
        return
    L = lib()
    a, b = ctypes.c_uint64(0), ctypes.c_uint64(0)
    L.g4_last_error_fields(ctypes.byref(a), ctypes.byref(b))
    raise EngError(code, L.g4_last_error().decode(), (a.value, b.value))


def _ptr(t):
    """Device (or host) address of a torch tensor or numpy array, or None."""
    if t is None:
        return None
    if isinstance(t, int):  # a raw address (Context.alloc)
        return t
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def _stream(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    return getattr(stream, "cuda_stream", stream)


# ------------------------------------------------------------------ policies
def layer_attention_kind(n_layers, layer):
    """'global' or 'local' (crates/llm-gemma4/src/idea/mod.rs:148-156)."""
    return "global" if lib().g4_layer_is_global(n_layers, layer) else "local"


def kv_source_layer(n_layers, shared_kv_layers, layer):
    """kv_source_layer (crates/llm-gemma4/src/eng/mod.rs:71-90)."""
    out = c_int(0)
    _raise(lib().g4_kv_source_layer(n_layers, shared_kv_layers, layer, ctypes.byref(out)))
    return out.value


def windowed_len(seq_len, window):
    """windowed_len (eng/mod.rs:10-12) as a Python range."""
    b, e = c_i64(0), c_i64(0)
    lib().g4_windowed_len(seq_len, window, ctypes.byref(b), ctypes.byref(e))
    return range(b.value, e.value)


def proportional_rope_freq_factors(head_dim, p):
    """proportional_rope_freq_factors (crates/llm-gemma4/src/idea/mod.rs:162-165)."""
    out = (c_f32 * (head_dim // 2))()
    lib().g4_proportional_rope_freq_factors(head_dim, p, out)
    return list(out)


# ------------------------------------------------------------------- context
def prefill_schedule(pos0, N, window, head_dim, n_kv_heads=1, num_cus=256):
    """g4_prefill_schedule: (units, bin_start) of the prefill kernel for a
    shape, as int32 numpy arrays -- units[i] = (block, t_lo, t_hi, slot),
    workgroup w runs units[bin_start[w]:bin_start[w+1]].  Host only."""
    import numpy as np
    counts = np.zeros(3, np.int32)
    units = np.zeros((1, 4), np.int32)
    bins = np.zeros(1, np.int32)
    code = lib().g4_prefill_schedule(pos0, N, window, head_dim, n_kv_heads, num_cus, units.ctypes.data, 1,
                                     bins.ctypes.data, 1, counts.ctypes.data)
    if code not in (0, 5):
        _raise(code)
    units = np.zeros((max(1, int(counts[0])), 4), np.int32)
    bins = np.zeros(int(counts[1]) + 1, np.int32)
    _raise(lib().g4_prefill_schedule(pos0, N, window, head_dim, n_kv_heads, num_cus, units.ctypes.data,
                                     len(units), bins.ctypes.data, len(bins), counts.ctypes.data))
    return units[:int(counts[0])], bins


class Context:
    """One device's backend context (g4_ctx)."""

    def __init__(self, device=0):
        h = c_vp()
        _raise(lib().g4_init(device, ctypes.byref(h)))
        self.handle = h
        self.device = device

    def close(self):
        if self.handle:
            _raise(lib().g4_release(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def check_status(self, stream=None):
        _raise(lib().g4_check_status(self.handle, _stream(stream)))

    def set_decode_chunk(self, keys):
        _raise(lib().g4_set_decode_chunk(self.handle, keys))

    def set_prefill_exact(self, exact):
        """1: prefill with f32 MFMA products only; 0: split-f16 products where the inputs allow."""
        _raise(lib().g4_set_prefill_exact(self.handle, int(exact)))

    # -- device memory (caller-owned buffers without torch) ----------------
    def alloc(self, nbytes):
        """A device address of nbytes on this context's device (None for 0)."""
        ptr = c_vp()
        _raise(lib().g4_alloc(self.handle, nbytes, ctypes.byref(ptr)))
        return ptr.value

    def free(self, ptr):
        _raise(lib().g4_free(self.handle, ptr))

    def copy_to_device(self, dst, src_host, nbytes):
        _raise(lib().g4_copy_to_device(self.handle, dst, _ptr(src_host), nbytes))

    def copy_to_host(self, dst_host, src, nbytes):
        _raise(lib().g4_copy_to_host(self.handle, _ptr(dst_host), src, nbytes))

    def copy_on_device(self, dst, src, nbytes):
        _raise(lib().g4_copy_on_device(self.handle, dst, src, nbytes))

    def sync(self, stream=None):
        _raise(lib().g4_sync(self.handle, _stream(stream)))

    def activate(self):
        _raise(lib().g4_activate(self.handle))

    # -- attention ---------------------------------------------------------
    def attend(self, q, keys, values, n_heads, n_kv_heads, scale=1.0):
        """attend (model.rs:348-366) on host float32 numpy arrays; returns out."""
        import numpy as np
        q = np.ascontiguousarray(q, dtype=np.float32)
        keys = np.ascontiguousarray(keys, dtype=np.float32)
        values = np.ascontiguousarray(values, dtype=np.float32)
        T = keys.shape[0] if keys.ndim > 1 else (keys.size // max(1, (q.size // n_heads) * n_kv_heads))
        out = np.zeros(q.size, dtype=np.float32)
        _raise(lib().g4_attend(self.handle, q.ctypes.data, q.size, keys.ctypes.data, values.ctypes.data, T,
                               n_heads, n_kv_heads, scale, out.ctypes.data))
        return out

    def attend_decode(self, q, k_cache, v_cache, kv_begin, kv_end, n_heads, n_kv_heads, head_dim,
                      out, scale=1.0, row_stride=None, stream=None):
        stride = row_stride if row_stride is not None else n_kv_heads * head_dim
        _raise(lib().g4_attend_decode(self.handle, _ptr(q), _ptr(k_cache), _ptr(v_cache), stride, kv_begin,
                                      kv_end, n_heads, n_kv_heads, head_dim, scale, _ptr(out), _stream(stream)))

    def attend_decode_noalloc(self, q, k_cache, v_cache, kv_begin, kv_end, n_heads, n_kv_heads, head_dim,
                              out, scale=1.0, row_stride=None, stream=None):
        """g4_attend_decode with its split partials in the static scratch (no allocation)."""
        stride = row_stride if row_stride is not None else n_kv_heads * head_dim
        _raise(lib().g4_attend_decode_noalloc(self.handle, _ptr(q), _ptr(k_cache), _ptr(v_cache), stride, kv_begin,
                                              kv_end, n_heads, n_kv_heads, head_dim, scale, _ptr(out),
                                              _stream(stream)))

    def attend_decode_batch(self, q, k_base, v_base, seq_row0, kv_begin, kv_end, max_kv_len, n_heads,
                            n_kv_heads, head_dim, out, scale=1.0, row_stride=None, stream=None):
        stride = row_stride if row_stride is not None else n_kv_heads * head_dim
        B = kv_begin.shape[0]
        _raise(lib().g4_attend_decode_batch(self.handle, B, _ptr(q), _ptr(k_base), _ptr(v_base), stride,
                                            _ptr(seq_row0), _ptr(kv_begin), _ptr(kv_end), max_kv_len, n_heads,
                                            n_kv_heads, head_dim, scale, _ptr(out), _stream(stream)))

    def attend_prefill(self, q, k_cache, v_cache, pos0, N, window, n_heads, n_kv_heads, head_dim, out,
                       scale=1.0, row_stride=None, stream=None):
        stride = row_stride if row_stride is not None else n_kv_heads * head_dim
        _raise(lib().g4_attend_prefill(self.handle, _ptr(q), _ptr(k_cache), _ptr(v_cache), stride, pos0, N,
                                       window, n_heads, n_kv_heads, head_dim, scale, _ptr(out), _stream(stream)))

    # -- preparation -------------------------------------------------------
    def rms_norm_rows(self, x, n_rows, width, weight, eps, out, stream=None):
        _raise(lib().g4_rms_norm_rows(self.handle, _ptr(x), n_rows, width, _ptr(weight), eps, _ptr(out),
                                      _stream(stream)))

    def rope_neox_rows(self, x, n_tokens, n_heads, head_dim, n_rot, pos0, base, freq_factors=None,
                       stream=None):
        nf = 0 if freq_factors is None else freq_factors.numel()
        _raise(lib().g4_rope_neox_rows(self.handle, _ptr(x), n_tokens, n_heads, head_dim, n_rot, pos0, base,
                                       _ptr(freq_factors), nf, _stream(stream)))

    def prepare_qkv(self, q, k, v, n_tokens, pos0, n_heads, n_kv_heads, head_dim, q_norm_w, k_norm_w, eps,
                    rope_base, freq_factors=None, k_rows=None, v_rows=None, row_stride=0, stream=None):
        """Fused q/k/v norm + RoPE (+ append into k_rows/v_rows), model.rs:394-406."""
        _raise(lib().g4_prepare_qkv(self.handle, _ptr(q), _ptr(k), _ptr(v), n_tokens, pos0, n_heads, n_kv_heads,
                                    head_dim, _ptr(q_norm_w), _ptr(k_norm_w), eps, rope_base, _ptr(freq_factors),
                                    _ptr(k_rows), _ptr(v_rows), row_stride, _stream(stream)))

    def decode_step_fused(self, q, k, v, q_norm_w, k_norm_w, eps, rope_base, freq_factors, position, k_cache,
                          v_cache, row_stride, n_rows, k_row, v_row, n_heads, n_kv_heads, head_dim, out, scale=1.0,
                          stream=None):
        """g4_decode_step_fused: q (and, with k, the new row) prepared inside the decode kernel."""
        _raise(lib().g4_decode_step_fused(self.handle, _ptr(q), _ptr(k), _ptr(v), _ptr(q_norm_w), _ptr(k_norm_w), eps,
                                          rope_base, _ptr(freq_factors), position, _ptr(k_cache), _ptr(v_cache),
                                          row_stride, n_rows, _ptr(k_row), _ptr(v_row), n_heads, n_kv_heads, head_dim,
                                          scale, _ptr(out), _stream(stream)))

    # -- mat-vecs over GGUF weight formats -----------------------------------
    def quantize_q8_0(self, x, n, scales, quants, stream=None):
        _raise(lib().g4_quantize_q8_0(self.handle, _ptr(x), n, _ptr(scales), _ptr(quants), _stream(stream)))

    def matvec_q8_0(self, w, rows, cols, xs, xq, out, softcap=None, stream=None):
        if softcap is None:
            _raise(lib().g4_matvec_q8_0(self.handle, _ptr(w), w.numel(), rows, cols, _ptr(xs), _ptr(xq), _ptr(out),
                                        _stream(stream)))
        else:
            _raise(lib().g4_matvec_q8_0_softcap(self.handle, _ptr(w), w.numel(), rows, cols, _ptr(xs), _ptr(xq),
                                                softcap, _ptr(out), _stream(stream)))

    def geglu_q8_0(self, gate, up, rows, cols, xs, xq, out, fp16_gelu=False, stream=None):
        _raise(lib().g4_geglu_q8_0(self.handle, _ptr(gate), _ptr(up), gate.numel(), rows, cols, _ptr(xs), _ptr(xq),
                                   int(fp16_gelu), _ptr(out), _stream(stream)))

    def project_q8_0(self, w, rows, cols, x, out, stream=None):
        _raise(lib().g4_project_q8_0(self.handle, _ptr(w), w.numel(), rows, cols, _ptr(x), _ptr(out), _stream(stream)))

    def gated_ffn_q8_0(self, gate, up, rows, cols, x, out, fp16_gelu=False, stream=None):
        _raise(lib().g4_gated_ffn_q8_0(self.handle, _ptr(gate), _ptr(up), gate.numel(), rows, cols, _ptr(x),
                                       int(fp16_gelu), _ptr(out), _stream(stream)))

    def logits_q8_0(self, w, rows, cols, x, cap, out, stream=None):
        _raise(lib().g4_logits_q8_0(self.handle, _ptr(w), w.numel(), rows, cols, _ptr(x), cap, _ptr(out),
                                    _stream(stream)))

    def matvec_q8_0_f32(self, w, rows, cols, x, out, f64_sums=False, stream=None):
        _raise(lib().g4_matvec_q8_0_f32(self.handle, _ptr(w), w.numel(), rows, cols, _ptr(x), int(f64_sums),
                                        _ptr(out), _stream(stream)))

    def matvec_bf16(self, w, rows, cols, x, out, stream=None):
        _raise(lib().g4_matvec_bf16(self.handle, _ptr(w), w.numel(), rows, cols, _ptr(x), _ptr(out), _stream(stream)))

    def matvec_f32(self, w, rows, cols, x, out, stream=None):
        _raise(lib().g4_matvec_f32(self.handle, _ptr(w), w.numel(), rows, cols, _ptr(x), _ptr(out), _stream(stream)))

    # -- ComputePort -------------------------------------------------------
    def port_matmul(self, a, b, m, n, k, out, stream=None):
        _raise(lib().g4_port_matmul(self.handle, _ptr(a), _ptr(b), m, n, k, _ptr(out), _stream(stream)))

    def port_rms_norm(self, x, weight, n, eps, out, stream=None):
        _raise(lib().g4_port_rms_norm(self.handle, _ptr(x), _ptr(weight), n, eps, _ptr(out), _stream(stream)))

    def port_softmax(self, x, n, out, stream=None):
        _raise(lib().g4_port_softmax(self.handle, _ptr(x), n, _ptr(out), _stream(stream)))

    def port_rope(self, x, length, pos, theta, dims, stream=None):
        _raise(lib().g4_port_rope(self.handle, _ptr(x), length, pos, theta, dims, _stream(stream)))

    def port_add(self, a, b, n, out, stream=None):
        _raise(lib().g4_port_add(self.handle, _ptr(a), _ptr(b), n, _ptr(out), _stream(stream)))


class KvCache:
    """Device-resident ContextMemory (crates/llm-eng/src/context_memory.rs:11-86)."""

    def __init__(self, ctx, widths, capacity, ring_rows=None):
        """ring_rows: per layer, 0 or the number of last positions a
        sliding-window ring keeps (g4_kv_create_ring)."""
        arr = (c_i64 * len(widths))(*widths)
        h = c_vp()
        if ring_rows is None:
            _raise(lib().g4_kv_create(ctx.handle, len(widths), arr, capacity, ctypes.byref(h)))
        else:
            rings = (c_i64 * len(widths))(*ring_rows)
            _raise(lib().g4_kv_create_ring(ctx.handle, len(widths), arr, capacity, rings, ctypes.byref(h)))
        self.handle = h
        self.ctx = ctx

    def close(self):
        if self.handle:
            lib().g4_kv_destroy(self.handle)
            self.handle = None

    def append(self, layer, k, v, stream=None):
        _raise(lib().g4_kv_append(self.handle, layer, _ptr(k), _ptr(v), _stream(stream)))

    def append_rows(self, layer, k, v, n, stream=None):
        _raise(lib().g4_kv_append_rows(self.handle, layer, _ptr(k), _ptr(v), n, _stream(stream)))

    def view(self, layer, length):
        """(k_ptr, v_ptr, row_stride) of the first `length` rows of `layer`."""
        k, v, s = c_vp(), c_vp(), c_i64(0)
        _raise(lib().g4_kv_view(self.handle, layer, length, ctypes.byref(k), ctypes.byref(v), ctypes.byref(s)))
        return k.value, v.value, s.value

    def view_rows(self, layer, begin, end):
        """(k_ptr, v_ptr, row_stride) of the rows of positions [begin, end)."""
        k, v, s = c_vp(), c_vp(), c_i64(0)
        _raise(lib().g4_kv_view_rows(self.handle, layer, begin, end, ctypes.byref(k), ctypes.byref(v),
                                     ctypes.byref(s)))
        return k.value, v.value, s.value

    def __len__(self):
        raise TypeError("use KvCache.len(layer)")

    def len(self, layer):
        return lib().g4_kv_len(self.handle, layer)

    def clear(self):
        lib().g4_kv_clear(self.handle)

    def layer_attention(self, hp, layer, position, q, k, v, q_norm_w, k_norm_w, rope_freqs, out, stream=None):
        """Gemma4CpuModel::layer's attention segment (model.rs:394-410) on the device;
        returns (source_layer, range(kv_begin, kv_end))."""
        src, b, e = c_int(0), c_i64(0), c_i64(0)
        _raise(lib().g4_layer_attention(self.ctx.handle, self.handle, ctypes.byref(hp), layer, position, _ptr(q),
                                        _ptr(k), _ptr(v), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(rope_freqs),
                                        _ptr(out), ctypes.byref(src), ctypes.byref(b), ctypes.byref(e),
                                        _stream(stream)))
        return src.value, range(b.value, e.value)

    def layer_prefill(self, hp, layer, pos0, n_tokens, q, k, v, q_norm_w, k_norm_w, rope_freqs, out, stream=None):
        """The layer's attention segment for prompt positions pos0 .. pos0+n_tokens-1 in one
        call (the token-at-a-time loop of generate.rs:37-41, batched); returns the source layer."""
        src = c_int(0)
        _raise(lib().g4_layer_prefill(self.ctx.handle, self.handle, ctypes.byref(hp), layer, pos0, n_tokens, _ptr(q),
                                      _ptr(k), _ptr(v), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(rope_freqs),
                                      _ptr(out), ctypes.byref(src), _stream(stream)))
        return src.value
