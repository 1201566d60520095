"""Device memory through the C ABI (g4_alloc, g4_copy_*, g4_free, g4_sync):
a binding can hold caller-owned buffers (the device image of F32Buf,
crates/llm-backend-cpu/src/buffer.rs:1-26) without any other runtime, and
the kernels read and write them."""
import numpy as np
import pytest

import g4hip

pytestmark = pytest.mark.gpu


def test_alloc_copy_free_round_trip(ctx):
    x = (np.arange(1000, dtype=np.float32) * 0.5 - 3.0).astype(np.float32)
    n = x.nbytes
    a, b, out = ctx.alloc(n), ctx.alloc(n), ctx.alloc(n)
    try:
        assert a and b and out and len({a, b, out}) == 3
        ctx.copy_to_device(a, x, n)
        ctx.copy_on_device(b, a, n)
        y = np.zeros_like(x)
        ctx.copy_to_host(y, b, n)
        assert np.array_equal(x, y)
        # the buffers serve the kernels: CpuPort::add (ops.rs:168-178) on them
        ctx.port_add(a, b, x.size, out, stream=0)
        ctx.sync(0)
        z = np.zeros_like(x)
        ctx.copy_to_host(z, out, n)
        assert np.array_equal(z, x + x)
    finally:
        for ptr in (a, b, out):
            ctx.free(ptr)


def test_empty_and_invalid_memory_calls(ctx):
    assert ctx.alloc(0) is None
    ctx.free(None)  # no-op
    ctx.copy_to_device(None, np.zeros(0, np.float32), 0)  # zero bytes: nothing to do
    with pytest.raises(g4hip.EngError, match="null pointer"):
        ctx.copy_to_host(np.zeros(4, np.float32), None, 16)
    p = ctx.alloc(64)
    try:
        with pytest.raises(g4hip.EngError, match="null pointer"):
            ctx.copy_on_device(p, None, 64)
    finally:
        ctx.free(p)
