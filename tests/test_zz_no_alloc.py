"""g4_attend_decode_noalloc: the single-sequence decode with its split
partials in the static device scratch, allocating nothing.

Called through the C ABI, its output must equal g4_attend_decode's bit for
bit (same kernels, same split plan) on two calls in a row, the second with a
smaller input (global layer d=512 over 4096 rows, then a sliding layer d=256
over 512), and match the oracle within the reference's tolerance.  In a fresh
context -- whose own workspace is still empty, so an allocation there would
show -- the device's free memory must not change across the calls.  A split
plan larger than the scratch is refused."""
import ctypes

import numpy as np
import pytest
import torch

import g4hip
import inputs as I
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-4
CASES = [(512, 4096, True), (256, 512, False)]  # the second call is smaller


def free_device_bytes():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_noalloc_decode_equals_the_allocating_decode(ctx):
    print("[case] g4_attend_decode_noalloc vs g4_attend_decode", flush=True)
    inputs = []
    for d, T, glob in CASES:
        q, K, V, _ = I.decode_case(60 + d, T, d, glob)
        inputs.append((d, T, q, K, V, *(torch.from_numpy(x).cuda() for x in (q, K, V))))
    refs = []
    for d, T, q, K, V, qd, Kd, Vd in inputs:  # the allocating entry point (loads the kernels too)
        ref = torch.zeros(8 * d, device="cuda")
        ctx.attend_decode(qd, Kd, Vd, 0, T, 8, 1, d, ref)
        ctx.check_status()
        refs.append(ref)
    fresh = g4hip.Context(0)
    try:
        outs = [torch.full((8 * d,), float("nan"), device="cuda") for d, *_ in inputs]
        torch.cuda.synchronize()
        free0 = free_device_bytes()
        for (d, T, q, K, V, qd, Kd, Vd), out in zip(inputs, outs):
            fresh.attend_decode_noalloc(qd, Kd, Vd, 0, T, 8, 1, d, out)
            fresh.check_status()
        free1 = free_device_bytes()
        for (d, T, q, K, V, *_), out, ref in zip(inputs, outs, refs):
            assert torch.equal(out, ref), (d, T)
            err = I.rel_err(out.cpu().numpy(), orc.attend(q, K, V, 8, 1))
            print(f"[parity] noalloc d={d} T={T}: rel err vs oracle {err:.2e}", flush=True)
            assert err <= TOL
        assert free1 == free0, f"device free memory moved by {free0 - free1} bytes"
    finally:
        fresh.close()


def test_noalloc_decode_refuses_a_plan_above_its_scratch(ctx):
    """16 query heads on one KV head, d=512, cut into 512 splits of 16 keys:
    16 MiB of partials, above the 8 MiB + 64 KiB scratch."""
    d, T = 512, 8192
    q = torch.zeros(16 * d, device="cuda")
    K = torch.zeros(T * d, device="cuda")
    out = torch.zeros(16 * d, device="cuda")
    ctx.set_decode_chunk(16)
    try:
        with pytest.raises(g4hip.EngError, match="needs .* bytes of split scratch, above the static 8454144"):
            ctx.attend_decode_noalloc(q, K, K, 0, T, 16, 1, d, out)
    finally:
        ctx.set_decode_chunk(0)
