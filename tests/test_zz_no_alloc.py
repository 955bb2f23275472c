"""qh_matmul_prefill_noalloc (the entry point that allocates nothing) against qh_matmul_prefill,
through the C ABI: the same kernels on the same inputs, so the outputs must be equal bit for bit.
Two calls in a row on one context, the second smaller than the first (the shared static scratch
keeps the first call's contents), then a call whose scratch would not fit is refused."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _hip_runtime():
    """The HIP runtime the library links (already loaded in this process)."""
    rt = ctypes.CDLL("libamdhip64.so")
    vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
    rt.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    rt.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
    rt.hipStreamEndCapture.argtypes = [vp, pvp]
    rt.hipGraphInstantiate.argtypes = [pvp, vp, vp, vp, ctypes.c_size_t]
    rt.hipGraphLaunch.argtypes = [vp, vp]
    rt.hipStreamSynchronize.argtypes = [vp]
    rt.hipGraphExecDestroy.argtypes = [vp]
    rt.hipGraphDestroy.argtypes = [vp]
    return rt


def _free_bytes(rt):
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert rt.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def _weights(hip, ctx, fmt, rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    if fmt == "int8":
        q, s = hip.quantize_int8(w)
        bufs = [ctx.upload(q), ctx.upload(s)]
        return ctx.weight(hip.FMT_INT8, rows, cols, bufs[0], bufs[1]), bufs
    q, s, z = hip.quantize_int4(w, 128)
    bufs = [ctx.upload(q), ctx.upload(s), ctx.upload(z)]
    return ctx.weight(hip.FMT_INT4, rows, cols, bufs[0], bufs[1], bufs[2], group=128), bufs


@pytest.mark.parametrize("calls", [
    # (format, rows, cols, M, bias): the config-5 down projection at 512 rows, then a
    # 37-row gate|up contraction
    [("int8", 896, 4864, 512, True), ("int4", 9728, 896, 37, False)],
    [("int4", 1152, 896, 300, True), ("int8", 896, 896, 5, True)],
])
def test_noalloc_prefill_equals_the_allocating_entry_point(ctx, hip, calls):
    for i, (fmt, rows, cols, M, with_bias) in enumerate(calls):
        print(f"noalloc call {i}: {fmt} {rows}x{cols}, M={M}", flush=True)
        W, bufs = _weights(hip, ctx, fmt, rows, cols, seed=10 + i)
        rng = np.random.default_rng(20 + i)
        x = ctx.upload(rng.standard_normal((M, cols)).astype(np.float32))
        bias = ctx.upload((rng.standard_normal(rows) * 0.02).astype(np.float32)) if with_bias else None
        y_ref, y_new = ctx.empty(M * rows * 4), ctx.empty(M * rows * 4)
        ctx.matmul_prefill(W, x, bias, y_ref, M)
        ctx.matmul_prefill_noalloc(W, x, bias, y_new, M)
        a, b = y_ref.read(), y_new.read()
        assert np.isfinite(a).all()
        np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
        for buf in bufs + [x, y_ref, y_new] + ([bias] if bias else []):
            buf.free()


def test_noalloc_prefill_refuses_shapes_beyond_its_scratch(ctx, hip):
    W, bufs = _weights(hip, ctx, "int8", 128, 8192, seed=3)
    x, y = ctx.upload(np.zeros((16, 8192), np.float32)), ctx.empty(16 * 128 * 4)
    with pytest.raises(hip.RangeError, match="no-allocation MFMA prefill has 25165824 bytes of scratch"):
        ctx.matmul_prefill_noalloc(W, x, None, y, 4096)      # 4096 x 8192 digit planes: 96 MiB
    ctx.matmul_prefill_noalloc(W, x, None, y, 16)            # a fitting call still works after it
    for b in bufs + [x, y]:
        b.free()


def test_noalloc_prefill_allocates_nothing(ctx, hip):
    """Warm calls leave the device's free memory where it was, and the call records into a
    global-mode stream capture, in which the runtime refuses device allocation: the capture
    ends cleanly, and its graph, replayed three times with eager work between the replays,
    gives the eager call's bits every time."""
    rt = _hip_runtime()
    M, rows, cols = 128, 896, 4864
    print(f"noalloc capture: int8 {rows}x{cols}, M={M}", flush=True)
    W, bufs = _weights(hip, ctx, "int8", rows, cols, seed=5)
    x = ctx.upload(np.random.default_rng(6).standard_normal((M, cols)).astype(np.float32))
    y_eager, y_graph = ctx.empty(M * rows * 4), ctx.empty(M * rows * 4)
    ctx.matmul_prefill_noalloc(W, x, None, y_eager, M)   # first call: code and scratch address resolved
    ctx.done()
    before = _free_bytes(rt)
    for _ in range(3):
        ctx.matmul_prefill_noalloc(W, x, None, y_eager, M)
    ctx.done()
    assert _free_bytes(rt) == before
    eager = y_eager.read()
    assert np.isfinite(eager).all()

    stream = ctypes.c_void_p(ctx.stream)
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    assert rt.hipStreamBeginCapture(stream, 0) == 0      # hipStreamCaptureModeGlobal
    try:
        ctx.matmul_prefill_noalloc(W, x, None, y_graph, M)
    finally:
        ended = rt.hipStreamEndCapture(stream, ctypes.byref(graph))
    assert ended == 0 and graph.value
    assert rt.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
    try:
        for rep in range(3):
            ctx.matmul_prefill(W, x, None, y_graph, 7)       # eager work on the same stream between replays
            ctx.done()
            assert rt.hipGraphLaunch(exe, stream) == 0
            assert rt.hipStreamSynchronize(stream) == 0
            got = y_graph.read()
            np.testing.assert_array_equal(got.view(np.uint32), eager.view(np.uint32), err_msg=f"replay {rep}")
    finally:
        rt.hipGraphExecDestroy(exe)
        rt.hipGraphDestroy(graph)
    for b in bufs + [x, y_eager, y_graph]:
        b.free()
