"""GPU parity of every operator against the CPU oracle on the same inputs
(the kernel harness of web/kernels.html: same-f16 inputs, bound max-abs /
max|ref| <= 1e-5, and bitwise checks where the arithmetic is exact)."""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

KERNEL_REL = 1e-5   # web/kernels.html:134


def rel_err(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    scale = np.max(np.abs(ref))
    return float(np.max(np.abs(got - ref)) / scale) if scale > 0 else float(np.max(np.abs(got)))


def ulps(a, b):
    return int(np.max(np.abs(np.asarray(a, np.float32).view(np.int32).astype(np.int64)
                             - np.asarray(b, np.float32).view(np.int32).astype(np.int64))))


def upload_weight(ctx, hip, w32, fmt, group=128):
    """Quantize with the product's loader quantizer; return (Weight, buffers, dequantized f32)."""
    rows, cols = w32.shape
    if fmt == "f16":
        h = O.f32_to_f16(w32)
        bufs = [ctx.upload(h)]
        return ctx.weight(hip.FMT_F16, rows, cols, bufs[0]), bufs, O.f16_to_f32(h)
    if fmt == "int8":
        q, s = hip.quantize_int8(w32)
        bufs = [ctx.upload(q), ctx.upload(s)]
        return ctx.weight(hip.FMT_INT8, rows, cols, bufs[0], bufs[1]), bufs, O.dequantize_int8(q, s)
    q, s, z = hip.quantize_int4(w32, group)
    bufs = [ctx.upload(q), ctx.upload(s), ctx.upload(z)]
    return (ctx.weight(hip.FMT_INT4, rows, cols, bufs[0], bufs[1], bufs[2], group), bufs,
            O.dequantize_int4(q, s, z, cols, group))


def free(*bufs):
    for b in bufs:
        if isinstance(b, (list, tuple)):
            free(*b)
        else:
            b.free()


SHAPES = [(896, 896), (128, 896), (4864, 896), (896, 4864)]


@pytest.mark.parametrize("fmt", ["f16", "int8", "int4"])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_matches_oracle(ctx, hip, fmt, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    w32 = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    bias = (rng.standard_normal(rows) * 0.02).astype(np.float32)
    W, wb, deq = upload_weight(ctx, hip, w32, fmt)
    dx, db, dy = ctx.upload(x), ctx.upload(bias), ctx.empty(rows * 4)
    ctx.matvec(W, dx, db, dy, 1)
    got = dy.read(count=rows)
    ref = O.matvec(deq, x, rows, cols, bias)
    print(f"matvec {fmt} {rows}x{cols}: rel {rel_err(got, ref):.2e} ulps {ulps(got, ref)}")
    assert rel_err(got, ref) <= KERNEL_REL
    # Same f32 dequantized weights and f64 accumulation as the CPU: only the f64 summation
    # order differs, which moves the f32 result by at most one ulp and rarely.
    assert ulps(got, ref) <= 1
    assert np.mean(got.view(np.uint32) == ref.view(np.uint32)) >= 0.999
    free(wb, dx, db, dy)


@pytest.mark.parametrize("fmt", ["int8", "int4"])
def test_matvec_irregular_quant_params(ctx, hip, fmt):
    # Scales and zero points the quantizer never writes (zero, negative, non-integer or
    # out-of-range zero points, huge scales) take the reference's dequant arithmetic
    # rather than the biased-byte form; either way each weight is the loader's f32.
    rows, cols, group = 64, 896, 128
    rng = np.random.default_rng(11)
    w32 = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    if fmt == "int8":
        q, s = hip.quantize_int8(w32)
        s[::5] = 0.0
        s[1::5] *= -1.0
        s[2::5] = np.float32(2.0 ** 110)
        bufs = [ctx.upload(q), ctx.upload(s)]
        W = ctx.weight(hip.FMT_INT8, rows, cols, bufs[0], bufs[1])
        deq = O.dequantize_int8(q, s)
    else:
        q, s, z = hip.quantize_int4(w32, group)
        s, z = s.reshape(rows, -1), z.reshape(rows, -1)
        z[::4, 0] = 2.5
        z[1::4, 1] = 17.0
        z[2::4, 2] = -3.0
        s[3::4, 3] *= -1.0
        s[::6, 4] = 0.0
        s, z = s.reshape(-1), z.reshape(-1)
        bufs = [ctx.upload(q), ctx.upload(s), ctx.upload(z)]
        W = ctx.weight(hip.FMT_INT4, rows, cols, bufs[0], bufs[1], bufs[2], group)
        deq = O.dequantize_int4(q, s, z, cols, group)
    dx, dy = ctx.upload(x), ctx.empty(rows * 4)
    ctx.matvec(W, dx, None, dy, 1)
    got = dy.read(count=rows)
    ref = O.matvec(deq, x, rows, cols)
    finite = np.isfinite(ref)
    assert np.array_equal(np.isfinite(got), finite)
    assert ulps(got[finite], ref[finite]) <= 1
    free(bufs, dx, dy)


def test_matvec_lm_head_shape_int8(ctx, hip):
    rows, cols = 151936, 896
    rng = np.random.default_rng(1)
    w32 = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    W, wb, deq = upload_weight(ctx, hip, w32, "int8")
    dx, dy = ctx.upload(x), ctx.empty(rows * 4)
    ctx.matvec(W, dx, None, dy, 1)
    got = dy.read(count=rows)
    ref = O.matvec(deq, x, rows, cols)
    assert rel_err(got, ref) <= KERNEL_REL
    assert ctx.argmax(dy, rows) == O.argmax(ref) or abs(got[O.argmax(ref)] - got.max()) < 1e-5
    free(wb, dx, dy)


@pytest.mark.parametrize("fmt", ["f16", "int8", "int4"])
@pytest.mark.parametrize("seq", [2, 3, 5, 8, 11])
def test_batched_matvec_equals_single_position_bitwise(ctx, hip, fmt, seq):
    # batchedMatvec's property (src/gpu/kernels.js:217-231): the position tile never
    # changes how an output is summed, so prefill equals decode bit for bit.
    rows, cols = 896, 4864 if fmt != "f16" else 896
    rng = np.random.default_rng(seq)
    w32 = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    X = rng.standard_normal((seq, cols)).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32)
    W, wb, _ = upload_weight(ctx, hip, w32, fmt)
    dX, db, dY = ctx.upload(X), ctx.upload(bias), ctx.empty(seq * rows * 4)
    ctx.matvec(W, dX, db, dY, seq)
    batched = dY.read(count=seq * rows).reshape(seq, rows)
    one, dy = [], ctx.empty(rows * 4)
    for t in range(seq):
        dx = ctx.upload(X[t])
        ctx.matvec(W, dx, db, dy, 1)
        one.append(dy.read(count=rows))
        dx.free()
    np.testing.assert_array_equal(batched.view(np.uint32), np.array(one).view(np.uint32))
    free(wb, dX, db, dY, dy)


MFMA_REL = KERNEL_REL   # int8 MFMA: exact codes, x in 24-bit fixed point per row, exact int32 sums


@pytest.mark.parametrize("fmt", ["int8", "int4"])
@pytest.mark.parametrize("M,rows,cols", [(1, 896, 896), (17, 1152, 896), (64, 896, 896), (130, 896, 4864),
                                         (512, 896, 896), (100, 9728, 896), (512, 896, 4864)])
def test_matmul_prefill_matches_oracle(ctx, hip, fmt, M, rows, cols):
    """The MFMA prefill contraction against the oracle's f64 matvec of every position, on
    the same dequantized weights: within MFMA_REL (a stated tolerance, as the reference
    gave its tiled matmul one, web/scaling.html:122-127)."""
    rng = np.random.default_rng(M * 31 + rows + cols)
    w32 = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    X = rng.standard_normal((M, cols)).astype(np.float32)
    bias = (rng.standard_normal(rows) * 0.02).astype(np.float32)
    W, wb, deq = upload_weight(ctx, hip, w32, fmt)
    dX, db, dY = ctx.upload(X), ctx.upload(bias), ctx.empty(M * rows * 4)
    ctx.matmul_prefill(W, dX, db, dY, M)
    got = dY.read(count=M * rows).reshape(M, rows)
    worst = 0.0
    for t in range(M):
        ref = O.matvec(deq, X[t], rows, cols, bias)
        worst = max(worst, rel_err(got[t], ref))
    print(f"matmul_prefill {fmt} M={M} {rows}x{cols}: worst row rel {worst:.2e}")
    assert worst <= MFMA_REL
    free(wb, dX, db, dY)


@pytest.mark.parametrize("M,rows,cols", [(5, 130, 32), (33, 200, 96), (70, 300, 1056)])
def test_matmul_prefill_half_last_step(ctx, hip, M, rows, cols):
    """int8 with K = 64 k + 32: the last K step's second half lies past the row (its weight
    loads re-read the row's last columns against zero digits), with ragged M and N and, at
    1056 columns, K split over many slices."""
    rng = np.random.default_rng(M + rows + cols)
    w32 = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    X = rng.standard_normal((M, cols)).astype(np.float32)
    W, wb, deq = upload_weight(ctx, hip, w32, "int8")
    dX, dY = ctx.upload(X), ctx.empty(M * rows * 4)
    ctx.matmul_prefill(W, dX, None, dY, M)
    got = dY.read(count=M * rows).reshape(M, rows)
    worst = max(rel_err(got[t], O.matvec(deq, X[t], rows, cols, None)) for t in range(M))
    assert worst <= MFMA_REL
    free(wb, dX, dY)


def test_matmul_prefill_rejects_f16_and_ragged_k(ctx, hip):
    rng = np.random.default_rng(0)
    W, wb, _ = upload_weight(ctx, hip, (rng.standard_normal((64, 896)) * 0.02).astype(np.float32), "f16")
    dX, dY = ctx.upload(np.zeros((4, 896), np.float32)), ctx.empty(4 * 64 * 4)
    with pytest.raises(hip.QwenHipError, match="int8 or int4"):
        ctx.matmul_prefill(W, dX, None, dY, 4)
    W8, wb8, _ = upload_weight(ctx, hip, (rng.standard_normal((64, 48)) * 0.02).astype(np.float32), "int8")
    with pytest.raises(hip.QwenHipError, match="multiple of 32"):
        ctx.matmul_prefill(W8, dX, None, dY, 4)
    free(wb, wb8, dX, dY)


@pytest.mark.parametrize("rows,cols", SHAPES + [(151936, 896)])
def test_matvec_f16_activation_list(ctx, hip, rows, cols):
    # Config 2: int8 weights, x ~ N(0,1) in f16, a list of distinct matrices in one launch.
    count = 3 if rows * cols < 10_000_000 else 1
    rng = np.random.default_rng(rows + 3 * cols)
    qs, ss, refs, xs = [], [], [], []
    for i in range(count):
        w32 = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
        q, s = hip.quantize_int8(w32)
        xh = O.f32_to_f16(rng.standard_normal(cols).astype(np.float32))
        qs.append(q), ss.append(s), xs.append(xh)
        refs.append(O.matvec(O.dequantize_int8(q, s), O.f16_to_f32(xh), rows, cols))
    dq, ds = ctx.upload(np.stack(qs)), ctx.upload(np.stack(ss))
    dx, dy = ctx.upload(np.stack(xs)), ctx.empty(count * rows * 4)
    W = ctx.weight(hip.FMT_INT8, rows, cols, dq, ds)
    ctx.matvec_xh_list(W, count, rows * cols, rows, dx, cols, dy)
    got = dy.read(count=count * rows).reshape(count, rows)
    for i in range(count):
        assert rel_err(got[i], refs[i]) <= KERNEL_REL
    free(dq, ds, dx, dy)


@pytest.mark.parametrize("rows,cols", [(1, 896), (5, 896), (1, 4864), (3, 8)])
def test_rmsnorm_matches_oracle_to_one_ulp(ctx, hip, rows, cols):
    rng = np.random.default_rng(cols)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    gain = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    dx, dg, dy = ctx.upload(x), ctx.upload(gain), ctx.empty(x.nbytes)
    ctx.rmsnorm(dx, dg, dy, rows, cols, 1e-6)
    got = dy.read(count=x.size).reshape(rows, cols)
    ref = np.stack([O.rmsnorm(x[r], gain, 1e-6) for r in range(rows)])
    assert ulps(got, ref) <= 1
    free(dx, dg, dy)


def test_rmsnorm_eps_inside_root(ctx, hip):
    x = np.array([1e-4, 1e-4], np.float32)
    dx, dg, dy = ctx.upload(x), ctx.upload(np.ones(2, np.float32)), ctx.empty(8)
    ctx.rmsnorm(dx, dg, dy, 1, 2, 1e-6)
    got = dy.read(count=2)
    assert abs(got[0] - 1e-4 / np.sqrt(1e-8 + 1e-6)) < 1e-6
    free(dx, dg, dy)


@pytest.mark.parametrize("rows,heads,base", [(1, 14, 0), (1, 2, 1023), (4, 14, 37), (1, 14, 32767)])
def test_rope_matches_oracle(ctx, hip, rows, heads, base):
    positions = 32768
    cos, sin = hip.rope_tables(64, 1e6, positions)
    rng = np.random.default_rng(base + heads)
    v = rng.standard_normal(rows * heads * 64).astype(np.float32)
    dv, dc, ds = ctx.upload(v), ctx.upload(cos), ctx.upload(sin)
    ctx.rope(dv, dc, ds, positions, rows, heads, 64, base)
    got = dv.read(count=v.size)
    ref = v.copy()
    inv = O.rope_freqs(64, 1e6)
    for r in range(rows):
        for h in range(heads):
            O.rope_inplace(ref, (r * heads + h) * 64, 64, base + r, inv)
    assert rel_err(got, ref) <= KERNEL_REL
    free(dv, dc, ds)


def test_rope_beyond_table_is_range_error(ctx, hip):
    cos, sin = hip.rope_tables(64, 1e6, 16)
    dv, dc, ds = ctx.upload(np.zeros(64, np.float32)), ctx.upload(cos), ctx.upload(sin)
    with pytest.raises(hip.RangeError, match="rope table"):
        ctx.rope(dv, dc, ds, 16, 1, 1, 64, 16)
    free(dv, dc, ds)


def kv_setup(ctx, hip, capacity, ctx_len, seed, kv_heads=2):
    """f16 caches holding ctx_len positions of K, V ~ N(0,1), written by qh_kv_append;
    returns device caches and the oracle's [pos, kv_dim] f32 views."""
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((ctx_len, kv_heads * 64)).astype(np.float32)
    v = rng.standard_normal((ctx_len, kv_heads * 64)).astype(np.float32)
    kc = ctx.empty(kv_heads * capacity * 64 * 2)
    vc = ctx.empty(hip.value_cache_bytes(capacity, kv_heads))
    dk, dv = ctx.upload(k), ctx.upload(v)
    ctx.kv_append(dk, dv, kc, vc, capacity, kv_heads, 64, 0, ctx_len)
    free(dk, dv)
    return kc, vc, O.through_f16(k), O.through_f16(v)


@pytest.mark.parametrize("capacity", [8, 13])
def test_kv_append_rounds_to_f16_exactly(ctx, hip, capacity):
    # keys position-major [kv_heads, capacity, 64]; values dimension-major
    # [kv_heads, 64, vstride] with vstride = capacity rounded up to 64 (128-byte rows)
    kc, vc, kr, vr = kv_setup(ctx, hip, capacity, 5, 0)
    got = kc.read(np.uint16, 2 * capacity * 64).reshape(2, capacity, 64)[:, :5]
    want = O.f32_to_f16(kr).reshape(5, 2, 64).transpose(1, 0, 2)
    np.testing.assert_array_equal(got, want)
    vstride = (capacity + 63) // 64 * 64
    assert hip.value_cache_bytes(capacity, 2) == 2 * 64 * vstride * 2
    got_v = vc.read(np.uint16, 2 * 64 * vstride).reshape(2, 64, vstride)[:, :, :5]
    want_v = O.f32_to_f16(vr).reshape(5, 2, 64).transpose(1, 2, 0)
    np.testing.assert_array_equal(got_v, want_v)
    with pytest.raises(hip.RangeError):
        ctx.kv_append(kc, vc, kc, vc, capacity, 2, 64, capacity - 2, 3)
    free(kc, vc)


def check_attention(got, ref, splitk):
    """Split-K: the kernel tolerance. Exact order: the CPU's arithmetic, so only the f64
    exp / sum ordering can differ -- a rare last-bit difference (<= 2 ulps, >= 99% equal)."""
    assert rel_err(got, ref) <= KERNEL_REL
    if not splitk:
        assert ulps(got, ref) <= 2
        assert np.mean(got.view(np.uint32) == ref.view(np.uint32)) >= 0.99


KINDS = ["exact", "splitk", "mfma"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("ctx_len", [1, 2, 63, 64, 65, 128, 1000, 1024, 4096])
def test_decode_attention_matches_oracle(ctx, hip, ctx_len, kind):
    heads, kv_heads = 14, 2
    kc, vc, kr, vr = kv_setup(ctx, hip, ctx_len + 3, ctx_len, ctx_len)
    q = np.random.default_rng(ctx_len + 1).standard_normal(heads * 64).astype(np.float32)
    dq, dout = ctx.upload(q), ctx.empty(heads * 64 * 4)
    ctx.attention(dq, kc, vc, ctx_len + 3, dout, 1, ctx_len - 1, heads, kv_heads, kind=kind)
    got = dout.read(count=heads * 64)
    ref = O.grouped_attention(q, kr, vr, 1, ctx_len - 1, heads, kv_heads, 64)
    print(f"attention ctx {ctx_len} {kind}: rel {rel_err(got, ref):.2e} ulps {ulps(got, ref)}")
    check_attention(got, ref, kind != "exact")
    free(kc, vc, dq, dout)


@pytest.mark.parametrize("ctx_len", [1, 100, 1000, 5000])
def test_attention_list_matches_single_calls(ctx, hip, ctx_len):
    """The list form (config 3's rotation in one launch) gives each cache the single-cache
    split-K result within the kernel tolerance of the oracle."""
    heads, kv_heads, count, cap = 14, 2, 5, ctx_len + 3
    vstride = hip.value_cache_bytes(cap, kv_heads) // (kv_heads * 64 * 2)
    rng = np.random.default_rng(ctx_len)
    kel, vel = kv_heads * cap * 64, kv_heads * 64 * vstride
    keys = O.f32_to_f16(rng.standard_normal(count * kel).astype(np.float32))
    vals = O.f32_to_f16(rng.standard_normal(count * vel).astype(np.float32))
    q = rng.standard_normal(heads * 64).astype(np.float32)
    dk, dv, dq, dout = ctx.upload(keys), ctx.upload(vals), ctx.upload(q), ctx.empty(count * heads * 64 * 4)
    ctx.attention_list(dq, dk, dv, kel, vel, count, cap, dout, ctx_len - 1, heads, kv_heads)
    got = dout.read(count=count * heads * 64).reshape(count, heads * 64)
    for i in range(count):
        kr = O.f16_to_f32(keys[i * kel:(i + 1) * kel]).reshape(kv_heads, cap, 64)[:, :ctx_len]
        vr = O.f16_to_f32(vals[i * vel:(i + 1) * vel]).reshape(kv_heads, 64, vstride)[:, :, :ctx_len]
        K = np.ascontiguousarray(kr.transpose(1, 0, 2).reshape(ctx_len, -1))
        V = np.ascontiguousarray(vr.transpose(2, 0, 1).reshape(ctx_len, -1))
        ref = O.grouped_attention(q, K, V, 1, ctx_len - 1, heads, kv_heads, 64)
        assert rel_err(got[i], ref) <= KERNEL_REL
    free(dk, dv, dq, dout)


# Config 3's timed (context, list length) shapes -- the list lengths are the smallest that
# keep the bench's launch shape -- and two ragged contexts: (slots, waves) per (cache, kv head).
# With one slot the block writes the output itself; with four the slots are merged by a launch
# of their own.
TIMED_LIST_PLANS = [(128, 128, (1, 1)), (1024, 128, (1, 4)), (4096, 128, (1, 8)), (32768, 32, (4, 8)),
                    (1000, 128, (1, 4)), (4000, 128, (1, 8))]


@pytest.mark.parametrize("ctx_len,count,plan", TIMED_LIST_PLANS)
def test_attention_list_timed_plans_match_oracle(ctx, hip, ctx_len, count, plan):
    """The launch shapes config 3 times: every cache of the list gets the oracle's grouped
    attention within the kernel tolerance (a sample of five caches is checked against the
    oracle, each distinct, and every output is finite)."""
    heads, kv_heads, cap = 14, 2, ctx_len
    assert hip.attention_list_plan(ctx_len, count, kv_heads) == plan
    vstride = hip.value_cache_bytes(cap, kv_heads) // (kv_heads * 64 * 2)
    rng = np.random.default_rng(ctx_len * 7 + count)
    kel, vel = kv_heads * cap * 64, kv_heads * 64 * vstride
    keys = rng.standard_normal(count * kel, dtype=np.float32).astype(np.float16).view(np.uint16)
    vals = rng.standard_normal(count * vel, dtype=np.float32).astype(np.float16).view(np.uint16)
    q = rng.standard_normal(heads * 64).astype(np.float32)
    print(f"list ctx {ctx_len} count {count} plan {plan}", flush=True)
    dk, dv, dq, dout = ctx.upload(keys), ctx.upload(vals), ctx.upload(q), ctx.empty(count * heads * 64 * 4)
    ctx.attention_list(dq, dk, dv, kel, vel, count, cap, dout, ctx_len - 1, heads, kv_heads)
    got = dout.read(count=count * heads * 64).reshape(count, heads * 64)
    assert np.all(np.isfinite(got))
    sample = sorted({0, 1, count // 2, int(rng.integers(2, count - 1)), count - 1})
    for i in sample:
        kr = O.f16_to_f32(keys[i * kel:(i + 1) * kel]).reshape(kv_heads, cap, 64)
        vr = O.f16_to_f32(vals[i * vel:(i + 1) * vel]).reshape(kv_heads, 64, vstride)[:, :, :ctx_len]
        K = np.ascontiguousarray(kr.transpose(1, 0, 2).reshape(ctx_len, -1))
        V = np.ascontiguousarray(vr.transpose(2, 0, 1).reshape(ctx_len, -1))
        ref = O.grouped_attention(q, K, V, 1, ctx_len - 1, heads, kv_heads, 64)
        err = rel_err(got[i], ref)
        print(f"  cache {i}: rel {err:.2e}", flush=True)
        assert err <= KERNEL_REL
    free(dk, dv, dq, dout)


@pytest.mark.parametrize("kind", KINDS)
def test_decode_attention_32k(ctx, hip, kind):
    ctx_len, heads, kv_heads = 32768, 14, 2
    kc, vc, kr, vr = kv_setup(ctx, hip, ctx_len, ctx_len, 5)
    q = np.random.default_rng(9).standard_normal(heads * 64).astype(np.float32)
    dq, dout = ctx.upload(q), ctx.empty(heads * 64 * 4)
    ctx.attention(dq, kc, vc, ctx_len, dout, 1, ctx_len - 1, heads, kv_heads, kind=kind)
    got = dout.read(count=heads * 64)
    ref = O.grouped_attention(q, kr, vr, 1, ctx_len - 1, heads, kv_heads, 64)
    check_attention(got, ref, kind != "exact")
    free(kc, vc, dq, dout)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("seq,past", [(5, 0), (3, 7), (70, 60), (130, 0), (512, 0), (33, 1000)])
def test_prefill_attention_matches_oracle(ctx, hip, seq, past, kind):
    heads, kv_heads = 14, 2
    total = past + seq
    kc, vc, kr, vr = kv_setup(ctx, hip, total, total, seq * 31 + past)
    q = np.random.default_rng(seq).standard_normal(seq * heads * 64).astype(np.float32)
    dq, dout = ctx.upload(q), ctx.empty(q.nbytes)
    ctx.attention(dq, kc, vc, total, dout, seq, past, heads, kv_heads, kind=kind)
    got = dout.read(count=q.size)
    ref = O.grouped_attention(q, kr, vr, seq, past, heads, kv_heads, 64)
    print(f"prefill attention seq {seq} past {past} {kind}: rel {rel_err(got, ref):.2e}")
    check_attention(got, ref, kind != "exact")
    free(kc, vc, dq, dout)


@pytest.mark.parametrize("kind", KINDS)
def test_prefill_attention_rows_equal_decode_rows_bitwise(ctx, hip, kind):
    # Query t of a prefill and the same query run alone at context past+t+1 give the same bits
    # (the MFMA form too: keys a query does not see enter its sums as exact zeros).
    seq, past, heads = 6, 100, 14
    total = past + seq
    kc, vc, _, _ = kv_setup(ctx, hip, total, total, 77)
    q = np.random.default_rng(3).standard_normal(seq * heads * 64).astype(np.float32)
    dq, dout = ctx.upload(q), ctx.empty(q.nbytes)
    ctx.attention(dq, kc, vc, total, dout, seq, past, heads, 2, kind=kind)
    full = dout.read(count=q.size).reshape(seq, -1)
    for t in range(seq):
        dq1, d1 = ctx.upload(q.reshape(seq, -1)[t]), ctx.empty(heads * 64 * 4)
        ctx.attention(dq1, kc, vc, total, d1, 1, past + t, heads, 2, kind=kind)
        np.testing.assert_array_equal(d1.read(count=heads * 64).view(np.uint32), full[t].view(np.uint32))
        free(dq1, d1)
    free(kc, vc, dq, dout)


@pytest.mark.parametrize("kind", KINDS)
def test_attention_first_position_returns_value(ctx, hip, kind):
    kc, vc, kr, vr = kv_setup(ctx, hip, 4, 1, 8)
    q = np.random.default_rng(0).standard_normal(14 * 64).astype(np.float32)
    dq, dout = ctx.upload(q), ctx.empty(14 * 64 * 4)
    ctx.attention(dq, kc, vc, 4, dout, 1, 0, 14, 2, kind=kind)
    got = dout.read(count=14 * 64).reshape(14, 64)
    for h in range(14):
        np.testing.assert_array_equal(got[h], vr[0, (h // 7) * 64:(h // 7 + 1) * 64])
    free(kc, vc, dq, dout)


@pytest.mark.parametrize("n", [1, 4864, 100003])
def test_swiglu_matches_oracle(ctx, hip, n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = (rng.standard_normal(n) * 2).astype(np.float32)
    dg, du = ctx.upload(g), ctx.upload(u)
    ctx.swiglu(dg, du, n)
    assert ulps(dg.read(count=n), O.swiglu(g, u)) <= 1
    free(dg, du)


def test_add_is_exact(ctx, hip):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(896).astype(np.float32)
    d = rng.standard_normal(896).astype(np.float32)
    dx, dd = ctx.upload(x), ctx.upload(d)
    ctx.add(dx, dd, 896)
    np.testing.assert_array_equal(dx.read(count=896), x + d)
    free(dx, dd)


@pytest.mark.parametrize("src_off,dst_off,n", [(0, 0, 1 << 20), (16, 48, 4096), (3, 5, 1001), (0, 0, 0),
                                               (0, 0, 7)])
def test_copy_moves_exactly_the_range(ctx, hip, src_off, dst_off, n):
    """GpuContext.copy (device.js:168-175): bytes [src_off, +n) land at dst_off, nothing
    around them changes (16-byte vector path when aligned, byte path otherwise)."""
    rng = np.random.default_rng(9)
    src = rng.integers(0, 256, size=n + 64, dtype=np.uint8)
    dst = rng.integers(0, 256, size=n + 64, dtype=np.uint8)
    ds, dd = ctx.upload(src), ctx.upload(dst)
    ctx.copy(ds, src_off, dd, dst_off, n)
    want = dst.copy()
    want[dst_off:dst_off + n] = src[src_off:src_off + n]
    np.testing.assert_array_equal(dd.read(np.uint8, n + 64), want)
    free(ds, dd)


def test_copy_rejects_overlap(ctx, hip):
    d = ctx.upload(np.zeros(256, np.uint8))
    with pytest.raises(hip.QwenHipError, match="overlap"):
        ctx.copy(d, 0, d, 16, 64)
    free(d)


@pytest.mark.parametrize("case", ["random", "ties", "nan0", "nan_mid", "inf", "neg", "tiny", "all_nan"])
def test_argmax_matches_strict_scan(ctx, hip, case):
    n = 151936 if case not in ("tiny",) else 3
    rng = np.random.default_rng(len(case))
    v = rng.standard_normal(n).astype(np.float32)
    if case == "ties":
        v[[100, 50000, 150000]] = 9.0
    elif case == "nan0":
        v[0] = np.nan
    elif case == "nan_mid":
        v[rng.integers(0, n, 100)] = np.nan
        v[77] = 8
    elif case == "inf":
        v[[9, 99999]] = np.inf
    elif case == "neg":
        v = -np.abs(v) - 1
    elif case == "all_nan":
        v[:] = np.nan
    dv = ctx.upload(v)
    assert ctx.argmax(dv, n) == O.argmax(v)
    free(dv)
