"""The loader's conversion on the device (qh_quantize, qh_model_load_tensor) against the
oracle's restatement of the reference quantizer (src/core/quantize.js:36-132) and f16
narrowing (src/core/dtype.js:81-113): codes, scales, zero points and f16 bits equal bit for
bit, from bf16 and f32 sources, including the values the reference's f64 arithmetic and
Math.min/Math.max give a meaning to (NaN, infinities, signed zeros, subnormals, rows whose
f32 scale underflows while the f64 scale the codes use does not)."""
import numpy as np
import pytest

import oracle_lib as O

pytestmark = pytest.mark.gpu

SPECIAL_F32 = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-45, 3.4e38, -3.4e38,
                        65504.0, 65520.0, 2.0 ** -25, 6.0e-8, 2.98e-8, 1.0 + 2.0 ** -11,
                        1.0 + 3 * 2.0 ** -11], np.float32)
# NaN bit patterns with payloads (quiet and signalling, both signs) for the narrowing.
NAN_BITS = np.array([0x7F800001, 0x7FBFE000, 0xFF812345, 0x7FC00000, 0xFFFFFFFF, 0x7F802000],
                    np.uint32)


def planted_f32(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[1, :] = 0.0                         # all-zero row / groups: scale 0, codes 0
    w[2, :] = -0.0
    w[3, 5] = 1.0                         # an outlier
    w[4, ::7] = np.nan                    # scattered NaN: skipped by the peak, code 0
    w[5, 3] = np.inf                      # infinite peak: scale inf, inverse 0
    w[6, 9] = -np.inf
    w[7, :] = np.nan                      # all NaN
    w[8, :len(SPECIAL_F32)] = SPECIAL_F32
    w[9, :] = np.float32(1e-44) * np.sign(w[9, :])   # f32 scale underflows, f64 scale does not
    w[10, :] = np.abs(w[10, :])           # one-signed rows / groups
    w[11, :] = -np.abs(w[11, :])
    if rows > 15:
        # Products exactly on a half-integer, rounded half away from zero (k + 1/2 is exact in
        # bf16 too): int8, a row peak of 127 makes the scale 1 (row 13); int4, every group of
        # 16 or more aligned elements spanning 0 .. 15 does (row 15).
        ties = np.arange(cols) % 32 - 15.5
        ties[::32] = 127.0
        w[13, :] = ties
        span = np.arange(cols) % 16 - 1.5
        span[::16] = 0.0
        span[1::16] = 15.0
        w[15, :] = span
        # A scale of 3 (peak 381), whose inverse is inexact in f32 and f64 alike: odd multiples
        # of 1.5 give products on, or within rounding of, k + 1/2 in both.
        odd = 1.5 * (2 * (np.arange(cols) % 40) - 39)
        odd[::40] = 381.0
        w[14, :] = odd
    return w


def planted_bf16(rows, cols, seed):
    # The top half of each f32 (any bits serve: the expectation widens these same bits).
    bits = (planted_f32(rows, cols, seed).view(np.uint32) >> 16).astype(np.uint16)
    bits[12, :4] = [0x7FC1, 0xFF81, 0x7F80, 0x0001]   # NaN payloads, inf, smallest subnormal
    return bits


def source(hip, src, rows, cols, seed):
    """(src_format, host array, its exact f32 widening)."""
    if src == "bf16":
        bits = planted_bf16(rows, cols, seed)
        return hip.FMT_BF16, bits, O.bf16_to_f32(bits)
    w = planted_f32(rows, cols, seed)
    return hip.FMT_F32, w, w


def bits32(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("src", ["bf16", "f32"])
@pytest.mark.parametrize("rows,cols", [(16, 896), (896, 896), (64, 4864), (13, 100)])
def test_int8_matches_oracle(ctx, hip, src, rows, cols):
    fmt, host, wide = source(hip, src, rows, cols, rows + cols)
    d = ctx.upload(host)
    data, scales, _ = ctx.quantize(d, fmt, rows, cols, hip.FMT_INT8)
    q = data.read(np.int8, rows * cols).reshape(rows, cols)
    s = scales.read(np.float32, rows)
    oq, os_ = O.quantize_int8(wide)
    np.testing.assert_array_equal(q, oq)
    np.testing.assert_array_equal(bits32(s), bits32(os_))
    assert s[1] == 0 and s[7] == 0 and np.isinf(s[5])
    for b in (d, data, scales):
        b.free()


@pytest.mark.parametrize("src", ["bf16", "f32"])
@pytest.mark.parametrize("rows,cols,group", [(16, 896, 128), (896, 896, 128), (64, 4864, 128),
                                             (16, 256, 32), (16, 96, 2), (14, 896, 896), (13, 200, 100)])
def test_int4_matches_oracle(ctx, hip, src, rows, cols, group):
    fmt, host, wide = source(hip, src, rows, cols, rows * cols + group)
    d = ctx.upload(host)
    data, scales, zeros = ctx.quantize(d, fmt, rows, cols, hip.FMT_INT4, group)
    ng = rows * (cols // group)
    q = data.read(np.uint8, rows * cols // 2).reshape(rows, cols // 2)
    s, z = scales.read(np.float32, ng), zeros.read(np.float32, ng)
    oq, os_, oz = O.quantize_int4(wide, group)
    np.testing.assert_array_equal(q, oq)
    np.testing.assert_array_equal(bits32(s), bits32(os_).ravel())
    np.testing.assert_array_equal(bits32(z), bits32(oz).ravel())
    for b in (d, data, scales, zeros):
        b.free()


@pytest.mark.parametrize("src", ["bf16", "f32"])
def test_f16_narrowing_matches_oracle(ctx, hip, src):
    rows, cols = 24, 640
    fmt, host, wide = source(hip, src, rows, cols, 5)
    if src == "f32":
        host = host.copy()
        host.view(np.uint32)[13, :len(NAN_BITS)] = NAN_BITS
        wide = host
    d = ctx.upload(host)
    data, _, _ = ctx.quantize(d, fmt, rows, cols, hip.FMT_F16)
    got = data.read(np.uint16, rows * cols).reshape(rows, cols)
    np.testing.assert_array_equal(got, O.f32_to_f16(wide))
    d.free()
    data.free()


class At:
    """A device address inside a buffer, as the bindings take it."""

    def __init__(self, buf, offset):
        self.ptr = buf.ptr + offset


@pytest.mark.parametrize("n", [7, 39, 4096 + 5])
@pytest.mark.parametrize("skip", [0, 1])
def test_conversion_tails_and_unaligned_sources(ctx, hip, n, skip):
    # n % 8 values past the last 16-byte vector, and (skip 1) a source one value past a 16-byte
    # boundary: the one-value-per-thread kernels and the general int8 / int4 forms.
    rng = np.random.default_rng(n + skip)
    w = (rng.standard_normal(n + 8) * 3).astype(np.float32)
    w[1], w[4] = np.nan, -np.inf
    bits = (w.view(np.uint32) >> 16).astype(np.uint16)
    for fmt_src, host, wide in ((hip.FMT_BF16, bits, O.bf16_to_f32(bits)), (hip.FMT_F32, w, w)):
        d = ctx.upload(host)
        src = At(d, skip * host.itemsize)
        want = wide[skip:skip + n]
        h16, _, _ = ctx.quantize(src, fmt_src, 1, n, hip.FMT_F16)
        np.testing.assert_array_equal(h16.read(np.uint16, n), O.f32_to_f16(want))
        f32, _, _ = ctx.quantize(src, fmt_src, 1, n, hip.FMT_F32)
        np.testing.assert_array_equal(f32.read(np.uint32, n), want.view(np.uint32))
        cols = n - n % 8
        if cols == 0:
            for b in (d, h16, f32):
                b.free()
            continue
        q, s, _ = ctx.quantize(src, fmt_src, 1, cols, hip.FMT_INT8)
        oq, os_ = O.quantize_int8(want[None, :cols])
        np.testing.assert_array_equal(q.read(np.int8, cols), oq[0])
        np.testing.assert_array_equal(bits32(s.read(np.float32, 1)), bits32(os_))
        q4, s4, z4 = ctx.quantize(src, fmt_src, 1, cols, hip.FMT_INT4, 8)
        oq, os_, oz = O.quantize_int4(want[None, :cols], 8)
        np.testing.assert_array_equal(q4.read(np.uint8, cols // 2), oq[0])
        np.testing.assert_array_equal(bits32(s4.read(np.float32, cols // 8)), bits32(os_).ravel())
        np.testing.assert_array_equal(bits32(z4.read(np.float32, cols // 8)), bits32(oz).ravel())
        for b in (d, h16, f32, q, s, q4, s4, z4):
            b.free()


def test_bf16_widening_is_exact(ctx, hip):
    bits = np.arange(1 << 16, dtype=np.uint16).reshape(256, 256)   # every bf16 value
    d = ctx.upload(bits)
    data, _, _ = ctx.quantize(d, hip.FMT_BF16, 256, 256, hip.FMT_F32)
    np.testing.assert_array_equal(data.read(np.uint32, 1 << 16).reshape(256, 256),
                                  bits.astype(np.uint32) << 16)
    d.free()
    data.free()


def test_full_size_output_projection(ctx, hip):
    # The tied embedding of Qwen2.5-0.5B [151936, 896] as the int8 output projection, and a
    # down projection [896, 4864] as int4: the loader's two largest conversions.
    rows, cols = 151936, 896
    bits = hip.synth_bf16(1, "model.embed_tokens.weight", 0.02, rows * cols).reshape(rows, cols)
    d = ctx.upload(bits)
    data, scales, _ = ctx.quantize(d, hip.FMT_BF16, rows, cols, hip.FMT_INT8)
    oq, os_ = O.quantize_int8(O.bf16_to_f32(bits))
    np.testing.assert_array_equal(data.read(np.int8, rows * cols).reshape(rows, cols), oq)
    np.testing.assert_array_equal(bits32(scales.read(np.float32, rows)), bits32(os_))
    for b in (d, data, scales):
        b.free()
    rows, cols = 896, 4864
    bits = hip.synth_bf16(1, "mlp.down_proj.weight", 0.02, rows * cols).reshape(rows, cols)
    d = ctx.upload(bits)
    data, scales, zeros = ctx.quantize(d, hip.FMT_BF16, rows, cols, hip.FMT_INT4, 128)
    oq, os_, oz = O.quantize_int4(O.bf16_to_f32(bits), 128)
    np.testing.assert_array_equal(data.read(np.uint8, rows * cols // 2).reshape(rows, cols // 2), oq)
    np.testing.assert_array_equal(bits32(scales.read(np.float32, oq.shape[0] * 38)), bits32(os_).ravel())
    np.testing.assert_array_equal(bits32(zeros.read(np.float32, oq.shape[0] * 38)), bits32(oz).ravel())
    for b in (d, data, scales, zeros):
        b.free()


def test_argument_errors(ctx, hip):
    d = ctx.upload(np.zeros((4, 96), np.float32))
    with pytest.raises(hip.RangeError, match="does not divide"):
        ctx.quantize(d, hip.FMT_F32, 4, 96, hip.FMT_INT4, 64)
    with pytest.raises(hip.QwenHipError, match="even"):
        ctx.quantize(d, hip.FMT_F32, 4, 96, hip.FMT_INT4, 3)
    with pytest.raises(hip.RangeError, match="at least 2"):
        ctx.quantize(d, hip.FMT_F32, 4, 96, hip.FMT_INT4, 1)
    with pytest.raises(hip.QwenHipError, match="bf16 or f32"):
        ctx.quantize(d, hip.FMT_INT8, 4, 96, hip.FMT_F16)
    with pytest.raises(hip.QwenHipError, match="writes"):
        ctx.quantize(d, hip.FMT_F32, 4, 96, hip.FMT_BF16)
    d.free()


def tiny(hip):
    return hip.ModelConfig(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=1000)


@pytest.mark.parametrize("scheme", ["f16", "int8", "int4"])
@pytest.mark.parametrize("src", ["bf16", "f32"])
def test_device_loaded_model_equals_host_quantized_model(ctx, hip, scheme, src):
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=9)
    lm = "int8" if scheme != "f16" else "f16"
    host = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, scheme, 128, lm), cfg, maxPositions=64)
    src_ckpt = ckpt if src == "bf16" else {
        k: (v if k == "model.embed_tokens.weight" else hip.bf16_to_f32(v)) for k, v in ckpt.items()}
    dev = hip.GpuModel.load_checkpoint(ctx, src_ckpt, cfg, scheme, 128, lm, maxPositions=64)
    assert dev.device_bytes == host.device_bytes
    prompt = hip.synth_tokens(9, "prompt", cfg.vocab, 7)
    ca, cb = host.newCache(32), dev.newCache(32)
    a, b = host.forward_tokens(prompt, ca), dev.forward_tokens(prompt, cb)
    np.testing.assert_array_equal(bits32(a["logits"]), bits32(b["logits"]))
    np.testing.assert_array_equal(host.decode(ca, a["argmax"], 8), dev.decode(cb, b["argmax"], 8))
    for x in (ca, cb, host, dev):
        x.destroy()


def test_load_tensor_rejects_what_set_tensor_rejects(ctx, hip):
    cfg = tiny(hip)
    ckpt = hip.synthesize_checkpoint(cfg, seed=9)
    name = "model.layers.0.mlp.down_proj.weight"
    with pytest.raises(hip.QwenHipError, match="expected shape"):
        hip.GpuModel.load_checkpoint(ctx, {**ckpt, name: ckpt[name].T.copy()}, cfg, "int4", 128)
    with pytest.raises(ValueError, match="bf16 bits"):
        hip.GpuModel.load_checkpoint(ctx, {**ckpt, name: ckpt[name].astype(np.float64)}, cfg, "int4", 128)
    with pytest.raises(hip.QwenHipError):
        hip.GpuModel.load_checkpoint(ctx, ckpt, cfg, "int4", 96)
