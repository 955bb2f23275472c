"""The measurement entry points bench.py reports beside the decode step: a decode launch timed
cold over copies of its operands (qh_decode_kernel_time_cold, and on streaming grids
qh_decode_kernel_time_stream), the pure-read ceiling and the
launch floor probes. They must run every role, report sane figures and leave the model and its
cache as they were (the cold timing writes only the position's own decode scratch)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_cold_timing_runs_every_role_and_leaves_the_decode_intact(ctx, hip):
    cfg = hip.ModelConfig(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=1000)
    ckpt = hip.synthesize_checkpoint(cfg, seed=11)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int4", 128, "int8"), cfg, maxPositions=128)
    prompt = hip.synth_tokens(11, "cold.prompt", cfg.vocab, 40)
    a, b = model.newCache(96), model.newCache(96)
    first = model.forward_tokens(prompt, a)["argmax"]
    model.forward_tokens(prompt, b)
    for role in ("qkv", "attention", "oproj", "gateup", "down", "head"):
        us, copies = model.kernel_time_cold(a, role, 4 << 20, 2)
        print(f"cold {role}: {copies} copies, {us:.2f} us")
        assert us > 0 and copies >= 2, (role, us, copies)
    for role in ("qkv", "oproj", "gateup", "down", "head"):
        for bpc in (1, 3):  # streaming grids: each team walks several rows (the multi-item form)
            us, copies = model.kernel_time_stream(a, role, bpc, 4 << 20, 2)
            print(f"stream {role} x{bpc}: {copies} copies, {us:.2f} us")
            assert us > 0 and copies >= 2, (role, bpc, us, copies)
    with pytest.raises(hip.QwenHipError, match="blocks_per_copy"):
        model.kernel_time_stream(a, "attention", 2, 4 << 20, 1)
    a.length = len(prompt)
    assert list(model.decode(a, first, 12)) == list(model.decode(b, first, 12))
    a.destroy()
    b.destroy()
    model.destroy()


def test_exact_numerics_has_no_attention_list(ctx, hip):
    cfg = hip.ModelConfig(hidden=128, intermediate=256, layers=2, heads=2, kv_heads=1, vocab=1000)
    ckpt = hip.synthesize_checkpoint(cfg, seed=12)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int8", 128, "int8"), cfg, maxPositions=64,
                              numerics="exact")
    c = model.newCache(32)
    model.forward_tokens([1, 2, 3], c)
    with pytest.raises(hip.QwenHipError, match="fast-numerics split-K"):
        model.kernel_time_cold(c, "attention", 4 << 20, 1)
    us, copies = model.kernel_time_cold(c, "gateup", 4 << 20, 1)
    assert us > 0 and copies >= 2
    c.destroy()
    model.destroy()


def test_read_ceiling_and_launch_floor(ctx):
    gbs = ctx.read_ceiling(256 << 20, 3)
    empty, static, dependent = ctx.launch_floor(0), ctx.launch_floor(2), ctx.launch_floor(1)
    print(f"read ceiling {gbs:.0f} GB/s; launch {empty:.2f} / {static:.2f} / {dependent:.2f} us")
    assert 100 < gbs < 10000
    assert 0 < empty < 50 and 0 < static < 50 and 0 < dependent < 50
