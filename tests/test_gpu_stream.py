"""The decode matvec launches on streaming grids (qh_decode_kernel_time_stream): the loop forms
of k_fused -- the grouped loop with its batched epilogues, flat weight lists, buffer-resource
loads and the chunk held in registers (q|k|v, o-proj, gate|up), and the ring loop (down, the
output head) -- must give the decode step's own launch shape's outputs bit for bit. The library
checks that on the first and the last copy of every list it times and fails the call otherwise,
so streaming each role over each weight format, both numerics and both team shapes (one and
several chunks per lane) is the parity test. The model's own decode must be untouched."""
import pytest

pytestmark = pytest.mark.gpu

CASES = [
    # (layer format, numerics, hidden, heads, kv_heads, intermediate)
    ("int8", "fast", 512, 8, 2, 1024),    # 32 chunks per row: 32-lane teams
    ("f16", "fast", 1024, 16, 2, 2048),   # 128 chunks per row: 64-lane teams, two chunks per lane
    ("int4", "exact", 128, 2, 1, 256),    # the f64 core
    ("int4", "fast", 640, 10, 2, 1280),   # 20 chunks per row, a partial team
]


@pytest.mark.parametrize("fmt,numerics,hidden,heads,kv_heads,inter", CASES)
def test_streaming_grids_match_the_step_launch(ctx, hip, fmt, numerics, hidden, heads, kv_heads, inter):
    cfg = hip.ModelConfig(hidden=hidden, intermediate=inter, layers=2, heads=heads, kv_heads=kv_heads, vocab=1000)
    ckpt = hip.synthesize_checkpoint(cfg, seed=21)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, fmt, 128, "int8"), cfg, maxPositions=96,
                              numerics=numerics)
    prompt = hip.synth_tokens(21, "stream.prompt", cfg.vocab, 33)
    a, b = model.newCache(80), model.newCache(80)
    first = model.forward_tokens(prompt, a)["argmax"]
    model.forward_tokens(prompt, b)
    for role in ("qkv", "oproj", "gateup", "down", "head"):
        for bpc in (1, 3):
            us, copies = model.kernel_time_stream(a, role, bpc, 24 << 20, 1)  # >= 2 copies of each
            print(f"{fmt}/{numerics} stream {role} x{bpc}: {copies} copies, {us:.2f} us")
            assert us > 0 and copies >= 2, (role, bpc, us, copies)
    a.length = len(prompt)
    assert list(model.decode(a, first, 8)) == list(model.decode(b, first, 8))
    a.destroy()
    b.destroy()
    model.destroy()


def test_streaming_grids_outside_the_flat_list(ctx, hip):
    """The grouped loop's other branch, one copy per grid row: a list of one copy, and a list
    whose weight bytes pass the 2 GiB a flat list's 32-bit buffer offsets reach (2.5 GiB of
    q|k|v copies, 286,720 weight bytes each). Both checked by the library against the step's
    launch shape as above."""
    cfg = hip.ModelConfig(hidden=640, intermediate=1280, layers=1, heads=10, kv_heads=2, vocab=1000)
    ckpt = hip.synthesize_checkpoint(cfg, seed=22)
    model = hip.GpuModel.load(ctx, hip.device_tensors(ckpt, cfg, "int4", 128, "int8"), cfg, maxPositions=64)
    c = model.newCache(48)
    model.forward_tokens(hip.synth_tokens(22, "stream.one", cfg.vocab, 20), c)
    for role in ("qkv", "oproj", "gateup"):
        us, copies = model.kernel_time_stream(c, role, 2, 1, 1)
        assert us > 0 and copies == 1, (role, us, copies)
    us, copies = model.kernel_time_stream(c, "qkv", 2, 5 << 29, 1)
    print(f"qkv over {copies} copies: {us:.1f} us")
    assert us > 0 and copies * (896 * 320) >= 1 << 31, copies
    c.destroy()
    model.destroy()
