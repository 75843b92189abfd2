"""Engines on separate streams at the same time: two dual-stream engines (each step's FFN-down runs as a stream-K
launch, each stream with its own partials workspace) and an SDXL engine run concurrently, and every result equals,
bit for bit, the same engine's result when it ran alone."""
import numpy as np
import pytest

import mkimage as M

pytestmark = pytest.mark.gpu

D, H, F, E = 3072, 24, 12288, 3584
SDXL_B = dict(blocks=2, dim=1280, heads=20, head_dim=64, ffn=5120, text_dim=2048)


def dual_engine(seed):
    # one block of the 1024x1024 shape: 4096 image + 256 text tokens, CFG batch 2 (8704 rows: the FFN-down GEMM's
    # 408 tiles take one whole wave and a stream-K tail)
    e = M.Engine(M.FAMILY_DUAL, blocks=1, dim=D, heads=H, head_dim=128, ffn=F, text_dim=E)
    e.init_random(seed)
    rng = np.random.default_rng(seed)
    for s in (0, 1):
        e.begin(rng.standard_normal((256, E)).astype(np.float32), 64, 64, s)
    lat = M.Dev.from_array(rng.standard_normal((4096, 64)).astype(np.float32))
    return e, lat


def test_dual_and_sdxl_engines_on_separate_streams_match_their_solo_bits(gpu):
    duals = [dual_engine(s) for s in (1, 2)]
    sx = M.Engine(M.FAMILY_SDXL, **SDXL_B)
    sx.init_random(3)
    rng = np.random.default_rng(3)
    for s in (0, 1):
        sx.begin(rng.standard_normal((77, 2048)).astype(np.float32), 32, 32, s)
    n = 1024
    x = M.Dev.from_array(rng.standard_normal((2, n, 1280)).astype(np.float32))
    outs = [M.Dev(4096 * 64 * 4) for _ in duals]
    y = M.Dev(2 * n * 1280 * 4)

    def read():
        return [o.to_array(np.float32, (4096, 64)) for o in outs] + [y.to_array(np.float32, (2, n, 1280))]

    # alone: one engine at a time, each finished before the next starts
    for (e, lat), o in zip(duals, outs):
        e.step_cfg_device(lat, 0.9, 0.85, 4.0, o)
        M.call("mk_stream_synchronize", e.stream())
    sx.sdxl_forward(x, 2, n, y)
    solo = read()
    for a in solo:
        assert np.isfinite(a).all()
    for a in outs + [y]:
        M.call("mk_memset", a.p, 0, a.nbytes)
    M.sync()
    # together: both dual steps queued on their engines' streams, the SDXL pass runs (and waits for its own stream)
    # while they are in flight
    for rep in range(2):
        for (e, lat), o in zip(duals, outs):
            e.step_cfg_device(lat, 0.9, 0.85, 4.0, o)
        sx.sdxl_forward(x, 2, n, y)
        for e, _ in duals:
            M.call("mk_stream_synchronize", e.stream())
        for got, want in zip(read(), solo):
            assert np.array_equal(got, want), f"repeat {rep}"
    for e, _ in duals:
        e.close()
    sx.close()
