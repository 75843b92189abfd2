"""Engine parity on the GPU: whole steps through the C ABI (mk_begin / mk_step / mk_step_cfg, mk_sdxl_forward)
against the oracle's graphs on the same seeded weights and inputs.

Tolerances (block and step outputs): cosine >= 0.9995 and max-rel = max|g - w| / max|w| <= 2e-2 with bf16 weights,
<= 5e-2 with fp8 weights. The reference's own Diff (relative RMS error, lowest row cosine) is reported with them.
"""
import numpy as np
import pytest

import mkimage as M
import mkref as R

pytestmark = pytest.mark.gpu

# The tiny MMDiT: 2 dual-stream blocks, hidden 512, 4 heads x 128, FFN 2048; 256 image tokens (a 16 x 16 grid of
# 2x2-patched 16-channel latents), 64 text tokens of width 512; sigma 0.5, seed 0.
TINY = dict(blocks=2, dim=512, heads=4, head_dim=128, ffn=2048, text_dim=512)
H_, W_, S_ = 16, 16, 64


def within(got, want, width, cos=0.9995, max_rel=2e-2):
    d = R.diff(got, want, width)
    assert d["cos"] >= cos and d["max_rel"] <= max_rel, d
    return d


def make_pair(family, fp8=False, seed=0, wstd=0.02, dims=TINY, f16=False):
    m = R.Model({M.FAMILY_DUAL: R.DUAL, M.FAMILY_Q21: R.Q21, M.FAMILY_SDXL: R.SDXL}[family], **dims, fp8=fp8,
                seed=seed, wstd=wstd, f16=f16)
    e = M.Engine(family, **dims, weight_dtype=M.FP8 if fp8 else M.F16 if f16 else M.BF16)
    M.upload_model(e, m.tensors())
    return m, e


def inputs(seed=0, B=2, S=S_, h=H_, w=W_, E=512):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((B, S, E)).astype(np.float32),
            rng.standard_normal((B, h * w, 64)).astype(np.float32))


@pytest.mark.parametrize("fp8", [False, True])
def test_dual_step_matches_oracle(gpu, fp8):
    m, e = make_pair(M.FAMILY_DUAL, fp8)
    prompt, lat = inputs()
    want_p = {}
    want = m.dual_step(prompt[:1], lat[:1], H_, W_, 0.5, want_p)
    e.begin(prompt[0], H_, W_, 0)
    got_p = {}
    e.set_probe(got_p)
    got = e.step(lat[0], 0.5, 0)
    tol = 5e-2 if fp8 else 2e-2
    within(got, want[0], 64, max_rel=tol)
    within(got_p[("temb", -1)], want_p[("temb", -1)], 512, cos=0.99999, max_rel=1e-3)
    within(got_p[("modulation", -1)], want_p[("modulation", -1)], 512, cos=0.99999, max_rel=1e-3)
    for i in range(TINY["blocks"]):
        within(got_p[("block", i)], want_p[("block", i)], 512, max_rel=tol)


def test_dual_cfg_batch_matches_two_oracle_passes(gpu):
    m, e = make_pair(M.FAMILY_DUAL)
    prompt, lat = inputs(1)
    for s in (0, 1):
        e.begin(prompt[s], H_, W_, s)
    x = lat[0]
    sig, sig_next, g = 0.75, 0.6, 4.0
    got = e.step_cfg(x, sig, sig_next, g)
    v = m.dual_step(prompt, np.stack([x, x]), H_, W_, sig)  # [pos, neg]
    want = x + (sig_next - sig) * (v[1] + g * (v[0] - v[1]))
    # compare the update (the latents themselves dominate the value)
    within(got - x, want - x, 64)
    # and the batch of 2 equals the single-sample steps it stands for
    pos = e.step(x, sig, 0)
    neg = e.step(x, sig, 1)
    within(got - x, (sig_next - sig) * (neg + g * (pos - neg)), 64, cos=0.99999, max_rel=1e-3)


@pytest.mark.parametrize("S0,S1", [(64, 41), (23, 64)])
def test_dual_cfg_batch_ragged_prompts_matches_two_oracle_passes(gpu, S0, S1):
    # prompts of different lengths (the reference runs each slot with its own S, engine.cpp:475-477) still run as one
    # batch of 2: the shorter prompt padded, its padding rows masked as keys, each sample's RoPE at its own frame
    m, e = make_pair(M.FAMILY_DUAL)
    rng = np.random.default_rng(9)
    p = [rng.standard_normal((S0, 512)).astype(np.float32), rng.standard_normal((S1, 512)).astype(np.float32)]
    x = rng.standard_normal((H_ * W_, 64)).astype(np.float32)
    for s in (0, 1):
        e.begin(p[s], H_, W_, s)
    sig, sig_next, g = 0.7, 0.55, 3.5
    got = e.step_cfg(x, sig, sig_next, g)
    v = [m.dual_step(p[s][None], x[None], H_, W_, sig)[0] for s in (0, 1)]
    want = x + (sig_next - sig) * (v[1] + g * (v[0] - v[1]))
    within(got - x, want - x, 64)
    # each sample's velocity in the padded batch (guidance 1: the positive's, 0: the negative's) against its own
    # single-slot step: the padded sample's keys sit at other tile positions, so its attention sums run in another
    # order and a few bf16 roundings of the attention output flip (2^-9 each): within 5e-3, cosine 0.99999
    dt = sig_next - sig
    for gg, slot in ((1.0, 0), (0.0, 1)):
        v_b = (e.step_cfg(x, sig, sig_next, gg) - x) / dt
        within(v_b, e.step(x, sig, slot), 64, cos=0.99999, max_rel=5e-3)
    # the padded batch repeats bit for bit
    assert np.array_equal(e.step_cfg(x, sig, sig_next, g), got)


def test_init_random_equals_uploaded_oracle_weights(gpu):
    # the device RNG reproduces the CPU reference's weights bit for bit: the same step, the same bits
    m, e = make_pair(M.FAMILY_DUAL, seed=3)
    e2 = M.Engine(M.FAMILY_DUAL, **TINY)
    e2.init_random(3)
    prompt, lat = inputs(2)
    for eng in (e, e2):
        eng.begin(prompt[0], H_, W_, 0)
    assert np.array_equal(e.step(lat[0], 0.3, 0), e2.step(lat[0], 0.3, 0))


def test_init_random_fp8_equals_uploaded(gpu):
    m, e = make_pair(M.FAMILY_DUAL, fp8=True, seed=4)
    e2 = M.Engine(M.FAMILY_DUAL, **TINY, weight_dtype=M.FP8)
    e2.init_random(4)
    prompt, lat = inputs(3)
    for eng in (e, e2):
        eng.begin(prompt[0], H_, W_, 0)
    assert np.array_equal(e.step(lat[0], 0.3, 0), e2.step(lat[0], 0.3, 0))


Q21 = dict(blocks=2, dim=512, heads=4, head_dim=128, ffn=1536, text_dim=512)


def test_q21_steps_with_text_cache_match_oracle(gpu):
    # the reference's own graph: step 1 runs [text; image], step 2 only the image against the cached text K / V;
    # the oracle recomputes the whole sequence each time (equal, since text rows see only text keys at t = 0)
    m, e = make_pair(M.FAMILY_Q21, dims=Q21, wstd=0.05)
    prompt, lat = inputs(4, B=1, S=40, h=12, w=10)
    e.begin(prompt[0], 12, 10, 0)
    for step, sig in enumerate((0.9, 0.7)):
        got_p, want_p = {}, {}
        e.set_probe(got_p)
        got = e.step(lat[0], sig, 0)
        want = m.q21_step(prompt[0], lat[0], 12, 10, sig, want_p)
        within(got, want, 64)
        N = 12 * 10
        for i in range(2):  # the image rows of each block (step 2 runs only those)
            within(got_p[("block", i)].reshape(-1, 512)[-N:], want_p[("block", i)].reshape(-1, 512)[-N:], 512)


# The reference's own model at its own shape (qwen_image.hpp:37-38, the 2.1 graph of qwen_image.cpp:144-293): one block
# of width 4096 (32 heads x 128, SwiGLU 12288, f16 heads, causal text prefix), a 64 x 64 latent grid (1024 x 1024
# pixels) and 256 prompt rows of width 4096.
Q21_FULL = dict(blocks=1, dim=4096, heads=32, head_dim=128, ffn=12288, text_dim=4096)


def test_q21_full_shape_steps_with_text_cache_match_oracle(gpu):
    # step 1 over [text; image], then step 2 over the image rows against the cached text K / V; the probes
    # image_ref_test dit compares (tests/image_ref_test.cpp:127-164), each against the oracle's
    m, e = make_pair(M.FAMILY_Q21, dims=Q21_FULL, seed=5)
    h = w = 64
    N, D = h * w, Q21_FULL["dim"]
    prompt, lat = inputs(5, B=1, S=256, h=h, w=w, E=Q21_FULL["text_dim"])
    e.begin(prompt[0], h, w, 0)
    for step, sig in enumerate((0.9, 0.7)):
        print(f"q21 full shape: step {step + 1}, sigma {sig}", flush=True)
        got_p, want_p = {}, {}
        e.set_probe(got_p)
        got = e.step(lat[0], sig, 0)
        e.set_probe(None)
        want = m.q21_step(prompt[0], lat[0], h, w, sig, want_p)
        d = within(got, want, 64)
        print("  velocity", d, flush=True)
        for name in ("temb", "modulation"):
            within(got_p[(name, -1)], want_p[(name, -1)], D, cos=0.99999, max_rel=1e-3)
        if ("txt_in", -1) in got_p:  # step 1 only: later steps reuse the cached text
            within(got_p[("txt_in", -1)], want_p[("txt_in", -1)], D)
        within(got_p[("img_in", -1)], want_p[("img_in", -1)], D)
        for name, layer in (("block", 0), ("norm_out", -1)):  # the image rows (step 2 runs only those)
            d = within(got_p[(name, layer)].reshape(-1, D)[-N:], want_p[(name, layer)].reshape(-1, D)[-N:], D)
            print(f"  {name}", d, flush=True)


def test_q21_step_errors(gpu):
    e = M.Engine(M.FAMILY_Q21, **Q21)
    with pytest.raises(M.MkError, match="before begin"):
        e.step(np.zeros((4, 64), np.float32), 0.5, 0)
    with pytest.raises(M.MkError, match="slot"):
        e.begin(np.zeros((3, 512), np.float32), 2, 2, 2)
    for bad in (np.zeros((3, 500), np.float32), np.zeros((0, 512), np.float32)):
        with pytest.raises(M.MkError, match="rows of 512"):
            e.begin(bad, 2, 2, 0)
    e.begin(np.zeros((3, 512), np.float32), 2, 2, 0)
    with pytest.raises(M.MkError, match="latents"):
        e.step(np.zeros((5, 64), np.float32), 0.5, 0)


SDXL_A = dict(blocks=1, dim=640, heads=10, head_dim=64, ffn=2560, text_dim=2048)


def test_sdxl_block_matches_oracle(gpu):
    m, e = make_pair(M.FAMILY_SDXL, dims=SDXL_A, wstd=0.05)
    rng = np.random.default_rng(5)
    n, S = 1024, 77
    x = rng.standard_normal((2, n, 640)).astype(np.float32)
    ctx = rng.standard_normal((2, S, 2048)).astype(np.float32)
    for s in (0, 1):
        e.begin(ctx[s], 32, 32, s)
    xd, yd = M.Dev.from_array(x), M.Dev(x.nbytes)
    e.sdxl_forward(xd, 2, n, yd)
    got = yd.to_array(np.float32, x.shape)
    for b in range(2):
        want = m.sdxl_trans(x[b], ctx[b])
        within(got[b] - x[b], want - x[b], 640)


def test_attention_full_size_sampled_rows(gpu):
    # config 2 at its full size: B=2, 24 heads x 128, 4096 image + 256 text tokens, QK-RMSNorm and RoPE applied by
    # the heads kernel; 48 sampled query rows per (batch, head) checked against the oracle's softmax over all keys
    B, H, T, S = 2, 24, 4352, 256
    rng = np.random.default_rng(6)
    D = H * 128
    qkv = R.bf16_round(rng.standard_normal((B, T, 3 * D)).astype(np.float32))
    cs = R.rope_table(S, 64, 64)
    nq = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    nk = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    q_pad, k_pad = 4352, 4352
    Q, K, V = M.Dev(B * H * q_pad * 256), M.Dev(B * H * k_pad * 256), M.Dev(B * H * k_pad * 256)
    X, csd, nqd, nkd = M.Dev.from_array(M.bf16_bits(qkv)), M.Dev.from_array(cs), M.Dev.from_array(nq), \
        M.Dev.from_array(nk)
    for col0, w_, out, pad, tr in ((0, nqd, Q, q_pad, 0), (D, nkd, K, k_pad, 0), (2 * D, None, V, k_pad, 1)):
        M.call("mk_heads", X.p, B, T, 3 * D, T * 3 * D, col0, H, 128, w_.p if w_ else None, 1e-6,
               None if tr else csd.p, 0 if tr else 2, out.p, pad, 0, tr, M.BF16, None)
    O = M.Dev(B * T * D * 2)
    M.call("mk_attention", Q.p, K.p, V.p, O.p, M.BF16, B, H, H, 128, T, q_pad, T, k_pad, D, T * D, 0, 0,
           float(1 / np.sqrt(128)), None, None)
    M.sync()
    got = M.bf16_to_f32(O.to_array(np.uint16, (B, T, D)))
    rows = np.sort(rng.choice(T, 48, replace=False))
    for b in range(B):
        qh = R.heads_norm_rope(qkv[b], H, 128, col0=0, w=nq, cs=cs, rope=2)
        kh = R.heads_norm_rope(qkv[b], H, 128, col0=D, w=nk, cs=cs, rope=2)
        vh = R.heads_norm_rope(qkv[b], H, 128, col0=2 * D)
        qh, kh, vh = (R.bf16_round(a) for a in (qh, kh, vh))
        want = R.attention(np.ascontiguousarray(qh[None, :, rows]), kh[None], vh[None], 1 / np.sqrt(128))
        within(got[b, rows], want[0], 128, cos=0.9999, max_rel=2e-2)


def test_generate_guided_equals_the_stepwise_loop(gpu):
    # the device loop is the host loop of Engine::generate over mk_step_cfg, bit for bit
    m, e = make_pair(M.FAMILY_DUAL)
    prompt, lat = inputs(7)
    for s in (0, 1):
        e.begin(prompt[s], H_, W_, s)
    sig = M.sigmas(3, H_ * W_)
    got = e.generate(lat[0], sig, 4.0)
    x = lat[0]
    for i in range(3):
        x = e.step_cfg(x, sig[i], sig[i + 1], 4.0)
    assert np.array_equal(got, x)


def test_generate_unguided_matches_oracle_euler(gpu):
    # guidance 1: slot 0 only; two Euler steps against the oracle's velocity at each step
    m, e = make_pair(M.FAMILY_DUAL)
    prompt, lat = inputs(8)
    e.begin(prompt[0], H_, W_, 0)
    sig = M.sigmas(2, H_ * W_, terminal=0.1)
    got = e.generate(lat[0], sig, 1.0)
    x = lat[0].copy()
    for i in range(2):
        v = m.dual_step(prompt[:1], x[None], H_, W_, float(sig[i]))[0]
        x = x + (sig[i + 1] - sig[i]) * v
    within(got - lat[0], x - lat[0], 64)
    with pytest.raises(M.MkError, match="begin both"):
        e.generate(lat[0], sig, 3.0)
    for bad in (sig[:1], sig[:0]):  # no step to take: refused before the library reads sigmas[1]
        with pytest.raises(M.MkError, match="steps \\+ 1"):
            e.generate(lat[0], bad, 1.0)


FULL = dict(blocks=1, dim=3072, heads=24, head_dim=128, ffn=12288, text_dim=3584)


@pytest.mark.parametrize("fp8,side", [(False, 64), (True, 32)])
def test_full_size_block_matches_oracle(gpu, fp8, side):
    # the benchmark's shapes (hidden 3072, 24 x 128 heads, FFN 12288, 4096 image + 256 text tokens of width 3584; the
    # fp8 case at 1024 image tokens to keep the oracle quick), one block, one sample: the GPU step (device-initialised
    # weights, bit-equal to the oracle's) against the oracle
    m = R.Model(R.DUAL, **FULL, fp8=fp8, seed=11)
    e = M.Engine(M.FAMILY_DUAL, **FULL, weight_dtype=M.FP8 if fp8 else M.BF16)
    e.init_random(11)
    rng = np.random.default_rng(12)
    prompt = rng.standard_normal((256, 3584)).astype(np.float32)
    lat = rng.standard_normal((side * side, 64)).astype(np.float32)
    e.begin(prompt, side, side, 0)
    got_p, want_p = {}, {}
    e.set_probe(got_p)
    got = e.step(lat, 0.8, 0)
    want = m.dual_step(prompt[None], lat[None], side, side, 0.8, want_p)[0]
    tol = 5e-2 if fp8 else 2e-2
    within(got_p[("block", 0)], want_p[("block", 0)], 3072, max_rel=tol)
    within(got, want, 64, max_rel=tol)
