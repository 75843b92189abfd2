"""The VAE decoder on the GPU through the C ABI (mk_conv3x3, mk_vae_*), src/image/engine.cpp:862-954.

- mk_conv3x3 (implicit-GEMM 3x3 conv over the padded pixel grid, IEEE half operands as the reference's F16
  convolution weights and half inputs) against torch's conv2d in float64 on the same half operands: fp32
  accumulation, so max |g - w| / max |w| <= 1e-4.
- The whole decode against the oracle's decoder (pinned to torch's conv2d / interpolate / softmax by
  tests/test_oracle_graph.py, at the reference's precision points: half convolution operands, half queries and
  probabilities against fp32 keys and values) on the same counter-RNG weights: cosine >= 0.9995 and max-rel <= 2e-2,
  at every probe (conv_in, mid block, each up block, conv_out) and on the clamped RGBA.
- Checkpoint loading: the oracle's weights written as Wan-layout causal 3-D convs (3 time taps, the last one real)
  decode bit-identically to the same weights drawn on the device.
"""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from safetensors.torch import save_file

import mkimage as M
import mkref as R

pytestmark = pytest.mark.gpu


def within(got, want, width, cos=0.9995, max_rel=2e-2):
    d = R.diff(got, want, width)
    assert d["cos"] >= cos and d["max_rel"] <= max_rel, d
    return d


def grid_rows(h, w):
    return (h + 2) * (w + 2) + 2 * (w + 3)


def to_grid(img, c_pad):
    """[h][w][c] -> the padded grid [(h+2)(w+2) + 2(w+3)][c_pad] with zero ring, slack and padding channels."""
    h, w, c = img.shape
    g = np.zeros((grid_rows(h, w), c_pad), dtype=img.dtype)
    S = w + 3
    for y in range(h):
        r0 = S + (y + 1) * (w + 2) + 1
        g[r0:r0 + w, :c] = img[y]
    return g


def from_grid(g, h, w, c):
    S = w + 3
    return np.stack([g[S + (y + 1) * (w + 2) + 1:S + (y + 1) * (w + 2) + 1 + w, :c] for y in range(h)])


# (the 150 x 150 grids take 192-channel tiles: more than a wave of 64- or 128-channel ones; 96 and 288 output
# channels take 128 x 96 tiles; widths of 128, 256 and 512 tile the pixels only, the others the padded rows)
@pytest.mark.parametrize("h, w, c, n, add", [(5, 7, 64, 64, False), (16, 16, 128, 192, False),
                                             (9, 33, 192, 64, True), (32, 40, 384, 384, True),
                                             (1, 1, 64, 128, False), (64, 3, 64, 256, False),
                                             (150, 150, 64, 192, True), (150, 150, 64, 384, False),
                                             (40, 37, 192, 96, False), (150, 150, 64, 96, True),
                                             (5, 7, 128, 288, True), (1, 2, 64, 96, False),
                                             (4, 128, 64, 96, True), (8, 256, 64, 192, False),
                                             (3, 512, 128, 64, True), (40, 256, 192, 384, True)])
def test_conv3x3_matches_torch(gpu, h, w, c, n, add):
    rng = np.random.default_rng(h * 1000 + w)
    x = M.f16_bits(rng.standard_normal((h, w, c)).astype(np.float32))
    wt = rng.standard_normal((n, c, 3, 3)).astype(np.float32) / np.sqrt(9 * c)
    wb = M.f16_bits(wt)
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    packed = np.ascontiguousarray(wb.transpose(0, 2, 3, 1).reshape(n, 9 * c))  # [n][tap][c], tap = 3 dy + dx
    y0 = rng.standard_normal((grid_rows(h, w), n)).astype(np.float32)
    dx, dw, db = M.Dev.from_array(to_grid(x, c)), M.Dev.from_array(packed), M.Dev.from_array(bias)
    dy = M.Dev.from_array(y0)
    S = w + 3
    a = M.ConvArgs(int(dx), int(dw), int(db), int(dy) + S * n * 4, h, w, c, n, n, M.F32,
                   M.EPI_ADD if add else M.EPI_STORE)
    M.call("mk_conv3x3", ctypes.byref(a), None)
    M.sync()
    got = from_grid(dy.to_array(np.float32, y0.shape), h, w, n)
    xt = torch.from_numpy(M.f16_to_f32(x)).double().permute(2, 0, 1)[None]
    want = F.conv2d(xt, torch.from_numpy(M.f16_to_f32(wb)).double(), torch.from_numpy(bias).double(), padding=1)
    want = want[0].permute(1, 2, 0).numpy()
    if add:
        want = want + from_grid(y0, h, w, n)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err <= 1e-4, err
    # the slack rows stay as they were (at most the (h + 2)(w + 2) grid rows are written)
    out = dy.to_array(np.float32, y0.shape)
    assert np.array_equal(out[:S], y0[:S]) and np.array_equal(out[-S:], y0[-S:])


# half output (STORE): the 96-wide tile's 32-channel slices, a 192-wide tile, pixel-tiled and padded-row widths
@pytest.mark.parametrize("h, w, c, n", [(4, 128, 64, 96), (7, 9, 128, 96), (8, 256, 64, 192), (5, 6, 64, 128)])
def test_conv3x3_half_output(gpu, h, w, c, n):
    rng = np.random.default_rng(h * 100 + w + n)
    x = M.f16_bits(rng.standard_normal((h, w, c)).astype(np.float32))
    wb = M.f16_bits((rng.standard_normal((n, c, 3, 3)) / np.sqrt(9 * c)).astype(np.float32))
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    packed = np.ascontiguousarray(wb.transpose(0, 2, 3, 1).reshape(n, 9 * c))
    y0 = np.full((grid_rows(h, w), n), 0x7E00, dtype=np.uint16)  # NaN patterns: rows the conv must not write
    dx, dw, db = M.Dev.from_array(to_grid(x, c)), M.Dev.from_array(packed), M.Dev.from_array(bias)
    dy = M.Dev.from_array(y0)
    S = w + 3
    a = M.ConvArgs(int(dx), int(dw), int(db), int(dy) + S * n * 2, h, w, c, n, n, M.F16, M.EPI_STORE)
    M.call("mk_conv3x3", ctypes.byref(a), None)
    M.sync()
    out = dy.to_array(np.uint16, y0.shape)
    got = M.f16_to_f32(from_grid(out, h, w, n))
    xt = torch.from_numpy(M.f16_to_f32(x)).double().permute(2, 0, 1)[None]
    want = F.conv2d(xt, torch.from_numpy(M.f16_to_f32(wb)).double(), torch.from_numpy(bias).double(), padding=1)
    want = want[0].permute(1, 2, 0).numpy()
    # one half rounding of the fp32 result: within 2^-11 relative of the largest value
    assert np.abs(got - want).max() <= np.abs(want).max() * 2.0 ** -11, np.abs(got - want).max()
    assert np.array_equal(out[:S], y0[:S]) and np.array_equal(out[-S:], y0[-S:])


def test_conv3x3_rejects_bad_shapes(gpu):
    a = M.ConvArgs(16, 16, 0, 16, 4, 4, 96, 64, 64, M.F32, M.EPI_STORE)  # 96 channels: not a multiple of 64
    assert M.lib().mk_conv3x3(ctypes.byref(a), None) == 1
    a = M.ConvArgs(16, 16, 0, 16, 4, 4, 64, 64, 64, M.F16, M.EPI_ADD)  # accumulate into half
    assert M.lib().mk_conv3x3(ctypes.byref(a), None) == 1
    a = M.ConvArgs(16, 16, 0, 16, 4, 4, 64, 64, 64, M.BF16, M.EPI_STORE)  # bf16 output: the operands are half
    assert M.lib().mk_conv3x3(ctypes.byref(a), None) == 1
    a = M.ConvArgs(16, 16, 0, 16, 4, 4, 64, 160, 160, M.F32, M.EPI_STORE)  # 160 outputs: not of 64 or 96
    assert M.lib().mk_conv3x3(ctypes.byref(a), None) == 1


MEAN = np.linspace(-0.3, 0.3, 16).astype(np.float32)
STD = np.linspace(0.5, 2.0, 16).astype(np.float32)


# base 96 is Qwen-Image's: 384 / 192 / 96 channels (96-channel inputs dense, 96-channel outputs unpadded); at 2 x 32
# tokens the 192- and 96-channel levels are 256 and 512 pixels wide, so their convolutions tile the pixels only and
# their norms run in the epilogues, and the 192-channel level's last conv writes the 2x grid itself; at 2 x 64 the
# 384-channel level at 256 pixels wide does too
@pytest.mark.parametrize("base, h, w", [(16, 2, 2), (16, 2, 3), (32, 4, 4), (96, 4, 4), (96, 2, 32), (96, 2, 64)])
def test_vae_decode_matches_oracle(gpu, base, h, w):
    ref = R.Vae(base, seed=5, mean=MEAN, std=STD)
    vae = M.Vae(base, mean=MEAN, std=STD)
    vae.init_random(5)
    tokens = np.random.default_rng(base + h * 10 + w).standard_normal((h * w, 64)).astype(np.float32)
    want_p, got_p = {}, {}
    want = ref.decode(tokens, h, w, want_p)
    vae.set_probe(got_p)
    got = vae.decode(tokens, h, w)
    assert got.shape == (16 * h, 16 * w, 4) and np.all(got[..., 3] == 1)
    assert set(got_p) == set(want_p)
    widths = {("vae_conv_in", -1): 4 * base, ("vae_mid", -1): 4 * base, ("vae_up", 0): 2 * base,
              ("vae_up", 1): 2 * base, ("vae_up", 2): base, ("vae_up", 3): base, ("vae_out", -1): 3}
    for k, wd in widths.items():
        within(got_p[k], want_p[k], wd)
    within(got[..., :3], want[..., :3], 3)
    # the decode is deterministic and probes do not change it
    vae.set_probe(None)
    assert np.array_equal(vae.decode(tokens, h, w), got)


def test_vae_mid_attention_over_256_pixels(gpu):
    # 8 x 8 tokens: 256 pixels in the mid block, whose one-head attention (scores, softmax, P V) runs over all of them;
    # the mid block's output against the oracle's exact softmax (the smaller decodes above check the whole path).
    ref = R.Vae(16, seed=7, mean=MEAN, std=STD)
    vae = M.Vae(16, mean=MEAN, std=STD)
    vae.init_random(7)
    tokens = np.random.default_rng(88).standard_normal((64, 64)).astype(np.float32)
    want_p, got_p = {}, {}
    ref.decode(tokens, 8, 8, want_p)
    vae.set_probe(got_p)
    vae.decode(tokens, 8, 8)
    for k in (("vae_conv_in", -1), ("vae_mid", -1)):
        within(got_p[k], want_p[k], 64)


def test_vae_checkpoint_with_causal_3d_convs(gpu, tmp_path):
    base, h, w = 16, 2, 2
    ref = R.Vae(base, seed=9, mean=MEAN, std=STD)
    rng = np.random.default_rng(0)
    ts = {}
    for name, a in ref.tensors():
        if a.ndim == 4 and "resample" not in name and "attentions" not in name:
            # CausalConv3d: [out][in][k][k][k] (time taps = k); a single frame sees only the last time tap. The
            # upsamplers' resample convs and the attention's 1x1 convs are 2-D in the checkpoint.
            kt = a.shape[-1]
            t = rng.standard_normal((a.shape[0], a.shape[1], kt) + a.shape[2:]).astype(np.float32)
            t[:, :, kt - 1] = a
            ts[name] = torch.from_numpy(t).to(torch.bfloat16)
        elif name.endswith(".gamma"):
            ts[name] = torch.from_numpy(a.reshape(-1, 1, 1, 1).copy())  # RMS_norm's broadcastable gamma
        else:
            ts[name] = torch.from_numpy(a.copy())
    save_file(ts, str(tmp_path / "vae.safetensors"))
    v1 = M.Vae(base, mean=MEAN, std=STD)
    assert v1.load_safetensors(tmp_path / "vae.safetensors") == len(ts)
    v2 = M.Vae(base, mean=MEAN, std=STD)
    v2.init_random(9)
    tokens = rng.standard_normal((h * w, 64)).astype(np.float32)
    assert np.array_equal(v1.decode(tokens, h, w), v2.decode(tokens, h, w))
    del ts["decoder.conv_out.bias"]
    save_file(ts, str(tmp_path / "bad.safetensors"))
    with pytest.raises(M.MkError, match="no tensor decoder.conv_out.bias"):
        M.Vae(base, mean=MEAN, std=STD).load_safetensors(tmp_path / "bad.safetensors")


def test_vae_argument_errors(gpu):
    vae = M.Vae(16, mean=MEAN, std=STD)
    with pytest.raises(M.MkError, match="latents must be"):
        vae.decode(np.zeros((4, 60), np.float32), 2, 2)
    with pytest.raises(M.MkError, match="256 tokens a side"):
        vae.decode(np.zeros((257, 64), np.float32), 257, 1)
    with pytest.raises(M.MkError, match="wrong shape"):
        vae.load("decoder.conv_in.weight", np.zeros((64, 16, 3, 2), np.float32))
    with pytest.raises(M.MkError, match="no tensor named"):
        vae.load("decoder.nope.weight", np.zeros(4, np.float32))
    with pytest.raises(M.MkError, match="mean and std need 16"):
        M.Vae(16, mean=MEAN[:3], std=STD)


def test_vae_full_size_properties(gpu):
    # the 1024x1024 decode (Qwen-Image's base 96, 64 x 64 tokens): with a constant latent every pixel farther from the
    # image border than the decoder's reach (about 150 output pixels: 12 convs at 1/8 scale, 7 at 1/4, 7 at 1/2, 7 at
    # full) sees identical inputs, and the mid block's attention gives identical queries identical outputs, so the
    # centre must be uniform bit for bit; random tokens decode to finite values deterministically.
    vae = M.Vae(96, mean=MEAN, std=STD)
    vae.init_random(1)
    # one value a channel for all four pixels of each token's 2x2 patch (value (c * 2 + py) * 2 + px): a constant
    # latent image
    tok = np.tile(np.repeat(np.random.default_rng(2).standard_normal(16).astype(np.float32), 4), (64 * 64, 1))
    img = vae.decode(tok, 64, 64)
    assert img.shape == (1024, 1024, 4) and np.all(img[..., 3] == 1)
    c = img[200:824, 200:824, :3]
    assert np.array_equal(c, np.broadcast_to(img[512, 512, :3], c.shape)), np.abs(c - img[512, 512, :3]).max()
    assert not np.array_equal(img[0, 0, :3], img[512, 512, :3])  # the border does differ
    rnd = np.random.default_rng(3).standard_normal((64 * 64, 64)).astype(np.float32)
    a, b = vae.decode(rnd, 64, 64), vae.decode(rnd, 64, 64)
    assert np.isfinite(a).all() and np.array_equal(a, b) and np.abs(a[..., :3]).max() <= 1
