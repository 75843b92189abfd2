"""The oracle's graphs pinned against independent CPU implementations built from PyTorch library routines
(F.linear, F.layer_norm, F.rms_norm, F.group_norm, F.scaled_dot_product_attention, F.gelu) in float64, written in the
module / chunk idiom of the public model code, with bf16 rounding at the same operand points. A wiring mistake in the
C++ oracle (a swapped shift / scale, the wrong stream's weights, a transposed operand, a dropped residual) fails these.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import mkref as R

torch.set_grad_enabled(False)


def bf(x):
    return x.to(torch.bfloat16).to(torch.float64)


def hf(x):
    """IEEE half: the heads' precision in the reference's own graphs (Qwen-Image 2.1, SDXL)."""
    return x.to(torch.float16).to(torch.float64)


class Weights:
    def __init__(self, model):
        self.t, self.kind = {}, {}
        for n, a, k in model.tensors():
            self.t[n], self.kind[n] = torch.from_numpy(a).double(), k

    def w(self, name):
        W = self.t[name + ".weight"]
        s = self.t.get(name + ".weight.scale")
        return W * s[:, None] if s is not None else W

    def linear(self, name, x, bias=True):
        b = self.t.get(name + ".bias") if bias else None
        if self.t.get(name + ".weight.scale") is not None:  # fp8: scale after the product, as stored
            y = F.linear(bf(x), self.t[name + ".weight"]) * self.t[name + ".weight.scale"]
            return y + b if b is not None else y
        # a half matrix (kind 3) takes its input in half, the others in bf16
        return F.linear(hf(x) if self.kind[name + ".weight"] == 3 else bf(x), self.w(name), b)

    def __getitem__(self, k):
        return self.t[k]


def timestep_embedding(sigma, dim=256):
    half = dim // 2
    freqs = torch.exp(-np.log(10000.0) * torch.arange(half, dtype=torch.float64) / half)
    arg = 1000.0 * sigma * freqs
    return torch.cat([torch.cos(arg), torch.sin(arg)])


def rope_rotate(x, cs):
    """x [H][T][128], cs [T][64][2]: interleaved pairs rotated (complex product)."""
    z = torch.view_as_complex(x.reshape(*x.shape[:-1], 64, 2).contiguous())
    r = torch.view_as_complex(cs.contiguous())
    return torch.view_as_real(z * r).reshape(x.shape)


def dual_reference(model, dims, prompt, latents, h, w, sigma):
    W = Weights(model)
    D, H = dims["dim"], dims["heads"]
    temb = W.linear("time_text_embed.timestep_embedder.linear_2",
                    F.silu(W.linear("time_text_embed.timestep_embedder.linear_1",
                                    timestep_embedding(sigma).unsqueeze(0))))
    S, N = prompt.shape[1], h * w
    cs = torch.from_numpy(R.rope_table(S, h, w)).double()
    outs = []
    for b in range(prompt.shape[0]):
        txt = W.linear("txt_in", F.rms_norm(torch.from_numpy(prompt[b]).double(), (dims["text_dim"],),
                                            W["txt_norm.weight"], eps=1e-6))
        img = W.linear("img_in", torch.from_numpy(latents[b]).double())
        for i in range(dims["blocks"]):
            p = f"transformer_blocks.{i}."
            img_mod1, img_mod2 = W.linear(p + "img_mod.1", F.silu(temb))[0].chunk(2)
            txt_mod1, txt_mod2 = W.linear(p + "txt_mod.1", F.silu(temb))[0].chunk(2)

            def modulate(x, m):
                shift, scale, gate = m.chunk(3)
                return F.layer_norm(x, (D,), eps=1e-6) * (1 + scale) + shift, gate

            def heads(x, norm):
                y = x.reshape(x.shape[0], H, 128).transpose(0, 1)
                return F.rms_norm(y, (128,), W[norm], eps=1e-6) if norm else y

            xi, gi = modulate(img, img_mod1)
            xt, gt = modulate(txt, txt_mod1)
            q = torch.cat([heads(W.linear(p + "attn.add_q_proj", xt), p + "attn.norm_added_q.weight"),
                           heads(W.linear(p + "attn.to_q", xi), p + "attn.norm_q.weight")], 1)
            k = torch.cat([heads(W.linear(p + "attn.add_k_proj", xt), p + "attn.norm_added_k.weight"),
                           heads(W.linear(p + "attn.to_k", xi), p + "attn.norm_k.weight")], 1)
            v = torch.cat([heads(W.linear(p + "attn.add_v_proj", xt), None),
                           heads(W.linear(p + "attn.to_v", xi), None)], 1)
            q, k = rope_rotate(q, cs), rope_rotate(k, cs)
            o = F.scaled_dot_product_attention(bf(q), bf(k), bf(v)).transpose(0, 1).reshape(S + N, D)
            txt = txt + gt * W.linear(p + "attn.to_add_out", o[:S])
            img = img + gi * W.linear(p + "attn.to_out.0", o[S:])
            xi, gi = modulate(img, img_mod2)
            xt, gt = modulate(txt, txt_mod2)
            img = img + gi * W.linear(p + "img_mlp.net.2",
                                      F.gelu(W.linear(p + "img_mlp.net.0.proj", xi), approximate="tanh"))
            txt = txt + gt * W.linear(p + "txt_mlp.net.2",
                                      F.gelu(W.linear(p + "txt_mlp.net.0.proj", xt), approximate="tanh"))
        scale, shift = W.linear("norm_out.linear", F.silu(temb))[0].chunk(2)
        outs.append(W.linear("proj_out", F.layer_norm(img, (D,), eps=1e-6) * (1 + scale) + shift))
    return torch.stack(outs).numpy()


def q21_reference(model, dims, prompt, latents, h, w, sigma):
    W = Weights(model)
    D, H, Fd = dims["dim"], dims["heads"], dims["ffn"]
    S, N = prompt.shape[0], h * w
    T = S + N
    tp = torch.stack([timestep_embedding(sigma), timestep_embedding(0.0)])
    temb = W.linear("time_text_embed.timestep_embedder.linear_2",
                    F.silu(W.linear("time_text_embed.timestep_embedder.linear_1", tp, False)), False)
    mod = W.linear("modulation.1", F.silu(temb), False)        # [2][4D]: scale1, gate1, scale2, gate2
    omod = W.linear("norm_out.linear", F.silu(temb), False)    # [2][D]
    rowmod = lambda m: torch.cat([m[1:].expand(S, -1), m[:1].expand(N, -1)])  # noqa: E731  text rows take t = 0
    mods = rowmod(mod)
    sc1, g1, sc2, g2 = mods.chunk(4, dim=1)
    tn = F.rms_norm(torch.from_numpy(prompt).double(), (dims["text_dim"],), W["txt_in.text_norm.weight"] + 1, eps=1e-6)
    txt = W.linear("txt_in.out_layer", F.gelu(W.linear("txt_in.in_layer", tn, False), approximate="tanh"), False)
    x = torch.cat([txt, W.linear("img_in", torch.from_numpy(latents).double(), False)])
    cs = torch.from_numpy(R.rope_table(S, h, w)).double()
    mask = torch.ones(T, T, dtype=torch.bool)
    mask[:S, :] = torch.ones(S, T, dtype=torch.bool).tril()
    for i in range(dims["blocks"]):
        p = f"transformer_blocks.{i}."
        xn = F.layer_norm(x, (D,), eps=1e-6) * (1 + sc1)
        hs = lambda y: y.reshape(T, H, 128).transpose(0, 1)  # noqa: E731
        q = rope_rotate(F.rms_norm(hs(W.linear(p + "attn.to_q", xn, False)), (128,), W[p + "attn.norm_q.weight"],
                                   eps=1e-6), cs)
        k = rope_rotate(F.rms_norm(hs(W.linear(p + "attn.to_k", xn, False)), (128,), W[p + "attn.norm_k.weight"],
                                   eps=1e-6), cs)
        v = hs(W.linear(p + "attn.to_v", xn, False))
        o = F.scaled_dot_product_attention(hf(q), hf(k), hf(v), attn_mask=mask).transpose(0, 1).reshape(T, D)
        x = x + torch.tanh(g1) * W.linear(p + "attn.to_out.0", o, False)
        xn = F.layer_norm(x, (D,), eps=1e-6) * (1 + sc2)
        m = F.silu(W.linear(p + "img_mlp.gate_layer", xn, False)) * W.linear(p + "img_mlp.proj", xn, False)
        x = x + torch.tanh(g2) * W.linear(p + "img_mlp.out", m, False)
    xn = F.layer_norm(x, (D,), eps=1e-6) * (1 + rowmod(omod))
    return W.linear("proj_out", xn[S:], False).numpy()


def sdxl_reference(model, dims, x, ctx):
    W = Weights(model)
    c, Fd = dims["dim"], dims["ffn"]
    H = c // 64
    xt = torch.from_numpy(x).double()
    n = xt.shape[0]
    hs = W.linear("proj_in", F.group_norm(xt.t().unsqueeze(0), 32, W["norm.weight"], W["norm.bias"], eps=1e-6)[0].t())
    ctx = torch.from_numpy(ctx).double()
    heads = lambda y: y.reshape(y.shape[0], H, 64).transpose(0, 1)  # noqa: E731
    for i in range(dims["blocks"]):
        p = f"transformer_blocks.{i}."
        ln = lambda j: F.layer_norm(hs, (c,), W[p + f"norm{j}.weight"], W[p + f"norm{j}.bias"], eps=1e-5)  # noqa
        h1 = ln(1)
        q, k, v = (heads(W.linear(p + f"attn1.to_{s}", h1, False)) for s in "qkv")
        o = F.scaled_dot_product_attention(hf(q), hf(k), hf(v)).transpose(0, 1).reshape(n, c)
        hs = hs + W.linear(p + "attn1.to_out.0", o)
        h2 = ln(2)
        q = heads(W.linear(p + "attn2.to_q", h2, False))
        k, v = heads(W.linear(p + "attn2.to_k", ctx, False)), heads(W.linear(p + "attn2.to_v", ctx, False))
        o = F.scaled_dot_product_attention(hf(q), hf(k), hf(v)).transpose(0, 1).reshape(n, c)
        hs = hs + W.linear(p + "attn2.to_out.0", o)
        hh, g = W.linear(p + "ff.net.0.proj", ln(3)).chunk(2, dim=1)
        hs = hs + W.linear(p + "ff.net.2", hh * F.gelu(g))
    return (W.linear("proj_out", hs) + xt).numpy()


# Weights of N(0, 0.1) make every branch matter (at 0.02 the skip path dominates and a swapped shift / scale moves
# the output by 2e-3); the correct graph then agrees to ~2e-3 (bf16 rounding flips between fp32 and fp64 sums), a
# swapped shift / scale is off by ~1, a reversed rotation by ~0.1, the text stream's norm weights on the image by 6e-3.
WSTD = 0.1


def agree(got, want, tol_rel=4e-3):
    d = R.diff(got, want, want.shape[-1])
    assert d["cos"] > 0.9999 and d["rel"] < tol_rel, d


DUAL = dict(kind=R.DUAL, blocks=2, dim=256, heads=2, head_dim=128, ffn=512, text_dim=192)


@pytest.mark.parametrize("fp8", [False, True])
def test_dual_step_matches_torch(fp8):
    m = R.Model(**DUAL, fp8=fp8, seed=7, wstd=WSTD)
    rng = np.random.default_rng(1)
    h, w, S = 4, 6, 9
    prompt = rng.standard_normal((2, S, 192)).astype(np.float32)
    lat = rng.standard_normal((2, h * w, 64)).astype(np.float32)
    got = m.dual_step(prompt, lat, h, w, 0.6)
    want = dual_reference(m, DUAL, prompt, lat, h, w, 0.6)
    agree(got, want)


def test_dual_step_probes():
    # the probes the GPU comparison uses: stage names, sizes and the block output's link to the step output
    m = R.Model(**DUAL, seed=3, wstd=WSTD)
    rng = np.random.default_rng(2)
    h, w, S = 2, 3, 4
    prompt = rng.standard_normal((2, S, 192)).astype(np.float32)
    lat = rng.standard_normal((2, h * w, 64)).astype(np.float32)
    probes = {}
    out = m.dual_step(prompt, lat, h, w, 0.3, probes)
    assert probes[("modulation", -1)].size == 2 * 2 * 6 * 256
    assert probes[("img_in", 1)].size == h * w * 256 and probes[("txt_in", 0)].size == S * 256
    assert {k for k in probes if k[0] == "block"} == {("block", i) for i in range(4)}
    # the output is proj_out of norm_out: linear in the probe
    W = m.get("proj_out.weight")
    want = R.gemm(probes[("norm_out", 1)].reshape(h * w, 256), W, m.get("proj_out.bias"))
    assert np.allclose(out[1], want, atol=1e-6)


def test_q21_step_matches_torch():
    dims = dict(kind=R.Q21, blocks=2, dim=256, heads=2, head_dim=128, ffn=384, text_dim=256)
    m = R.Model(**dims, seed=11, wstd=0.05)
    rng = np.random.default_rng(4)
    h, w, S = 4, 4, 7
    prompt = rng.standard_normal((S, 256)).astype(np.float32)
    lat = rng.standard_normal((h * w, 64)).astype(np.float32)
    # at N(0, 0.05) the graph agrees to 6.1e-4; without the tanh gate it is off by 1.7e-3, without the causal text
    # prefix 7e-3, with the text rows on the timestep's modulation 1.4e-2, with bf16 heads instead of half 1.1e-3
    agree(m.q21_step(prompt, lat, h, w, 0.8), q21_reference(m, dims, prompt, lat, h, w, 0.8), 8e-4)


@pytest.mark.parametrize("f16", [False, True])
def test_sdxl_trans_matches_torch(f16):
    # agrees to 2.3e-3 with half heads; bf16 heads would be off by 5.8e-3. With half matrices: 7.8e-4, and inputs
    # to them rounded to bf16 instead of half would be off by 4.6e-3
    dims = dict(kind=R.SDXL, blocks=2, dim=128, heads=2, head_dim=64, ffn=256, text_dim=192)
    m = R.Model(**dims, seed=5, wstd=WSTD, f16=f16)
    rng = np.random.default_rng(6)
    x = rng.standard_normal((40, 128)).astype(np.float32)
    ctx = rng.standard_normal((11, 192)).astype(np.float32)
    agree(m.sdxl_trans(x, ctx), sdxl_reference(m, dims, x, ctx), 1.5e-3 if f16 else 4e-3)


def test_sdxl_half_matrices():
    # with f16 the matrices Engine::matrix keeps (proj_in / proj_out, to_out, attn2.to_q, ff) hold half values of the
    # same N(0, wstd) draws, q|k|v and the context's k|v stay bf16; a half matrix's GEMM rounds its input to half
    dims = dict(kind=R.SDXL, blocks=1, dim=128, heads=2, head_dim=64, ffn=256, text_dim=192)
    a, b = R.Model(**dims, seed=9, f16=False), R.Model(**dims, seed=9, f16=True)
    half = {"proj_in.weight", "proj_out.weight", "transformer_blocks.0.attn1.to_out.0.weight",
            "transformer_blocks.0.attn2.to_q.weight", "transformer_blocks.0.attn2.to_out.0.weight",
            "transformer_blocks.0.ff.net.0.proj.weight", "transformer_blocks.0.ff.net.2.weight"}
    kinds = {n: k for n, _, k in b.tensors()}
    assert {n for n, k in kinds.items() if k == 3} == half
    for (n, wa, ka), (_, wb, kb) in zip(a.tensors(), b.tensors()):
        if n in half:
            assert ka == 1 and kb == 3
            assert np.array_equal(wb, wb.astype(np.float16).astype(np.float32))  # half-exact
            assert not np.array_equal(wa, wb)  # not the bf16 values
            assert np.abs(wa - wb).max() <= 2 ** -8 * np.abs(wb).max()  # the same draws
        else:
            assert np.array_equal(wa, wb)


# ---- VAE decoder (src/image/engine.cpp:862-954), written in the idiom of the public Wan-2.1 decoder: conv2d with
# padding 1, RMS norm over channels, nearest interpolation, one-head attention; at the reference's precision points:
# half weights and half inputs for every convolution (docs/performance.md:13), half queries and probabilities against
# fp32 keys and values in the attention (engine.cpp:764-773) ----

def vae_reference(vae, tokens, h, w, rnd=hf):
    t = {n: torch.from_numpy(a).double() for n, a in vae.tensors()}
    z = vae.z

    def conv(x, name):  # x [1][c][H][W]; the input and the weights rounded to half
        W = t[name + ".weight"]
        return F.conv2d(rnd(x), rnd(W), t[name + ".bias"], padding=W.shape[-1] // 2)

    def rms(x, g, silu=True):
        c = x.shape[1]
        y = x / torch.sqrt((x * x).sum(1, keepdim=True) + 1e-24) * (c ** 0.5) * g[None, :, None, None]
        return rnd(F.silu(y) if silu else y)

    def res(x, p):
        hh = conv(rms(x, t[p + ".norm1.gamma"]), p + ".conv1")
        hh = conv(rms(hh, t[p + ".norm2.gamma"]), p + ".conv2")
        return hh + (conv(x, p + ".conv_shortcut") if p + ".conv_shortcut.weight" in t else x)

    def attn(x):
        a = "decoder.mid_block.attentions.0."
        _, c, H, W_ = x.shape
        xn = rms(x, t[a + "norm.gamma"], silu=False)
        Wq = rnd(t[a + "to_qkv.weight"][:, :, 0, 0])
        bq = t[a + "to_qkv.bias"]
        seq = xn.flatten(2).transpose(1, 2)[0]  # [n][c]
        q = hf(F.linear(seq, Wq[:c], bq[:c]))  # half queries
        k = F.linear(seq, Wq[c:2 * c], bq[c:2 * c])  # fp32 keys and values
        v = F.linear(seq, Wq[2 * c:], bq[2 * c:])
        p = hf(torch.softmax((q @ k.T).float().double() / c ** 0.5, dim=-1))  # scores fp32, P half
        o = (p @ v).T.reshape(1, c, H, W_)
        return x + conv(o, a + "proj")

    tok = torch.from_numpy(np.asarray(tokens, np.float64)).reshape(h, w, z, 2, 2)
    lat = tok.permute(2, 0, 3, 1, 4).reshape(1, z, 2 * h, 2 * w)  # channel c of pixel (2y + py, 2x + px)
    lat = lat * torch.from_numpy(vae.std).double()[None, :, None, None] + \
        torch.from_numpy(vae.mean).double()[None, :, None, None]
    x = conv(lat, "post_quant_conv")  # a 1x1 convolution like the others
    x = conv(x, "decoder.conv_in")
    x = res(x, "decoder.mid_block.resnets.0")
    x = attn(x)
    x = res(x, "decoder.mid_block.resnets.1")
    for i in range(4):
        p = f"decoder.up_blocks.{i}"
        for j in range(3):
            x = res(x, f"{p}.resnets.{j}")
        if i < 3:
            x = conv(F.interpolate(x, scale_factor=2, mode="nearest"), f"{p}.upsamplers.0.resample.1")
    x = conv(rms(x, t["decoder.norm_out.gamma"]), "decoder.conv_out")
    rgb = x[0].permute(1, 2, 0).clamp(-1, 1)
    return torch.cat([rgb, torch.ones_like(rgb[..., :1])], -1).numpy()


@pytest.mark.parametrize("h, w", [(2, 2), (2, 3)])
def test_vae_decode_matches_torch(h, w):
    rng = np.random.default_rng(7)
    vae = R.Vae(16, seed=3, mean=rng.standard_normal(16) * 0.1, std=1 + rng.random(16))
    tokens = rng.standard_normal((h * w, 64)).astype(np.float32)
    got = vae.decode(tokens, h, w)
    want = vae_reference(vae, tokens, h, w)
    assert got.shape == (16 * h, 16 * w, 4) and np.all(got[..., 3] == 1)
    agree(got[..., :3], want[..., :3], tol_rel=1.5e-3)
    # the precision points matter at that tolerance: the same graph with bf16 convolution operands is 4x outside it
    d = R.diff(got[..., :3], vae_reference(vae, tokens, h, w, rnd=bf)[..., :3], 3)
    assert d["rel"] > 4e-3, d
