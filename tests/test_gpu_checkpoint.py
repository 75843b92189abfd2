"""Checkpoint loading and LoRA merging on the GPU, through the C ABI: mk_engine_load_safetensors (the reference's
load_transformer / upload / upload_rows, src/image/qwen_image.cpp:79-111) and mk_engine_add_lora (add_lora with merging,
targets as QwenImage::lora_target gives them, src/image/qwen_image.cpp:295-331).

Loading is bit-exact: a checkpoint written from the oracle's weights steps exactly as the same weights uploaded by name
do (and within the step tolerance of the oracle), and every dtype conversion equals the one torch makes on the host.
The LoRA merge is held to the textbook W + scale (alpha / rank) B A in float64, rounded once to the stored type: at
most one bf16 unit in the last place apart (the device sums in fp32), and for fp8 rows the scale max / 448 of the
merged row and each code within half an e4m3 step of the merged value. Everything the LoRA does not name stays
bit-identical."""
import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import mkimage as M
import mkref as R
from test_gpu_engine import H_, S_, TINY, W_, inputs, make_pair, within

pytestmark = pytest.mark.gpu

Q21 = dict(blocks=2, dim=512, heads=4, head_dim=128, ffn=1536, text_dim=512)
SDXL = dict(blocks=1, dim=640, heads=10, head_dim=64, ffn=2560, text_dim=2048)


def state(e):
    """Every weight of an engine as stored, with fp8 scales under name + '.scale'."""
    out = {}
    for name, dt, r, c in e.tensors():
        out[name] = (e.fetch(name, dt, r, c), dt)
        if dt == M.FP8:
            out[name + ".scale"] = (e.fetch(name + ".scale", M.F32, r, 1), M.F32)
    return out


def as_torch(a, dt):
    if dt == M.BF16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    if dt == M.FP8:
        return torch.from_numpy(a.copy()).view(torch.float8_e4m3fn)
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))


def oracle_checkpoint(m):
    """The oracle's weights as a checkpoint: bf16 matrices, fp8 matrices with their per-row scales, fp32 vectors."""
    out = {}
    for name, a, kind in m.tensors():
        if kind == 0:
            out[name] = torch.from_numpy(a)
        elif kind == 1:
            out[name] = torch.from_numpy(a).to(torch.bfloat16)  # exact: the oracle's matrices are bf16 values
        else:
            out[name] = torch.from_numpy(a).to(torch.float8_e4m3fn)  # exact: e4m3 values
    return out


def same_state(a, b, skip=()):
    assert a.keys() == b.keys()
    for k in a:
        if k not in skip:
            assert np.array_equal(a[k][0], b[k][0]), k


def test_oracle_checkpoint_steps_like_the_oracle(gpu, tmp_path):
    m, e_up = make_pair(M.FAMILY_DUAL, seed=5)
    path = tmp_path / "dual.safetensors"
    save_file(oracle_checkpoint(m), str(path))
    e = M.Engine(M.FAMILY_DUAL, **TINY)
    assert e.load_safetensors(path) == len(e.tensors())
    prompt, lat = inputs(4)
    for eng in (e, e_up):
        eng.begin(prompt[0], H_, W_, 0)
    got = e.step(lat[0], 0.4, 0)
    assert np.array_equal(got, e_up.step(lat[0], 0.4, 0))
    within(got, m.dual_step(prompt[:1], lat[:1], H_, W_, 0.4)[0], 64)


def test_fp8_checkpoint_with_scales(gpu, tmp_path):
    m, e_up = make_pair(M.FAMILY_DUAL, fp8=True, seed=6)
    path = tmp_path / "dual_fp8.safetensors"
    save_file(oracle_checkpoint(m), str(path))
    e = M.Engine(M.FAMILY_DUAL, **TINY, weight_dtype=M.FP8)
    e.load_safetensors(path)
    same_state(state(e), state(e_up))


def test_bf16_checkpoint_into_fp8_engine_quantises_like_init(gpu, tmp_path):
    # init_random of an fp8 engine quantises the bf16 draws per row; loading those draws from a file must agree
    eb = M.Engine(M.FAMILY_DUAL, **TINY)
    eb.init_random(7)
    save_file({k: as_torch(a, dt) for k, (a, dt) in state(eb).items()}, str(tmp_path / "b.safetensors"))
    ef = M.Engine(M.FAMILY_DUAL, **TINY, weight_dtype=M.FP8)
    ef.load_safetensors(tmp_path / "b.safetensors")
    er = M.Engine(M.FAMILY_DUAL, **TINY, weight_dtype=M.FP8)
    er.init_random(7)
    same_state(state(ef), state(er))


@pytest.mark.parametrize("family, dims", [(M.FAMILY_Q21, Q21), (M.FAMILY_SDXL, SDXL)])
def test_sharded_f32_checkpoint_with_prefix_round_trips(gpu, tmp_path, family, dims):
    e = M.Engine(family, **dims)
    e.init_random(8)
    st = state(e)
    names = sorted(st)
    # fp32 on file (bf16 values, so the conversion back is exact), a single-file checkpoint prefix, two shards
    ts = {"model.diffusion_model." + k: torch.from_numpy(
        M.bf16_to_f32(a) if dt == M.BF16 else a.astype(np.float32)) for k, (a, dt) in st.items()}
    half = len(names) // 2
    keys = ["model.diffusion_model." + k for k in names]
    save_file({k: ts[k] for k in keys[:half]}, str(tmp_path / "m-00001.safetensors"))
    save_file({k: ts[k] for k in keys[half:]}, str(tmp_path / "m-00002.safetensors"))
    e2 = M.Engine(family, **dims)
    assert e2.load_safetensors(tmp_path) == len(names)
    same_state(state(e2), st)


def test_sdxl_transformer_at_its_unet_path(gpu, tmp_path):
    # a UNet checkpoint holding two spatial transformers (sdxl.cpp:264-306 reads each under kUnet + its path): the
    # engine takes the one its prefix names, and the other's (deeper) blocks do not count against the engine's
    e_a = M.Engine(M.FAMILY_SDXL, **SDXL)
    e_a.init_random(21)
    e_b = M.Engine(M.FAMILY_SDXL, **SDXL)
    e_b.init_random(22)
    ts = {}
    for path, e in (("input_blocks.4.1.", e_a), ("output_blocks.2.1.", e_b)):
        for k, (a, dt) in state(e).items():
            ts["model.diffusion_model." + path + k] = torch.from_numpy(
                M.bf16_to_f32(a) if dt == M.BF16 else a.astype(np.float32))
    # a deeper transformer elsewhere in the UNet: more blocks than the engine holds
    ts["model.diffusion_model.middle_block.1.transformer_blocks.9.norm1.weight"] = torch.zeros(8)
    save_file(ts, str(tmp_path / "unet.safetensors"))
    e = M.Engine(M.FAMILY_SDXL, **SDXL)
    n = e.load_safetensors(tmp_path / "unet.safetensors", prefix="model.diffusion_model.output_blocks.2.1.")
    assert n == len(state(e_b))
    same_state(state(e), state(e_b))
    # without the prefix the names are not found
    with pytest.raises(M.MkError, match="no tensor"):
        M.Engine(M.FAMILY_SDXL, **SDXL).load_safetensors(tmp_path / "unet.safetensors")


def test_f16_checkpoint_rounds_like_torch(gpu, tmp_path):
    e = M.Engine(M.FAMILY_DUAL, **TINY)
    e.init_random(9)
    st = state(e)
    ts = {}
    for k, (a, dt) in st.items():
        t = as_torch(a, dt).float() * 3.7  # off the bf16 grid once in f16
        ts[k] = t.to(torch.float16)
    save_file(ts, str(tmp_path / "h.safetensors"))
    e2 = M.Engine(M.FAMILY_DUAL, **TINY)
    e2.load_safetensors(tmp_path / "h.safetensors")
    for k, (a, dt) in state(e2).items():
        want = ts[k].to(torch.bfloat16 if dt == M.BF16 else torch.float32)
        got = as_torch(a, dt)
        assert torch.equal(got.view(torch.int16) if dt == M.BF16 else got,
                           want.view(torch.int16) if dt == M.BF16 else want), k


def test_sdxl_f16_matrices_kept_half(gpu, tmp_path):
    # an SDXL engine with F16 weights keeps the matrices Engine::matrix keeps F16 (proj_in / proj_out, to_out,
    # attn2.to_q, ff: engine.cpp:292-302, sdxl.cpp:267-306) as half, q|k|v and the context's k|v as bf16: its random
    # init is the oracle's half model bit for bit, an F16 checkpoint of it loads back bit for bit, and a bf16 engine
    # reading the same file rounds the half matrices to bf16 as torch does
    m = R.Model(R.SDXL, **SDXL, f16=True, seed=13)
    e = M.Engine(M.FAMILY_SDXL, **SDXL, weight_dtype=M.F16)
    e.init_random(13)
    st = state(e)
    kinds = {}
    for name, a, kind in m.tensors():
        got, dt = st[name]
        kinds[name] = kind
        if kind == 3:
            assert dt == M.F16 and np.array_equal(got, M.f16_bits(a)), name
        elif kind == 1:
            assert dt == M.BF16 and np.array_equal(got, M.bf16_bits(a)), name
        else:
            assert dt == M.F32 and np.array_equal(got, a), name
    assert sum(k == 3 for k in kinds.values()) == 7 and sum(k == 1 for k in kinds.values()) == 5  # q, k, v; k2, v2
    ts = {k: torch.from_numpy(a.view(np.float16).copy()) if dt == M.F16 else as_torch(a, dt)
          for k, (a, dt) in st.items()}
    save_file(ts, str(tmp_path / "sdxl_f16.safetensors"))
    e2 = M.Engine(M.FAMILY_SDXL, **SDXL, weight_dtype=M.F16)
    assert e2.load_safetensors(tmp_path / "sdxl_f16.safetensors") == len(st)
    same_state(state(e2), st)
    e3 = M.Engine(M.FAMILY_SDXL, **SDXL)
    e3.load_safetensors(tmp_path / "sdxl_f16.safetensors")
    for k, (a, dt) in state(e3).items():
        if kinds[k] == 3:
            assert dt == M.BF16
            assert torch.equal(as_torch(a, dt).view(torch.int16), ts[k].to(torch.bfloat16).view(torch.int16)), k
    # a LoRA merges into a half matrix within one half unit in the last place of the float64 merge
    rng = np.random.default_rng(5)
    D, Fd = SDXL["dim"], SDXL["ffn"]
    lw = {}
    a1, b1 = lora_pair(rng, D, Fd, 8)
    lw["transformer_blocks.0.ff.net.2.lora_A.weight"], lw["transformer_blocks.0.ff.net.2.lora_B.weight"] = a1, b1
    save_file(lw, str(tmp_path / "lora.safetensors"))
    before = st["transformer_blocks.0.ff.net.2.weight"][0]
    assert e.add_lora(tmp_path / "lora.safetensors", 0.7) == (1, 0)
    after, dt = state(e)["transformer_blocks.0.ff.net.2.weight"]
    assert dt == M.F16
    want = M.f16_to_f32(before).astype(np.float64) + 0.7 * (b1.double().numpy() @ a1.double().numpy())
    got = M.f16_to_f32(after).astype(np.float64)
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -14))) - 10)
    assert (np.abs(got - want) <= ulp * 1.0001 + 1e-8).all()
    assert np.mean(after == M.f16_bits(want.astype(np.float32))) >= 0.99


def test_checkpoint_errors(gpu, tmp_path):
    e = M.Engine(M.FAMILY_DUAL, **TINY)
    e.init_random(1)
    base = {k: as_torch(a, dt) for k, (a, dt) in state(e).items()}

    def attempt(ts, match, fp8=False):
        p = tmp_path / "bad.safetensors"
        save_file(ts, str(p))
        e2 = M.Engine(M.FAMILY_DUAL, **TINY, weight_dtype=M.FP8 if fp8 else M.BF16)
        with pytest.raises(M.MkError, match=match):
            e2.load_safetensors(p)

    missing = dict(base)
    del missing["transformer_blocks.1.attn.add_k_proj.weight"]
    attempt(missing, "no tensor transformer_blocks.1.attn.add_k_proj.weight")
    wrong = dict(base)
    wrong["proj_out.weight"] = wrong["proj_out.weight"].t().contiguous()
    attempt(wrong, "proj_out.weight has dims")
    extra = dict(base)
    extra["transformer_blocks.2.attn.to_q.weight"] = base["transformer_blocks.1.attn.to_q.weight"].clone()
    attempt(extra, "engine has 2 blocks")
    f8 = dict(base)
    f8["transformer_blocks.0.attn.to_q.weight"] = base["transformer_blocks.0.attn.to_q.weight"].to(torch.float8_e4m3fn)
    attempt(f8, "F8_E4M3 but the engine stores it as BF16")
    attempt(f8, "needs its per-row scale", fp8=True)
    ints = dict(base)
    ints["txt_norm.weight"] = torch.zeros(512, dtype=torch.int32)
    attempt(ints, "txt_norm.weight has dtype I32")


# ---- LoRA ----

def bf16_round(x):
    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def ulp_bf16(x):
    a = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def lora_pair(rng, rows, cols, r, dtype=torch.bfloat16):
    a = torch.from_numpy(rng.standard_normal((r, cols)).astype(np.float32) * 0.05).to(dtype)
    b = torch.from_numpy(rng.standard_normal((rows, r)).astype(np.float32) * 0.05).to(dtype)
    return a, b


def check_bf16_merge(before, after, a, b, factor):
    want = before.astype(np.float64) + factor * (b.double().numpy() @ a.double().numpy())
    got = M.bf16_to_f32(after).astype(np.float64)
    err = np.abs(got - want)
    assert (err <= ulp_bf16(want) * 1.0001 + 1e-8).all(), err.max()  # + the fp32 sum's error near zero
    exact = np.mean(after == bf16_round(want))
    assert exact >= 0.99, exact


def test_lora_merge_bf16_naming_styles(gpu, tmp_path):
    rng = np.random.default_rng(0)
    e = M.Engine(M.FAMILY_DUAL, **TINY)
    e.init_random(11)
    before = state(e)
    D, F = TINY["dim"], TINY["ffn"]
    ts = {}
    # PEFT / Diffusers names under a "transformer." prefix, with alpha
    a1, b1 = lora_pair(rng, D, D, 8)
    ts["transformer.transformer_blocks.0.attn.to_k.lora_A.weight"] = a1
    ts["transformer.transformer_blocks.0.attn.to_k.lora_B.weight"] = b1
    ts["transformer.transformer_blocks.0.attn.to_k.alpha"] = torch.tensor(4.0)
    # Kohya names ('_' for '.'), down / up, alpha, fp32 on file
    a2, b2 = lora_pair(rng, F, D, 16, torch.float32)
    ts["lora_unet_transformer_blocks_1_img_mlp_net_0_proj.lora_down.weight"] = a2
    ts["lora_unet_transformer_blocks_1_img_mlp_net_0_proj.lora_up.weight"] = b2
    ts["lora_unet_transformer_blocks_1_img_mlp_net_0_proj.alpha"] = torch.tensor([32.0])
    # a module inside the stacked modulation weights, no alpha
    a3, b3 = lora_pair(rng, 6 * D, D, 4)
    ts["transformer_blocks.0.img_mod.1.lora_A.weight"] = a3
    ts["transformer_blocks.0.img_mod.1.lora_B.weight"] = b3
    # skipped: a text-encoder module and a full-weight difference
    a4, b4 = lora_pair(rng, 64, 32, 4)
    ts["lora_te1_text_model_encoder_layers_0_mlp_fc1.lora_down.weight"] = a4
    ts["lora_te1_text_model_encoder_layers_0_mlp_fc1.lora_up.weight"] = b4
    ts["transformer_blocks.1.attn.to_out.0.diff"] = torch.zeros(D, D)
    save_file(ts, str(tmp_path / "lora.safetensors"))
    scale = 0.8
    assert e.add_lora(tmp_path / "lora.safetensors", scale) == (3, 2)
    after = state(e)
    targets = {"transformer_blocks.0.attn.to_k.weight": (a1, b1, scale * 4.0 / 8),
               "transformer_blocks.1.img_mlp.net.0.proj.weight": (a2, b2, scale * 32.0 / 16),
               "transformer_blocks.0.img_mod.1.weight": (a3, b3, scale)}
    for name, (a, b, f) in targets.items():
        check_bf16_merge(M.bf16_to_f32(before[name][0]), after[name][0], a.float(), b.float(), f)
    same_state(before, after, skip=targets)


def test_lora_merge_fp8_rescales_rows(gpu, tmp_path):
    rng = np.random.default_rng(1)
    e = M.Engine(M.FAMILY_DUAL, **TINY, weight_dtype=M.FP8)
    e.init_random(12)
    before = state(e)
    D = TINY["dim"]
    a, b = lora_pair(rng, D, D, 8)
    save_file({"transformer_blocks.1.attn.to_q.lora_A.weight": a, "transformer_blocks.1.attn.to_q.lora_B.weight": b},
              str(tmp_path / "l8.safetensors"))
    assert e.add_lora(tmp_path / "l8.safetensors", 1.5) == (1, 0)
    after = state(e)
    name = "transformer_blocks.1.attn.to_q.weight"
    table = R.e4m3_table().astype(np.float64)
    w0 = table[before[name][0]] * before[name + ".scale"][0][:, None].astype(np.float64)
    want = w0 + 1.5 * (b.double().numpy() @ a.double().numpy())
    want_scale = np.abs(want).max(1) / 448.0
    got_scale = after[name + ".scale"][0].astype(np.float64)
    assert np.allclose(got_scale, want_scale, rtol=1e-5, atol=0), np.abs(got_scale / want_scale - 1).max()
    got = table[after[name][0]] * got_scale[:, None]
    half_step = np.abs(want) * 2.0 ** -4 + 2.0 ** -10 * got_scale[:, None]
    assert (np.abs(got - want) <= half_step * 1.001).all()
    same_state(before, after, skip={name, name + ".scale"})


def test_lora_q21_gate_up_spans_both_halves(gpu, tmp_path):
    rng = np.random.default_rng(2)
    e = M.Engine(M.FAMILY_Q21, **Q21)
    e.init_random(13)
    before = state(e)
    D, F = Q21["dim"], Q21["ffn"]
    a, b = lora_pair(rng, 2 * F, D, 8)
    save_file({"transformer_blocks.0.img_mlp.gate_up.lora_A.weight": a,
               "transformer_blocks.0.img_mlp.gate_up.lora_B.weight": b}, str(tmp_path / "gu.safetensors"))
    assert e.add_lora(tmp_path / "gu.safetensors") == (1, 0)
    after = state(e)
    g, u = "transformer_blocks.0.img_mlp.gate_layer.weight", "transformer_blocks.0.img_mlp.proj.weight"
    w0 = np.concatenate([M.bf16_to_f32(before[g][0]), M.bf16_to_f32(before[u][0])])
    check_bf16_merge(w0, np.concatenate([after[g][0], after[u][0]]), a.float(), b.float(), 1.0)
    same_state(before, after, skip={g, u})


def test_lora_errors_leave_weights_alone(gpu, tmp_path):
    rng = np.random.default_rng(3)
    e = M.Engine(M.FAMILY_DUAL, **TINY)
    e.init_random(14)
    before = state(e)
    D = TINY["dim"]
    a, b = lora_pair(rng, D, D, 8)
    a_bad, _ = lora_pair(rng, D, D + 64, 8)
    p = tmp_path / "bad.safetensors"
    # a good module first, then one whose down matrix has the wrong width: nothing is merged
    save_file({"transformer_blocks.0.attn.to_q.lora_A.weight": a, "transformer_blocks.0.attn.to_q.lora_B.weight": b,
               "transformer_blocks.0.attn.to_v.lora_A.weight": a_bad,
               "transformer_blocks.0.attn.to_v.lora_B.weight": b.clone()}, str(p))
    with pytest.raises(M.MkError, match="do not fit"):
        e.add_lora(p)
    save_file({"transformer_blocks.0.attn.to_q.lora_A.weight": a}, str(p))
    with pytest.raises(M.MkError, match="only one of"):
        e.add_lora(p)
    # a DoRA magnitude beside the pair: refused rather than merged without it
    save_file({"transformer_blocks.0.attn.to_q.lora_A.weight": a, "transformer_blocks.0.attn.to_q.lora_B.weight": b,
               "transformer_blocks.0.attn.to_q.dora_scale": torch.ones(1, D)}, str(p))
    with pytest.raises(M.MkError, match="DoRA"):
        e.add_lora(p)
    same_state(before, state(e))


def test_lora_merge_fp8_exact_zeros(gpu, tmp_path):
    # Merged values that are exactly zero encode as zero: a row of zero codes whose LoRA rows are zero stays a zero
    # row (scale 1), and columns whose weights and LoRA columns are zero stay zero in every row.
    rng = np.random.default_rng(3)
    e = M.Engine(M.FAMILY_DUAL, **TINY, weight_dtype=M.FP8)
    e.init_random(14)
    D = TINY["dim"]
    name = "transformer_blocks.0.attn.to_k.weight"
    codes = e.fetch(name, M.FP8, D, D).copy()
    scale = e.fetch(name + ".scale", M.F32, D, 1).copy()
    codes[5] = 0
    codes[:, :16] = 0
    e.load(name, codes, M.FP8)
    e.load(name + ".scale", scale, M.F32)
    a, b = lora_pair(rng, D, D, 8)
    a[:, :16] = 0
    b[5] = 0
    save_file({"transformer_blocks.0.attn.to_k.lora_A.weight": a, "transformer_blocks.0.attn.to_k.lora_B.weight": b},
              str(tmp_path / "z.safetensors"))
    assert e.add_lora(tmp_path / "z.safetensors", 1.0) == (1, 0)
    got = e.fetch(name, M.FP8, D, D)
    got_scale = e.fetch(name + ".scale", M.F32, D, 1)
    table = R.e4m3_table()
    assert got_scale[5] == 1.0
    assert (table[got[5]] == 0).all()
    assert (table[got[:, :16]] == 0).all()
    assert (table[got[np.arange(D) != 5][:, 16:]] != 0).mean() > 0.9
