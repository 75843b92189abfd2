"""The oracle (oracle/mkref.cpp) pinned against independent checks, on the CPU:
  - golden vectors from PyTorch's library routines (tests/golden/golden.npz);
  - fp64 brute force on tiny inputs;
  - closed forms and invariants of the reference's host-side functions (rope3, sinusoid, sigmas, patchify).
"""
import pathlib

import numpy as np
import pytest

import mkref as R

G = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "golden.npz")


def close(a, b, tol):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    err = np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)
    assert err <= tol, f"max rel error {err:.3e} > {tol:.1e}"


# ---- number formats ----

def test_bf16_rounding_matches_torch():
    bits = np.array([R.lib().mkref_f32_to_bf16(float(v)) for v in G["bf16_in"]], dtype=np.uint16)
    want = G["bf16_bits"]
    fin = np.isfinite(G["bf16_in"])
    assert np.array_equal(bits[fin], want[fin])
    assert np.array_equal(R.bf16_bits(G["bf16_in"])[fin], want[fin])  # the vectorised twin used by the tests


def test_e4m3_decode_matches_torch():
    dec = R.e4m3_table()
    want = G["e4m3_decode"]
    ok = ~np.isnan(want)
    assert np.array_equal(np.isnan(dec), np.isnan(want))
    assert np.array_equal(dec[ok], want[ok])


def test_e4m3_encode_matches_torch():
    codes = np.array([R.lib().mkref_f32_to_e4m3(float(v)) for v in G["e4m3_in"]], dtype=np.uint8)
    assert np.array_equal(codes, G["e4m3_codes"])


def test_e4m3_encode_saturates():
    for v in (448.0, 449.0, 1e6):
        assert R.lib().mkref_f32_to_e4m3(v) == 0x7E
        assert R.lib().mkref_f32_to_e4m3(-v) == 0xFE


# ---- RNG ----

def test_rng_moments_and_determinism():
    a = R.normal(200000, 0, "w")
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    assert np.array_equal(a, R.normal(200000, 0, "w"))
    assert not np.array_equal(a[:100], R.normal(100, 1, "w"))
    assert not np.array_equal(a[:100], R.normal(100, 0, "v"))
    b = R.normal(1000, 0, "w", mean=1.0, std=0.02, round_bf16=True)
    assert np.array_equal(b, R.bf16_round(b))


# ---- primitives vs library routines ----

def test_ln_modulate_golden():
    close(R.ln_modulate(G["ln_x"], G["ln_scale"], G["ln_shift"]), G["ln_y"], 1e-6)


def test_ln_modulate_scale_zero_is_layer_norm():
    x = G["ln_x"]
    y = R.ln_modulate(x, np.zeros(96, np.float32))
    xd = x.astype(np.float64)
    close(y, (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6), 1e-6)


def test_layer_norm_golden():
    close(R.layer_norm(G["ln_x"], G["lna_g"], G["lna_b"]), G["lna_y"], 1e-6)


def test_rms_norm_golden():
    close(R.rms_norm(G["ln_x"], G["rms_w"]), G["rms_y"], 1e-6)


def test_group_norm_golden():
    close(R.group_norm(G["gn_x"], G["gn_g"], G["gn_b"]), G["gn_y"], 1e-6)


def test_activations_golden():
    close(R.gelu_tanh(G["act_x"]), G["gelu_tanh"], 1e-6)
    close(R.silu(G["act_x"]), G["silu"], 1e-6)
    close(R.geglu(G["geglu_x"]), G["geglu_y"], 1e-6)
    close(R.swiglu(G["geglu_x"]), G["swiglu_y"], 1e-6)


def test_gemm_golden():
    close(R.gemm(G["gemm_a"], G["gemm_w"], G["gemm_b"]), G["gemm_y"], 1e-6)


def test_gemm_bf16_rounds_activations_only():
    # an activation with bits below bf16 precision: the GEMM sees it rounded
    A = np.array([[1.0 + 2 ** -10, 3.0]], np.float32)
    W = np.array([[1.0, 0.0]], np.float32)
    assert R.gemm(A, W)[0, 0] == 1.0


def test_gemm_fp8_scale():
    rng = np.random.default_rng(3)
    A = rng.standard_normal((5, 64)).astype(np.float32)
    q = R.e4m3_table()[rng.integers(0, 0x7E, (16, 64))].astype(np.float32)
    s = rng.random(16).astype(np.float32) + 0.1
    want = R.bf16_round(A).astype(np.float64) @ q.T.astype(np.float64) * s
    close(R.gemm(A, q, wscale=s), want, 1e-6)


@pytest.mark.parametrize("name,block", [("attn", 0), ("attn64", 0), ("attnc", 0xFFFFFFFF), ("attnp", 12)])
def test_attention_golden(name, block):
    q, k, v = G[name + "_q"], G[name + "_k"], G[name + "_v"]
    d = q.shape[-1]
    close(R.attention(q, k, v, 1 / np.sqrt(d), 0, block), G[name + "_o"], 2e-6)


def test_attention_online_equals_two_pass_on_offset_queries():
    # q_pos0 shifts the causal prefix: rows q_pos0.. of a longer sequence see the same keys as in the full pass
    q, k, v = G["attnp_q"], G["attnp_k"], G["attnp_v"]
    full = R.attention(q, k, v, 1 / np.sqrt(128), 0, 12)
    tail = R.attention(np.ascontiguousarray(q[:, :, 8:]), k, v, 1 / np.sqrt(128), 8, 12)
    close(tail, full[:, 8:], 1e-6)


# ---- heads, RoPE, host functions ----

def test_rope_table_closed_form():
    S, h, w = 5, 3, 4
    cs = R.rope_table(S, h, w)
    assert cs.shape == (S + h * w, 64, 2)
    assert np.allclose(cs[..., 0] ** 2 + cs[..., 1] ** 2, 1, atol=1e-6)
    dims = [16, 56, 56]
    inv = np.concatenate([1.0 / 10000.0 ** (np.arange(0, d, 2) / d) for d in dims])
    axis = np.repeat([0, 1, 2], [8, 28, 28])

    def angles(pos):
        return np.array([pos[a] for a in axis]) * inv

    for t in range(S):  # text at (t, t, t)
        assert np.allclose(cs[t, :, 0], np.cos(angles((t, t, t))), atol=2e-6)
    for y in range(h):  # image at (S, y - (h - h//2), x - (w - w//2))
        for x in range(w):
            pos = (S, y - (h - h // 2), x - (w - w // 2))
            assert np.allclose(cs[S + y * w + x, :, 1], np.sin(angles(pos)), atol=2e-6)


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_heads_norm_rope_preserves_pair_norms(mode):
    rng = np.random.default_rng(mode)
    rows, heads, d = 6, 3, 128
    x = rng.standard_normal((rows, heads * d)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    cs = R.rope_table(2, 2, 2)[:rows]
    y = R.heads_norm_rope(x, heads, d, w=w, cs=cs, rope=mode)  # [heads][rows][d]
    ref = R.heads_norm_rope(x, heads, d, w=w)                   # norm only
    xr = x.reshape(rows, heads, d).astype(np.float64).transpose(1, 0, 2)
    rms = np.sqrt((xr ** 2).mean(-1, keepdims=True) + 1e-6)
    close(ref, xr / rms * w, 1e-6)
    if mode == 0:
        close(y, ref, 0)
        return
    i0 = np.arange(0, d, 2) if mode == 2 else np.arange(d // 2)
    i1 = i0 + 1 if mode == 2 else i0 + d // 2
    # rotation: per-pair norms kept, and the rotated pair equals the complex product with exp(i angle)
    close(y[..., i0] ** 2 + y[..., i1] ** 2, ref[..., i0] ** 2 + ref[..., i1] ** 2, 1e-5)
    z = (ref[..., i0] + 1j * ref[..., i1]) * (cs[None, :, :, 0] + 1j * cs[None, :, :, 1])
    close(y[..., i0], z.real, 1e-5)
    close(y[..., i1], z.imag, 1e-5)


def test_heads_scatter_rows():
    x = np.arange(2 * 256, dtype=np.float32).reshape(2, 256)
    y = R.heads_norm_rope(x, 2, 128, out_rows=5, out_row0=3)
    assert np.array_equal(y[1, 4], x[1, 128:])
    assert np.array_equal(y[0, 3], x[0, :128])
    assert not y[:, :3].any()


def test_sinusoid_closed_form():
    s = R.sinusoid(1000 * 0.37)
    f = np.exp(-np.log(10000) * np.arange(128) / 128)
    close(s[:128], np.cos(370 * f), 2e-4)  # fp32 argument rounding at arg ~ 370
    close(s[128:], np.sin(370 * f), 2e-4)
    assert np.array_equal(R.sinusoid(0.0)[:128], np.ones(128, np.float32))


def test_sigmas_invariants():
    s = R.sigmas(40, 4096)
    assert s[0] == 1.0 and s[-1] == 0.0 and len(s) == 41
    assert np.all(np.diff(s) < 0)
    # mu at 4096 tokens = max_shift 1.15: sigma(t) = e^mu / (e^mu + 1/t - 1)
    t = 1 + (1 / 40 - 1) * 20 / 39
    assert abs(s[20] - np.exp(1.15) / (np.exp(1.15) + 1 / t - 1)) < 1e-6
    # at base_seq tokens mu = base_shift
    assert abs(R.sigmas(2, 256)[1] - np.exp(0.5) / (np.exp(0.5) + 1)) < 1e-6
    # a terminal stretches the last level to it
    assert abs(R.sigmas(10, 1024, terminal=0.02)[9] - 0.02) < 1e-6


def test_patchify_round_trip_and_layout():
    rng = np.random.default_rng(0)
    lat = rng.standard_normal((16, 8, 6)).astype(np.float32)  # [C][2h][2w], h = 4, w = 3
    tok = R.patchify(lat, 4, 3)
    assert np.array_equal(R.unpatchify(tok, 16, 4, 3), lat)
    # token (y/2, x/2), feature c*4 + (y%2)*2 + x%2 (the reference's unpack layout)
    assert tok[1 * 3 + 2, 5 * 4 + 1 * 2 + 0] == lat[5, 3, 4]


def test_f16_rounding_matches_numpy_half():
    # the oracle's IEEE half rounding against numpy's float32 -> float16 conversion (nearest even): random values over
    # every binade a half holds, the subnormal range, the overflow edge, and every midpoint between adjacent halves
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200000) * np.exp2(rng.uniform(-30, 17, 200000))).astype(np.float32)
    h = np.arange(0, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = ((h[:-1].astype(np.float64) + h[1:]) / 2).astype(np.float32)  # exact in float32
    special = np.array([0.0, -0.0, 65504.0, 65519.9, 65520.0, 7e4, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0001,
                        6.0e-8, np.inf, -np.inf], dtype=np.float32)
    for a in (x, mids, -mids, special):
        want = a.astype(np.float16).astype(np.float32)
        assert np.array_equal(R.f16_round(a).view(np.uint32), want.view(np.uint32))
