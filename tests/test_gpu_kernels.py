"""Kernel parity on the GPU: each entry point of the kernel-dispatch surface (include/mkimage.h), called through the C
ABI on seeded inputs, against the oracle (oracle/mkref.cpp). Index / byte work (patchify, the RNG fill, fp8 codes,
layouts) is bit-exact; floating point is within the stated tolerance."""
import ctypes as C

import numpy as np
import pytest

import mkimage as M
import mkref as R

pytestmark = pytest.mark.gpu


_live = []  # device buffers of the running test: kept until it ends, so no pointer outlives its allocation


@pytest.fixture(autouse=True)
def _keep_buffers():
    yield
    M.sync()
    _live.clear()


def dev(a):
    d = M.Dev.from_array(np.ascontiguousarray(a))
    _live.append(d)
    return d


def bdev(a):
    """bf16 device copy of a float array."""
    d = M.Dev.from_array(M.bf16_bits(a))
    _live.append(d)
    return d


def fetch(d, shape, dtype=np.float32):
    return d.to_array(dtype, shape)


def fetch_bf16(d, shape):
    return M.bf16_to_f32(d.to_array(np.uint16, shape))


def maxrel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def gemm(A, W, **kw):
    M.call("mk_gemm", C.byref(gemm_args(A, W, **kw)), None)
    M.sync()


def gemm_args(A, W, *, bias=None, wscale=None, epi=M.EPI_STORE, c=None, c_dtype=M.F32, M_=None, batch=1, lda=None,
              ldc=0, sa=0, sc=0, gate=None, gate_alt=0, split=0, seg=0, w_dtype=M.BF16, heads=None, a_off=0):
    g = M.GemmArgs()
    g.a, g.w = A.p + a_off, W.p
    g.wscale = wscale.p if wscale is not None else None
    g.bias = bias.p if bias is not None else None
    g.c = c.p if c is not None else None
    g.gate = gate.p if gate is not None else None
    g.gate_alt, g.split, g.seg_rows = gate_alt, split, seg
    g.M, g.N, g.K = M_
    g.lda, g.ldc, g.stride_a, g.stride_c, g.batch = lda, ldc, sa, sc, batch
    g.w_dtype, g.c_dtype, g.epilogue = w_dtype, c_dtype, epi
    g.heads = C.pointer(heads) if heads is not None else None
    g._keep = heads
    return g


def gemm_grouped(*args):
    arr = (M.GemmArgs * len(args))(*args)
    M.call("mk_gemm_grouped", C.cast(arr, C.c_void_p), len(args), None)
    M.sync()


# ---------------------------------------------------------------------------------------------------------------
# GEMM

def hdev(a):
    """IEEE half device copy of a float array."""
    d = M.Dev.from_array(M.f16_bits(a))
    _live.append(d)
    return d


# the cross attention's context K and V^T from one k|v GEMM (q NULL), as half from the fp32 accumulators
# (sdxl.cpp:697-708: heads_half of the fp32 projection): within one half rounding of the float64 product, where a bf16
# intermediate (bf16 store, then half) is not
def test_gemm_heads64_kv_only_rounds_once(gpu, rng):
    S, E, H = 77, 2048, 4
    s_pad = 80
    A = rng.standard_normal((S, E)).astype(np.float32)
    W = R.bf16_round((rng.standard_normal((2 * H * 64, E)) / np.sqrt(E)).astype(np.float32))
    b = rng.standard_normal(2 * H * 64).astype(np.float32) * 0.1
    Kd, Vt = M.Dev(H * s_pad * 64 * 2), M.Dev(H * 64 * s_pad * 2)
    _live.extend([Kd, Vt])
    ha = M.HeadsArgs(None, Kd.p, Vt.p, H, 64, 0, s_pad, 0, 0, None, None, None, 0, 1e-6, 0.0, M.F16)
    gemm(bdev(A), bdev(W), bias=dev(b), epi=M.EPI_HEADS, c_dtype=M.BF16, M_=(S, 2 * H * 64, E), lda=E, heads=ha)
    y = R.bf16_round(A).astype(np.float64) @ W.astype(np.float64).T + b
    k_want = y[:, :H * 64].reshape(S, H, 64).transpose(1, 0, 2)
    v_want = y[:, H * 64:].reshape(S, H, 64).transpose(1, 2, 0)
    k_got = M.f16_to_f32(Kd.to_array(np.uint16, (H, s_pad, 64)))[:, :S]
    v_got = M.f16_to_f32(Vt.to_array(np.uint16, (H, 64, s_pad)))[:, :, M.vt_col(np.arange(S))]
    for got, want in ((k_got, k_want), (v_got, v_want)):
        tol = np.abs(want) * (2.0 ** -11 + 1e-5) + 1e-6
        assert np.all(np.abs(got - want) <= tol)
        twice = M.f16_to_f32(M.f16_bits(R.bf16_round(want.astype(np.float32))))
        assert np.any(np.abs(twice - want) > tol)


# f16 operands (the VAE's products): STORE into fp32 and half, ADD into fp32, and the pair sum of a weight stacked as
# two halves, over the tile shapes the plan takes (few rows: 128 x 128; 64-, 128- and 256-wide tiles)
@pytest.mark.parametrize("Mr, N, K", [(100, 256, 128), (700, 256, 192), (600, 128, 256), (1000, 64, 320),
                                      (3000, 512, 128)])
def test_gemm_half_operands_match_float64(gpu, rng, Mr, N, K):
    A = rng.standard_normal((Mr, K)).astype(np.float32)
    W = (rng.standard_normal((N, K)) / np.sqrt(K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) * 0.1
    Ah, Wh = M.f16_to_f32(M.f16_bits(A)).astype(np.float64), M.f16_to_f32(M.f16_bits(W)).astype(np.float64)
    want = Ah @ Wh.T + b
    dA, dW, db = hdev(A), hdev(W), dev(b)
    c32 = dev(np.zeros((Mr, N), np.float32))
    gemm(dA, dW, bias=db, c=c32, c_dtype=M.F32, M_=(Mr, N, K), lda=K, ldc=N, w_dtype=M.F16)
    assert maxrel(fetch(c32, (Mr, N)), want) <= 1e-5
    c16 = dev(np.zeros((Mr, N), np.uint16))
    gemm(dA, dW, bias=db, c=c16, c_dtype=M.F16, M_=(Mr, N, K), lda=K, ldc=N, w_dtype=M.F16)
    assert maxrel(M.f16_to_f32(c16.to_array(np.uint16, (Mr, N))), want) <= 2.0 ** -11
    x0 = rng.standard_normal((Mr, N)).astype(np.float32)
    cx = dev(x0)
    gemm(dA, dW, bias=db, c=cx, c_dtype=M.F32, M_=(Mr, N, K), lda=K, ldc=N, w_dtype=M.F16, epi=M.EPI_ADD)
    assert maxrel(fetch(cx, (Mr, N)), x0 + want) <= 1e-5
    if N % 128 == 0:
        # an fp32 weight as hi + lo halves stacked along the rows: C = A (W_hi + W_lo)^T, half output
        F_ = N // 2
        Wf = (rng.standard_normal((F_, K)) / np.sqrt(K)).astype(np.float32)
        hi = M.f16_to_f32(M.f16_bits(Wf))
        lo = M.f16_to_f32(M.f16_bits(Wf - hi))
        cp = dev(np.zeros((Mr, F_), np.float32))
        gemm(dA, hdev(np.concatenate([hi, lo])), c=cp, c_dtype=M.F32, M_=(Mr, N, K), lda=K, ldc=F_, w_dtype=M.F16,
             epi=M.EPI_PAIR_SUM)
        got = fetch(cp, (Mr, F_))
        # hi + lo holds the fp32 weight to ~2^-22: the product matches the fp32 weight's, not only its half rounding
        assert maxrel(got, Ah @ Wf.astype(np.float64).T) <= 1e-5
        assert maxrel(Ah @ hi.astype(np.float64).T, Ah @ Wf.astype(np.float64).T) > 1e-5

# ---------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("Mr,N,K", [(300, 256, 192), (512, 1024, 256), (77, 128, 64), (1000, 64, 128), (5, 640, 2560)])
def test_gemm_store_f32(gpu, rng, Mr, N, K):
    A = rng.standard_normal((Mr, K)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.05)
    b = rng.standard_normal(N).astype(np.float32)
    out = M.Dev(Mr * N * 4)
    gemm(bdev(A), bdev(W), bias=dev(b), c=out, M_=(Mr, N, K), lda=K, ldc=N)
    want = R.gemm(A, W, b)
    assert maxrel(fetch(out, (Mr, N)), want) < 1e-5


def test_gemm_gelu_bf16(gpu, rng):
    Mr, N, K = 260, 512, 320
    A = rng.standard_normal((Mr, K)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.1)
    b = rng.standard_normal(N).astype(np.float32)
    out = M.Dev(Mr * N * 2)
    gemm(bdev(A), bdev(W), bias=dev(b), c=out, c_dtype=M.BF16, epi=M.EPI_GELU_TANH, M_=(Mr, N, K), lda=K, ldc=N)
    want = R.gelu_tanh(R.gemm(A, W, b))
    got = fetch_bf16(out, (Mr, N))
    assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6


def test_gemm_gelu_wide_range(gpu, rng):
    # pre-activations over about +-60 (the epilogue's 2^(x (c1 + c2 x^2)) overflows to +inf for large negative x and
    # underflows to 0 for large positive x): every element within bf16 rounding of the oracle's tanh form, all finite
    Mr, N, K = 256, 256, 256
    A = R.bf16_round(rng.standard_normal((Mr, K)).astype(np.float32))  # the operands the GPU multiplies
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 1.25)
    out = M.Dev(Mr * N * 2)
    gemm(bdev(A), bdev(W), c=out, c_dtype=M.BF16, epi=M.EPI_GELU_TANH, M_=(Mr, N, K), lda=K, ldc=N)
    y = R.gemm(A, W)
    want = R.gelu_tanh(y)
    got = fetch_bf16(out, (Mr, N))
    assert np.abs(y).max() > 40 and (y < -10).any()
    assert np.isfinite(got).all()
    assert (np.abs(got - want) <= 2 ** -7 * np.abs(want) + 1e-6).all()


@pytest.mark.parametrize("epi", [M.EPI_GATE_ADD, M.EPI_GATE_TANH, M.EPI_ADD])
def test_gemm_residual_epilogues(gpu, rng, epi):
    # batched with strides (rows of one batch item inside a longer sequence), gate rows split as the 2.1 graph's
    B, Mr, N, K, T = 2, 200, 256, 128, 230
    A = rng.standard_normal((B, T, K)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.05)
    b = rng.standard_normal(N).astype(np.float32)
    gates = rng.standard_normal((2, N)).astype(np.float32)
    X = rng.standard_normal((B, Mr, N)).astype(np.float32)
    Xd = dev(X)
    split = 37
    # A holds the whole sequence [B][T][K]; the GEMM reads rows 30 .. 30 + Mr of each batch item
    gemm(bdev(A), bdev(W), bias=dev(b), c=Xd, epi=epi, M_=(Mr, N, K), batch=B, lda=K, ldc=N, sa=T * K, sc=Mr * N,
         gate=dev(gates), gate_alt=N, split=split, seg=Mr, a_off=30 * K * 2)
    want = X.astype(np.float64).copy()
    for bi in range(B):
        y = R.gemm(A[bi, 30:], W, b)
        if epi == M.EPI_ADD:
            want[bi] += y
        else:
            g = np.where(np.arange(Mr)[:, None] < split, gates[1], gates[0])
            want[bi] += (np.tanh(g) if epi == M.EPI_GATE_TANH else g) * y
    assert maxrel(fetch(Xd, (B, Mr, N)), want) < 1e-5


def test_gemm_fp8_weights(gpu, rng):
    Mr, N, K = 333, 256, 256
    A = rng.standard_normal((Mr, K)).astype(np.float32)
    Wf = rng.standard_normal((N, K)).astype(np.float32) * 0.02
    scale = (np.abs(Wf).max(1) / 448).astype(np.float32)
    codes = np.array([[R.lib().mkref_f32_to_e4m3(float(v)) for v in row] for row in Wf / scale[:, None]],
                     dtype=np.uint8)
    q = R.e4m3_table()[codes]
    b = rng.standard_normal(N).astype(np.float32)
    out = M.Dev(Mr * N * 4)
    gemm(bdev(A), dev(codes), bias=dev(b), wscale=dev(scale), c=out, M_=(Mr, N, K), lda=K, ldc=N, w_dtype=M.FP8)
    assert maxrel(fetch(out, (Mr, N)), R.gemm(A, q, b, wscale=scale)) < 1e-5


def test_gemm_fp8_every_code(gpu):
    # one-hot activations pick single weight columns: C[m][n] = e4m3(code m) * scale[n], exactly, for every
    # non-NaN code (the fp8 -> bf16 conversion on the way into LDS is exact)
    table = R.e4m3_table()
    codes = np.arange(256, dtype=np.uint8)
    codes[np.isnan(table)] = 0
    N, K = 64, 256
    W = np.tile(codes, (N, 1))
    A = np.eye(K, dtype=np.float32)
    scale = np.linspace(0.5, 2.0, N).astype(np.float32)
    out = M.Dev(K * N * 4)
    _live.append(out)
    gemm(bdev(A), dev(W), wscale=dev(scale), c=out, M_=(K, N, K), lda=K, ldc=N, w_dtype=M.FP8)
    want = (table[codes][:, None].astype(np.float32) * scale[None, :]).astype(np.float32)
    assert np.array_equal(fetch(out, (K, N)), want)


@pytest.mark.parametrize("mode,row0,q_row0,k_scale,odt", [(2, 40, 40, 0.0, M.BF16), (1, 0, 0, 0.0, M.BF16),
                                                          (0, 17, 0, 0.0, M.BF16), (2, 40, 40, 0.3, M.BF16),
                                                          (2, 40, 0, 0.3, M.F16), (0, 0, 0, 0.0, M.F16)])
def test_gemm_heads_epilogue(gpu, rng, mode, row0, q_row0, k_scale, odt):
    # q | k | v columns -> per-head RMSNorm + RoPE -> Q, K [b][h][pad][128] and V^T [b][h][128][pad]
    B, Mr, H = 2, 150, 2
    D = H * 128
    K_ = 256
    q_pad, k_pad = 256, 256
    A = rng.standard_normal((B, Mr, K_)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((3 * D, K_)).astype(np.float32) * 0.05)
    b = rng.standard_normal(3 * D).astype(np.float32) * 0.1
    nq = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    nk = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    cs = R.rope_table(row0, 14, 14)[: row0 + Mr] if row0 else R.rope_table(0, 15, 10)[:Mr]
    Q, Kd, Vt = M.Dev(B * H * q_pad * 256), M.Dev(B * H * k_pad * 256), M.Dev(B * H * k_pad * 256)
    ha = M.HeadsArgs(Q.p, Kd.p, Vt.p, H, 128, q_pad, k_pad, row0, q_row0, None, None, None, mode, 1e-6, k_scale,
                     odt)
    nqd, nkd, csd = dev(nq), dev(nk), dev(cs)
    ha.norm_q, ha.norm_k, ha.rope = nqd.p, nkd.p, csd.p
    Ad = bdev(A)
    gemm(Ad, bdev(W), bias=dev(b), epi=M.EPI_HEADS, c_dtype=M.BF16, M_=(Mr, 3 * D, K_), batch=B, lda=K_,
         sa=Mr * K_, heads=ha)
    get = (lambda d, sh: M.f16_to_f32(d.to_array(np.uint16, sh))) if odt == M.F16 else fetch_bf16
    gq = get(Q, (B, H, q_pad, 128))
    gk = get(Kd, (B, H, k_pad, 128))
    gv = get(Vt, (B, H, 128, k_pad))
    for bi in range(B):
        y = R.gemm(A[bi], W, b)
        tab = cs[row0:]
        wq = R.heads_norm_rope(y, H, 128, col0=0, w=nq, cs=tab, rope=mode)
        wk = R.heads_norm_rope(y, H, 128, col0=D, w=nk, cs=tab, rope=mode) * (k_scale or 1.0)
        wv = R.heads_norm_rope(y, H, 128, col0=2 * D)
        vcols = M.vt_col(np.arange(row0, row0 + Mr))
        for got, want in ((gq[bi][:, q_row0:q_row0 + Mr], wq), (gk[bi][:, row0:row0 + Mr], wk),
                          (gv[bi][:, :, vcols].transpose(0, 2, 1), wv)):
            assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6
    # rows outside the written range stay zero (a tile's rows past M store into the last row, with its bits)
    assert not gk[:, :, :row0].any() and not gk[:, :, row0 + Mr:].any()
    assert not gq[:, :, :q_row0].any() and not gq[:, :, q_row0 + Mr:].any()


# 64-dim heads (the SDXL form: half, no norm, no RoPE) on 128-channel tiles: q | k | v and Q alone, batch 2, row
# counts that end inside a tile and inside a 16-key group; each value within one rounding (half or bf16) of the
# oracle's GEMM, padding rows untouched (zero)
@pytest.mark.parametrize("Mr,H,qonly,odt,k_scale", [(1024, 20, False, M.F16, 0.0), (300, 10, False, M.F16, 0.5),
                                                    (77, 4, False, M.BF16, 0.0), (1024, 20, True, M.F16, 0.0),
                                                    (130, 2, True, M.BF16, 0.0)])
def test_gemm_heads64_epilogue(gpu, rng, Mr, H, qonly, odt, k_scale):
    B, d, K_ = 2, 64, 320
    D = H * d
    parts = 1 if qonly else 3
    q_pad, k_pad = -(-Mr // 256) * 256, -(-Mr // 64) * 64
    A = rng.standard_normal((B, Mr, K_)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((parts * D, K_)).astype(np.float32) * 0.05)
    b = rng.standard_normal(parts * D).astype(np.float32) * 0.1
    Q = dev(np.zeros(B * H * q_pad * d, np.uint16))
    Kd = None if qonly else dev(np.zeros(B * H * k_pad * d, np.uint16))
    Vt = None if qonly else dev(np.zeros(B * H * k_pad * d, np.uint16))
    ha = M.HeadsArgs(Q.p, None if qonly else Kd.p, None if qonly else Vt.p, H, d, q_pad, k_pad, 0, 0, None, None,
                     None, 0, 0.0, k_scale, odt)
    gemm(bdev(A), bdev(W), bias=dev(b), epi=M.EPI_HEADS, c_dtype=M.BF16, M_=(Mr, parts * D, K_), batch=B, lda=K_,
         sa=Mr * K_, heads=ha)
    get = (lambda t, sh: M.f16_to_f32(t.to_array(np.uint16, sh))) if odt == M.F16 else fetch_bf16
    rnd = R.f16_round if odt == M.F16 else R.bf16_round
    ulp = 2 ** -10 if odt == M.F16 else 2 ** -7
    gq = get(Q, (B, H, q_pad, d))
    outs = [(gq, 0)]
    if not qonly:
        outs += [(get(Kd, (B, H, k_pad, d)), D), (get(Vt, (B, H, d, k_pad)), 2 * D)]
    for bi in range(B):
        y = R.gemm(A[bi], W, b)
        for j, (g, col0) in enumerate(outs):
            want = y[:, col0:col0 + D].reshape(Mr, H, d).transpose(1, 0, 2)  # [H][Mr][d]
            if j == 1:
                want = want * (k_scale or 1.0)
            if j == 2:
                got = g[bi][:, :, M.vt_col(np.arange(Mr))].transpose(0, 2, 1)
                pad = g[bi][:, :, M.vt_col(np.arange(Mr, k_pad))] if Mr < k_pad else np.zeros(1)
            else:
                got = g[bi][:, :Mr]
                pad = g[bi][:, Mr:]
            assert np.abs(got - rnd(want)).max() <= ulp * np.abs(want).max()
            assert not pad.any()


def test_gemm_grouped_residual_equals_separate_launches(gpu, rng):
    # an image-like and a text-like problem (own A, W, bias, gate, residual, M and strides) in one launch give the
    # bits of two launches, and match the oracle
    N, K = 256, 192
    probs = []
    for Mr, B in ((300, 2), (40, 2)):
        A = rng.standard_normal((B, Mr, K)).astype(np.float32)
        W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.05)
        b = rng.standard_normal(N).astype(np.float32)
        gt = rng.standard_normal(N).astype(np.float32)
        X = rng.standard_normal((B, Mr, N)).astype(np.float32)
        probs.append((Mr, B, A, W, b, gt, X, bdev(A), bdev(W), dev(b), dev(gt)))
    outs = []
    for grouped in (False, True):
        xs = [dev(pr[6]) for pr in probs]
        args = [gemm_args(Ad, Wd, bias=bd, c=xd, epi=M.EPI_GATE_ADD, M_=(Mr, N, K), batch=B, lda=K, ldc=N,
                          sa=Mr * K, sc=Mr * N, gate=gd)
                for (Mr, B, _, _, _, _, _, Ad, Wd, bd, gd), xd in zip(probs, xs)]
        if grouped:
            gemm_grouped(*args)
        else:
            for g in args:
                M.call("mk_gemm", C.byref(g), None)
            M.sync()
        outs.append([fetch(xd, pr[6].shape) for xd, pr in zip(xs, probs)])
    for sep, grp, (Mr, B, A, W, b, gt, X, *_) in zip(outs[0], outs[1], probs):
        assert np.array_equal(sep, grp)
        want = X.astype(np.float64) + gt * np.stack([R.gemm(A[i], W, b) for i in range(B)])
        assert maxrel(grp, want) < 1e-5


def test_gemm_grouped_heads_and_gelu(gpu, rng):
    # the QKV pair of a dual-stream block: text rows at 0, image rows at row0 = S, own norms, one Q / K / V^T
    Bt, H, S, Nimg, K_ = 2, 2, 24, 136, 256
    D = H * 128
    q_pad = k_pad = 256
    Q, Kd, Vt = [M.Dev(Bt * H * q_pad * 256) for _ in range(3)]
    cs = R.rope_table(S, 8, 17)
    csd = dev(cs)
    args, ref = [], []
    for rows, row0 in ((Nimg, S), (S, 0)):
        A = rng.standard_normal((Bt, rows, K_)).astype(np.float32)
        W = R.bf16_round(rng.standard_normal((3 * D, K_)).astype(np.float32) * 0.05)
        b = rng.standard_normal(3 * D).astype(np.float32) * 0.1
        nq = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
        nk = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
        ha = M.HeadsArgs(Q.p, Kd.p, Vt.p, H, 128, q_pad, k_pad, row0, row0, dev(nq).p, dev(nk).p, csd.p, 2, 1e-6)
        args.append(gemm_args(bdev(A), bdev(W), bias=dev(b), epi=M.EPI_HEADS, c_dtype=M.BF16, M_=(rows, 3 * D, K_),
                              batch=Bt, lda=K_, sa=rows * K_, heads=ha))
        ref.append((rows, row0, A, W, b, nq, nk))
    gemm_grouped(*args)
    gq = fetch_bf16(Q, (Bt, H, q_pad, 128))
    gk = fetch_bf16(Kd, (Bt, H, k_pad, 128))
    gv = fetch_bf16(Vt, (Bt, H, 128, k_pad))
    for rows, row0, A, W, b, nq, nk in ref:
        for bi in range(Bt):
            y = R.gemm(A[bi], W, b)
            tab = cs[row0:row0 + rows]
            vcols = M.vt_col(np.arange(row0, row0 + rows))
            wq = R.heads_norm_rope(y, H, 128, col0=0, w=nq, cs=tab, rope=2)
            wk = R.heads_norm_rope(y, H, 128, col0=D, w=nk, cs=tab, rope=2)
            wv = R.heads_norm_rope(y, H, 128, col0=2 * D)
            for got, want in ((gq[bi][:, row0:row0 + rows], wq), (gk[bi][:, row0:row0 + rows], wk),
                              (gv[bi][:, :, vcols].transpose(0, 2, 1), wv)):
                assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6
    # GELU pair into one hidden buffer (image rows, then text rows)
    N, K = 512, 128
    A0, A1 = (rng.standard_normal((r, K)).astype(np.float32) for r in (300, 48))
    W0, W1 = (R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.1) for _ in range(2))
    hid = M.Dev((300 + 48) * N * 2)
    _live.append(hid)
    g0 = gemm_args(bdev(A0), bdev(W0), c=hid, c_dtype=M.BF16, epi=M.EPI_GELU_TANH, M_=(300, N, K), lda=K, ldc=N)
    g1 = gemm_args(bdev(A1), bdev(W1), c_dtype=M.BF16, epi=M.EPI_GELU_TANH, M_=(48, N, K), lda=K, ldc=N)
    g1.c = hid.p + 300 * N * 2
    gemm_grouped(g0, g1)
    got = fetch_bf16(hid, (348, N))
    for g, want in ((got[:300], R.gelu_tanh(R.gemm(A0, W0))), (got[300:], R.gelu_tanh(R.gemm(A1, W1)))):
        assert np.abs(g - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6
    # problems of unequal N are refused
    g1.N = 256
    arr = (M.GemmArgs * 2)(g0, g1)
    assert M.lib().mk_gemm_grouped(C.cast(arr, C.c_void_p), 2, None) == 1
    assert b"equal N" in M.lib().mk_last_error()


# Stream-K: launches of a wave or more of 256 x 256 tiles whose last wave would leave CUs idle split the tail's k
# steps over the whole chip (partials published by one workgroup, added by the one closing the tile).
@pytest.mark.parametrize("epi,cdt,w8", [(M.EPI_GATE_ADD, M.F32, False), (M.EPI_GATE_ADD, M.F32, True),
                                        (M.EPI_GELU_TANH, M.BF16, False)])
def test_gemm_stream_k_matches_oracle_and_repeats(gpu, rng, epi, cdt, w8):
    N = 3072 if epi == M.EPI_GATE_ADD else 12288
    K = 256
    shapes = ((8192, 1), (512, 1))  # 34 token tiles: 408 (or 1632) tiles, 1.6 (6.4) waves
    A = [rng.standard_normal((Mr, K)).astype(np.float32) for Mr, _ in shapes]
    if w8:
        Wf = rng.standard_normal((N, K)).astype(np.float32) * 0.05
        scale = (np.abs(Wf).max(1) / 448).astype(np.float32)
        table = R.e4m3_table()
        mags, a = table[:127], np.abs(Wf / scale[:, None])
        i = np.clip(np.searchsorted(mags, a), 1, 126)
        near = np.where(a - mags[i - 1] <= mags[i] - a, i - 1, i).astype(np.uint8)
        codes = near | np.where(Wf < 0, 0x80, 0).astype(np.uint8)
        Wq, Wd, sd = table[codes] * scale[:, None], dev(codes), dev(scale)
    else:
        Wq = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.05)
        Wd, sd = bdev(Wq), None
    b = dev(rng.standard_normal(N).astype(np.float32))
    gt = rng.standard_normal(N).astype(np.float32)
    X = [rng.standard_normal((Mr, N)).astype(np.float32) for Mr, _ in shapes]
    outs = []
    for rep in range(2):
        cs = [dev(x) if epi == M.EPI_GATE_ADD else M.Dev(Mr * N * 2) for x, (Mr, _) in zip(X, shapes)]
        _live.extend(cs)
        args = [gemm_args(bdev(a), Wd, bias=b, wscale=sd, c=c, c_dtype=cdt, epi=epi, M_=(Mr, N, K), lda=K, ldc=N,
                          gate=dev(gt), w_dtype=M.FP8 if w8 else M.BF16)
                for a, c, (Mr, _) in zip(A, cs, shapes)]
        gemm_grouped(*args)
        outs.append([fetch(c, (Mr, N)) if cdt == M.F32 else fetch_bf16(c, (Mr, N)) for c, (Mr, _) in zip(cs, shapes)])
    bias = fetch(b, (N,))
    for i, (Mr, _) in enumerate(shapes):
        assert np.array_equal(outs[0][i], outs[1][i])  # the fixed reduction order repeats bit for bit
        y = R.gemm(A[i], Wq, bias)
        if epi == M.EPI_GATE_ADD:
            assert maxrel(outs[0][i], X[i].astype(np.float64) + gt * y) < 1e-5
        else:
            want = R.gelu_tanh(y)
            assert np.abs(outs[0][i] - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6


def _sk_problem(rng, K=6144):
    """A grouped gated-residual GEMM that runs stream-K: 8192 + 512 rows x 3072 x K (408 tiles of 256 x 256, 1.6 waves
    on 256 compute units, K of 96 k steps)."""
    N = 3072
    shapes = (8192, 512)
    A = [R.bf16_round(rng.standard_normal((Mr, K)).astype(np.float32)) for Mr in shapes]
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    b = rng.standard_normal(N).astype(np.float32)
    gt = rng.standard_normal(N).astype(np.float32)
    X = [rng.standard_normal((Mr, N)).astype(np.float32) for Mr in shapes]
    return dict(N=N, K=K, shapes=shapes, A=A, W=W, b=b, gt=gt, X=X, Ad=[bdev(a) for a in A], Wd=bdev(W), bd=dev(b),
                gd=dev(gt))


def _sk_launch(P, stream=None):
    cs = [dev(x) for x in P["X"]]
    args = [gemm_args(a, P["Wd"], bias=P["bd"], c=c, epi=M.EPI_GATE_ADD, M_=(Mr, P["N"], P["K"]), lda=P["K"],
                      ldc=P["N"], gate=P["gd"]) for a, c, Mr in zip(P["Ad"], cs, P["shapes"])]
    arr = (M.GemmArgs * 2)(*args)
    _live.append(arr)
    M.call("mk_gemm_grouped", C.cast(arr, C.c_void_p), 2, stream)
    return cs


def test_gemm_stream_k_long_k_matches_oracle_and_repeats(gpu, rng):
    P = _sk_problem(rng)
    outs = []
    for _ in range(2):
        cs = _sk_launch(P)
        M.sync()
        outs.append([fetch(c, (Mr, P["N"])) for c, Mr in zip(cs, P["shapes"])])
    for i, Mr in enumerate(P["shapes"]):
        assert np.array_equal(outs[0][i], outs[1][i])  # the fixed reduction order repeats bit for bit
        rows = np.sort(rng.choice(Mr, 48, replace=False))
        want = P["X"][i][rows].astype(np.float64) + P["gt"] * R.gemm(P["A"][i][rows], P["W"], P["b"])
        assert maxrel(outs[0][i][rows], want) < 1e-5


def test_gemm_stream_k_on_two_streams_at_once(gpu, rng):
    # two streams issue stream-K launches concurrently (each its own workspace): every result equals the same
    # launch run alone
    P = [_sk_problem(np.random.default_rng(s)) for s in (21, 22)]
    alone = []
    for p in P:
        cs = _sk_launch(p)
        M.sync()
        alone.append([fetch(c, (Mr, p["N"])) for c, Mr in zip(cs, p["shapes"])])
    streams = []
    for _ in range(2):
        h = C.c_void_p()
        M.call("mk_stream_create", C.byref(h))
        streams.append(h.value)
    try:
        runs = []
        for _ in range(3):
            for p, st in zip(P, streams):
                runs.append((p, _sk_launch(p, st), len(runs) % 2))
        for st in streams:
            M.call("mk_stream_synchronize", st)
        for p, cs, j in runs:
            for i, (c, Mr) in enumerate(zip(cs, p["shapes"])):
                assert np.array_equal(fetch(c, (Mr, p["N"])), alone[j][i])
    finally:
        M.sync()
        for st in streams:
            M.call("mk_stream_destroy", st)


def test_gemm_stream_k_gave_up_wait_is_reported(gpu, rng):
    # a zero wait bound makes every owner of a split tile give up at once (the kernel still completes, from whatever
    # the partial slots hold); the next synchronisation reports it, once, and the default bound restores results
    P = _sk_problem(rng)
    ref = _sk_launch(P)
    M.sync()
    want = [fetch(c, (Mr, P["N"])) for c, Mr in zip(ref, P["shapes"])]
    M.call("mk_gemm_set_wait_limit", 0)
    try:
        _sk_launch(P)
        assert M.lib().mk_synchronize() == 3  # MK_ERR_DEVICE
        assert b"gave up" in M.lib().mk_last_error()
    finally:
        M.call("mk_gemm_set_wait_limit", 1 << 26)
    M.sync()  # reported once
    cs = _sk_launch(P)
    M.sync()
    for c, Mr, w in zip(cs, P["shapes"], want):
        assert np.array_equal(fetch(c, (Mr, P["N"])), w)


def test_gemm_stream_k_heads(gpu, rng):
    # the QKV heads epilogue on 4.5 waves of tiles: 2 x 4096 rows, 24 heads
    B, Mr, H, K_ = 2, 4096, 24, 256
    D = H * 128
    q_pad = k_pad = 4096
    A = rng.standard_normal((B, Mr, K_)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((3 * D, K_)).astype(np.float32) * 0.05)
    bb = rng.standard_normal(3 * D).astype(np.float32) * 0.1
    nq = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    nk = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    cs = R.rope_table(0, 64, 64)
    Q, Kd, Vt = M.Dev(B * H * q_pad * 256), M.Dev(B * H * k_pad * 256), M.Dev(B * H * k_pad * 256)
    _live.extend([Q, Kd, Vt])
    ha = M.HeadsArgs(Q.p, Kd.p, Vt.p, H, 128, q_pad, k_pad, 0, 0, dev(nq).p, dev(nk).p, dev(cs).p, 2, 1e-6, 0.0)
    gemm(bdev(A), bdev(W), bias=dev(bb), epi=M.EPI_HEADS, c_dtype=M.BF16, M_=(Mr, 3 * D, K_), batch=B, lda=K_,
         sa=Mr * K_, heads=ha)
    rows = np.sort(rng.choice(Mr, 200, replace=False))
    gq = fetch_bf16(Q, (B, H, q_pad, 128))
    gk = fetch_bf16(Kd, (B, H, k_pad, 128))
    gv = fetch_bf16(Vt, (B, H, 128, k_pad))
    for bi in range(B):
        y = R.gemm(A[bi][rows], W, bb)
        tab = cs[rows]
        wq = R.heads_norm_rope(y, H, 128, col0=0, w=nq, cs=tab, rope=2)
        wk = R.heads_norm_rope(y, H, 128, col0=D, w=nk, cs=tab, rope=2)
        wv = R.heads_norm_rope(y, H, 128, col0=2 * D)
        for got, want in ((gq[bi][:, rows], wq), (gk[bi][:, rows], wk),
                          (gv[bi][:, :, M.vt_col(rows)].transpose(0, 2, 1), wv)):
            assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6


def test_vt_col_is_an_involution_within_groups():
    k = np.arange(4096)
    assert np.array_equal(M.vt_col(M.vt_col(k)), k)
    assert np.array_equal(np.sort(M.vt_col(k[:16])), k[:16])
    assert list(M.vt_col(np.arange(16))) == [0, 1, 2, 3, 8, 9, 10, 11, 4, 5, 6, 7, 12, 13, 14, 15]


def test_gemm_rejects_bad_shapes(gpu):
    g = M.GemmArgs()
    d = M.Dev(1024)
    g.a = g.w = g.c = d.p
    g.M, g.N, g.K, g.lda, g.ldc, g.batch, g.w_dtype = 4, 60, 64, 64, 60, 1, M.BF16
    assert M.lib().mk_gemm(C.byref(g), None) == 1
    assert b"multiples of 64" in M.lib().mk_last_error()


def test_gemm_empty_problems(gpu, rng):
    # a problem with no rows (M = 0) or no batch items launches nothing and leaves C as it was; beside a non-empty
    # problem in a grouped launch it drops out, and the other problem gets the bits of its own launch
    N, K, Mr = 128, 128, 200
    A = rng.standard_normal((Mr, K)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.05)
    Ad, Wd = bdev(A), bdev(W)
    sentinel = np.full(Mr * N, 7.5, np.float32)
    for m, batch in ((0, 1), (Mr, 0)):
        out = dev(sentinel)
        gemm(Ad, Wd, c=out, M_=(m, N, K), batch=batch, lda=K, ldc=N)
        assert np.array_equal(fetch(out, (Mr * N,)), sentinel), (m, batch)
    solo, grp, idle = dev(sentinel), dev(sentinel), dev(sentinel)
    gemm(Ad, Wd, c=solo, M_=(Mr, N, K), lda=K, ldc=N)
    gemm_grouped(gemm_args(Ad, Wd, c=grp, M_=(Mr, N, K), lda=K, ldc=N),
                 gemm_args(Ad, Wd, c=idle, M_=(0, N, K), lda=K, ldc=N))
    assert np.array_equal(fetch(grp, (Mr, N)), fetch(solo, (Mr, N)))
    assert np.array_equal(fetch(idle, (Mr * N,)), sentinel)
    assert maxrel(fetch(solo, (Mr, N)), R.gemm(A, W)) < 1e-5


def test_elementwise_empty_inputs(gpu):
    # zero elements or rows: the call succeeds and writes nothing
    sentinel = np.full(256, 7.5, np.float32)
    x, y, g = dev(sentinel), dev(sentinel), dev(sentinel)
    M.call("mk_silu", x.p, 0, None)
    M.call("mk_gelu_tanh", x.p, 0, None)
    M.call("mk_rms_norm", x.p, 0, 64, g.p, 0.0, 1e-6, y.p, None)
    M.call("mk_gate_add", x.p, y.p, M.F32, 0, 64, g.p, 0, 0, 1, 0, None)
    M.sync()
    for d in (x, y, g):
        assert np.array_equal(fetch(d, (256,)), sentinel)


# ---------------------------------------------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------------------------------------------

def hdev(a):
    """IEEE half device copy of a float array."""
    d = M.Dev.from_array(M.f16_bits(a))
    _live.append(d)
    return d


def run_attention(q, k, v, scale, q_pos0=0, block=0, dtype=M.BF16, hole=None):
    """q [B][H][Tq][d], k, v [B][Hkv][Tk][d] (floats exact in `dtype`, bf16 or f16; Hkv dividing H) through
    mk_attention; returns [B][Tq][H*d]."""
    B, H, Tq, d = q.shape
    Hkv, Tk = k.shape[1], k.shape[2]
    q_pad = (Tq + 255) // 256 * 256
    k_pad = (Tk + 63) // 64 * 64
    qp = np.zeros((B, H, q_pad, d), np.float32)
    qp[:, :, :Tq] = q
    kp = np.zeros((B, Hkv, k_pad, d), np.float32)
    kp[:, :, :Tk] = k
    vt = np.zeros((B, Hkv, d, k_pad), np.float32)
    vt[:, :, :, M.vt_col(np.arange(Tk))] = v.transpose(0, 1, 3, 2)
    out = dev(np.zeros(B * Tq * H * d, np.uint16))
    up = hdev if dtype == M.F16 else bdev
    kh = None if hole is None else np.ascontiguousarray(np.array(hole, dtype=np.uint32).reshape(-1))
    M.call("mk_attention", up(qp).p, up(kp).p, up(vt).p, out.p, dtype, B, H, Hkv, d, Tq, q_pad, Tk, k_pad, H * d,
           Tq * H * d, q_pos0, block, scale, None if kh is None else kh.ctypes.data, None)
    M.sync()
    return fetch_bf16(out, (B, Tq, H * d))


# ragged query blocks and a ragged last key tile over a long key range (d 128: 300 queries, 2000 keys)
@pytest.mark.parametrize("d,Tq,Tk,block,q_pos0", [(128, 300, 300, 0, 0), (128, 64, 4352 // 17, 0, 0),
                                                  (64, 333, 77, 0, 0), (64, 256, 1000, 0, 0), (128, 300, 2000, 0, 0),
                                                  (128, 200, 260, 60, 60), (128, 260, 260, 60, 0),
                                                  (128, 190, 190, 0xFFFFFFFF, 0)])
def test_attention_matches_oracle(gpu, rng, d, Tq, Tk, block, q_pos0):
    B, H = 2, 3
    q = R.bf16_round(rng.standard_normal((B, H, Tq, d)).astype(np.float32))
    k = R.bf16_round(rng.standard_normal((B, H, Tk, d)).astype(np.float32))
    v = R.bf16_round(rng.standard_normal((B, H, Tk, d)).astype(np.float32))
    got = run_attention(q, k, v, 1 / np.sqrt(d), q_pos0, block)
    want = R.attention(q, k, v, 1 / np.sqrt(d), q_pos0, block)
    dd = R.diff(got, want, d)
    # P is rounded to bf16 for the MFMA, the output stored bf16
    assert dd["min_cos"] > 0.9999 and dd["max_rel"] < 1e-2, dd


# the reference's half heads (its 2.1 graph and SDXL): half Q, K, V and probabilities, the scale-0 path (K carrying
# the softmax scale in log2 units) as the engine runs it, with the causal text prefix and offset queries
@pytest.mark.parametrize("d,Tq,Tk,block,q_pos0,scale", [(128, 300, 300, 0, 0, 0.0), (128, 200, 460, 60, 260, 0.0),
                                                        (128, 260, 260, 60, 0, 0.0), (64, 333, 77, 0, 0, 0.125),
                                                        (64, 256, 1000, 0, 0, 0.125), (128, 300, 2000, 0, 0, 0.0)])
def test_attention_half_matches_oracle(gpu, rng, d, Tq, Tk, block, q_pos0, scale):
    B, H = 2, 3
    q = R.f16_round(rng.standard_normal((B, H, Tq, d)).astype(np.float32))
    k = rng.standard_normal((B, H, Tk, d)).astype(np.float32)
    if scale == 0.0:
        k = k / np.sqrt(d) * np.log2(np.e)
    k = R.f16_round(k)
    v = R.f16_round(rng.standard_normal((B, H, Tk, d)).astype(np.float32))
    eff = float(np.log(2.0)) if scale == 0.0 else scale
    got = run_attention(q, k, v, scale, q_pos0, block, dtype=M.F16)
    want = R.attention(q, k, v, eff, q_pos0, block)
    dd = R.diff(got, want, d)
    assert dd["min_cos"] > 0.9999 and dd["max_rel"] < 1e-2, dd


@pytest.mark.parametrize("d,Tq,Tk,block,q_pos0,kscale", [
    (128, 300, 300, 0, 0, 1.0), (128, 4352 // 17, 4352, 0, 0, 1.0), (64, 333, 77, 0, 0, 1.0),
    (128, 200, 260, 60, 60, 1.0), (128, 260, 260, 60, 0, 1.0), (128, 190, 190, 0xFFFFFFFF, 0, 1.0),
    (128, 256, 512, 0, 0, 6.0), (128, 300, 2000, 0, 0, 6.0), (64, 256, 1000, 0xFFFFFFFF, 0, 6.0)])
def test_attention_unit_scale(gpu, rng, d, Tq, Tk, block, q_pos0, kscale):
    # scale 0: K already carries the softmax scale in log2 units (K' = bf16(k / sqrt(d) * log2 e)); equal to the
    # softmax of q K'^T ln 2. kscale 6 makes the logits large (the running max moves on many tiles).
    B, H = 2, 3
    q = R.bf16_round(rng.standard_normal((B, H, Tq, d)).astype(np.float32))
    k = rng.standard_normal((B, H, Tk, d)).astype(np.float32) * kscale
    kp = R.bf16_round(k / np.sqrt(d) * np.log2(np.e))
    v = R.bf16_round(rng.standard_normal((B, H, Tk, d)).astype(np.float32))
    got = run_attention(q, kp, v, 0.0, q_pos0, block)
    want = R.attention(q, kp, v, float(np.log(2.0)), q_pos0, block)
    dd = R.diff(got, want, d)
    assert dd["min_cos"] > 0.9999 and dd["max_rel"] < 1e-2, dd


# Scores that jump late in the key range (unit scale, bf16 and half): keys [s, s + 40) carry a logit some 30 log2
# units above every earlier score, so the running max moves by far more than the lazy-rescale margin on a tile that
# is not the first. Before that tile's redo its speculative probabilities reach 2^30 (+inf in half), and the lane's
# row-sum part that decides the redo has to catch it.
@pytest.mark.parametrize("dtype", [M.BF16, M.F16])
@pytest.mark.parametrize("s", [600, 984])
def test_attention_late_score_jump(gpu, rng, dtype, s):
    B, H, Tq, Tk, d = 1, 2, 256, 1024, 128
    rnd = R.f16_round if dtype == M.F16 else R.bf16_round
    q = rng.standard_normal((B, H, Tq, d)).astype(np.float32)
    q[..., 0] = 1.0
    q = rnd(q)
    kp = rng.standard_normal((B, H, Tk, d)).astype(np.float32) / np.sqrt(d) * np.log2(np.e)
    kp[:, :, s:s + 40, 0] = 30.0
    kp = rnd(kp)
    v = rnd(rng.standard_normal((B, H, Tk, d)).astype(np.float32))
    got = run_attention(q, kp, v, 0.0, dtype=dtype)
    want = R.attention(q, kp, v, float(np.log(2.0)), 0, 0)
    assert np.all(np.isfinite(got))
    dd = R.diff(got, want, d)
    assert dd["min_cos"] > 0.9999 and dd["max_rel"] < 1e-2, dd


def test_attention_golden(gpu):
    import pathlib
    G = np.load(pathlib.Path(__file__).resolve().parent / "golden" / "golden.npz")
    for name, block in (("attn", 0), ("attn64", 0), ("attnc", 0xFFFFFFFF), ("attnp", 12)):
        q, k, v = G[name + "_q"], G[name + "_k"], G[name + "_v"]
        got = run_attention(q, k, v, 1 / np.sqrt(q.shape[-1]), 0, block)
        dd = R.diff(got, G[name + "_o"], q.shape[-1])
        assert dd["min_cos"] > 0.9999 and dd["max_rel"] < 1e-2, (name, dd)


# ---------------------------------------------------------------------------------------------------------------
# bandwidth-bound kernels
# ---------------------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n", [3072, 2048, 4096, 1280])  # row-sized kernels for 2048/3072/4096, generic otherwise
def test_ln_modulate(gpu, rng, n):
    rows = 230
    x = (rng.standard_normal((rows, n)) * 3 + 1).astype(np.float32)
    mod = rng.standard_normal((2, 2, n)).astype(np.float32) * 0.3  # row r<split takes mod[1]: [shift, scale]
    y = M.Dev(rows * n * 2)
    md = dev(mod)
    split, seg = 20, 115
    M.call("mk_ln_modulate", dev(x).p, rows, n, md.p + n * 4, md.p, 2 * n, split, seg, 1e-6, y.p, None)
    M.sync()
    got = fetch_bf16(y, (rows, n))
    alt = (np.arange(rows) % seg) < split
    for r in (0, 19, 20, 114, 115, 134, 135, 229):
        m = mod[1] if alt[r] else mod[0]
        want = R.ln_modulate(x[r:r + 1], m[1], m[0])
        assert np.abs(got[r] - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6


def test_gate_add_tanh_bf16(gpu, rng):
    rows, n = 100, 512
    x = rng.standard_normal((rows, n)).astype(np.float32)
    y = R.bf16_round(rng.standard_normal((rows, n)).astype(np.float32))
    g = rng.standard_normal((2, n)).astype(np.float32)
    xd = dev(x)
    M.call("mk_gate_add", xd.p, bdev(y).p, M.BF16, rows, n, dev(g).p, n, 30, rows, 1, None)
    M.sync()
    want = x + np.tanh(np.where(np.arange(rows)[:, None] < 30, g[1], g[0])) * y
    assert maxrel(fetch(xd, (rows, n)), want) < 1e-6


@pytest.mark.parametrize("d,mode,transpose,odt", [(128, 2, 0, M.BF16), (128, 1, 0, M.BF16), (64, 0, 0, M.BF16),
                                                  (128, 0, 1, M.BF16), (64, 0, 1, M.BF16), (128, 2, 0, M.F16),
                                                  (64, 0, 0, M.F16), (128, 0, 1, M.F16), (64, 0, 1, M.F16)])
def test_heads(gpu, rng, d, mode, transpose, odt):
    B, rows, H = 2, 90, 3
    ld = 3 * H * d
    x = R.bf16_round(rng.standard_normal((B, rows, ld)).astype(np.float32))
    w = None if transpose or d == 64 else (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    cs = R.rope_table(10, 10, 10)
    row0, n_pad = 7, 128
    out = M.Dev(B * H * n_pad * d * 2)
    wd = dev(w) if w is not None else None
    csd = dev(cs)
    M.call("mk_heads", bdev(x).p, B, rows, ld, rows * ld, H * d, H, d, wd.p if wd else None, 1e-6,
           csd.p if mode else None, mode, out.p, n_pad, row0, transpose, odt, None)
    M.sync()
    shape = (B, H, d, n_pad) if transpose else (B, H, n_pad, d)
    got = M.f16_to_f32(out.to_array(np.uint16, shape)) if odt == M.F16 else fetch_bf16(out, shape)
    for bi in range(B):
        want = R.heads_norm_rope(x[bi], H, d, col0=H * d, w=w, cs=cs[row0:] if mode else None, rope=mode)
        if transpose:
            g = got[bi][:, :, M.vt_col(np.arange(row0, row0 + rows))].transpose(0, 2, 1)
        else:
            g = got[bi][:, row0:row0 + rows]
        assert np.abs(g - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("d,odt", [(64, M.BF16), (128, M.BF16), (64, M.F16), (128, M.F16)])
def test_heads_plain_layout_is_an_exact_copy(gpu, rng, d, odt):
    # no norm, no rope: the 16-byte copy path; every value lands bit for bit at [batch][head][row0 + r] (as half: the
    # bf16 value rounded to nearest even, as numpy rounds it)
    B, rows, H, row0, n_pad = 2, 77, 5, 3, 96
    ld = 3 * H * d
    x = M.bf16_bits(rng.standard_normal((B, rows, ld)).astype(np.float32) * 3.0)
    out = M.Dev(B * H * n_pad * d * 2)
    M.call("mk_heads", M.Dev.from_array(x).p, B, rows, ld, rows * ld, H * d, H, d, None, 1e-6, None, 0, out.p, n_pad,
           row0, 0, odt, None)
    M.sync()
    got = out.to_array(np.uint16, (B, H, n_pad, d))[:, :, row0:row0 + rows]
    want = x[:, :, H * d:2 * H * d].reshape(B, rows, H, d).transpose(0, 2, 1, 3)
    if odt == M.F16:
        want = M.f16_bits(M.bf16_to_f32(want))
    assert np.array_equal(got, want)


# one-row kernels for K in {2048, 3072, 4096}; the LDS-staged kernel for the rest and for rows 2..4
@pytest.mark.parametrize("rows,K,silu", [(1, 3072, 1), (1, 2048, 0), (1, 4096, 1), (1, 1024, 1), (2, 3072, 1),
                                         (4, 2048, 0)])
def test_gemv_modulation(gpu, rng, rows, K, silu):
    N = 6 * 3072 + 63  # a ragged last group of outputs
    x = rng.standard_normal((rows, K)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.02)
    b = rng.standard_normal(N).astype(np.float32)
    y = M.Dev(rows * N * 4)
    M.call("mk_gemv", dev(x).p, rows, K, bdev(W).p, dev(b).p, N, y.p, silu, None)
    M.sync()
    want = R.gemm(R.silu(x) if silu else x, W, b)  # x' rounded to bf16 as the GEMMs' activation operand
    assert maxrel(fetch(y, (rows, N)), want) < 1e-5


@pytest.mark.parametrize("n", [12, 260, 640, 1280, 3072, 4096])  # 1, 2, 3, 5, 12 and 16 float4s a lane
def test_norms(gpu, rng, n):
    rows = 70
    x = (rng.standard_normal((rows, n)) * 2 + 0.3).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    y = M.Dev(rows * n * 2)
    M.call("mk_layer_norm", dev(x).p, rows, n, dev(g).p, dev(b).p, 1e-5, y.p, None)
    M.sync()
    want = R.layer_norm(x, g, b, 1e-5)
    assert np.abs(fetch_bf16(y, (rows, n)) - want).max() <= 2 ** -8 * np.abs(want).max()
    M.call("mk_rms_norm", dev(x).p, rows, n, dev(g - 1).p, 1.0, 1e-6, y.p, None)  # zero-centred weight + 1
    M.sync()
    want = R.rms_norm(x, g)
    assert np.abs(fetch_bf16(y, (rows, n)) - want).max() <= 2 ** -8 * np.abs(want).max()
    if n != 1280:
        return
    xg = rng.standard_normal((2, 300, 640)).astype(np.float32)
    gg = (1 + 0.1 * rng.standard_normal(640)).astype(np.float32)
    yg = M.Dev(2 * 300 * 640 * 2)
    M.call("mk_group_norm", dev(xg).p, 2, 300, 640, 32, dev(gg).p, dev(b[:640]).p, 1e-6, yg.p, None)
    M.sync()
    got = fetch_bf16(yg, (2, 300, 640))
    for bi in range(2):
        want = R.group_norm(xg[bi], gg, b[:640], 32, 1e-6)
        assert np.abs(got[bi] - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-5
    # channels not a multiple of 4 (the one-channel-a-thread apply), a partial last chunk of rows
    xs = (rng.standard_normal((2, 37, 90)) * 3 + 1).astype(np.float32)
    gs, bs = (1 + 0.1 * rng.standard_normal(90)).astype(np.float32), (0.1 * rng.standard_normal(90)).astype(np.float32)
    ys = M.Dev(2 * 37 * 90 * 2)
    M.call("mk_group_norm", dev(xs).p, 2, 37, 90, 3, dev(gs).p, dev(bs).p, 1e-6, ys.p, None)
    M.sync()
    got = fetch_bf16(ys, (2, 37, 90))
    for bi in range(2):
        want = R.group_norm(xs[bi], gs, bs, 3, 1e-6)
        assert np.abs(got[bi] - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-5


def test_glu(gpu, rng):
    rows, F = 50, 640
    hg = rng.standard_normal((rows, 2 * F)).astype(np.float32) * 2
    m = M.Dev(rows * F * 2)
    for name, ref in (("mk_swiglu", R.swiglu), ("mk_geglu", R.geglu)):
        M.call(name, dev(hg).p, M.F32, rows, F, m.p, None)
        M.sync()
        want = ref(hg)
        assert np.abs(fetch_bf16(m, (rows, F)) - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6


@pytest.mark.parametrize("F", [640, 100])
def test_glu_bf16_vector_path_equals_scalar_path(gpu, rng, F):
    # bf16 input: 16-byte-aligned buffers with F a multiple of 8 take the 8-wide kernel; the same data 2 bytes off
    # alignment take the element-wise one. Bit-identical, and within bf16 rounding of the oracle.
    rows = 37
    hg = M.bf16_bits(rng.standard_normal((rows, 2 * F)).astype(np.float32) * 2)
    a_in, b_in = M.Dev(hg.nbytes + 16), M.Dev(hg.nbytes + 16)
    a_in.write(hg)
    b_in.write(hg, offset=2)
    a_out, b_out = M.Dev(rows * F * 2 + 16), M.Dev(rows * F * 2 + 16)
    for name, ref in (("mk_swiglu", R.swiglu), ("mk_geglu", R.geglu)):
        M.call(name, a_in.p, M.BF16, rows, F, a_out.p, None)
        M.call(name, int(b_in.p) + 2, M.BF16, rows, F, int(b_out.p) + 2, None)
        M.sync()
        got_a = a_out.to_array(np.uint16, (rows * F + 8,))[:rows * F]
        got_b = b_out.to_array(np.uint16, (rows * F + 8,))[1:rows * F + 1]
        assert np.array_equal(got_a, got_b), name
        want = ref(M.bf16_to_f32(hg))
        got = M.bf16_to_f32(got_a).reshape(rows, F)
        assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6, name


def test_cfg_euler_exact(gpu, rng):
    n = 4096 * 64
    x, pos, neg = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    out = M.Dev(n * 4)
    M.call("mk_cfg_euler", dev(x).p, dev(pos).p, dev(neg).p, n, np.float32(4.0), np.float32(-0.05), out.p, None)
    M.sync()
    v = (neg + np.float32(4.0) * (pos - neg)).astype(np.float32)
    want = (x + np.float32(-0.05) * v).astype(np.float32)
    assert np.abs(fetch(out, (n,)) - want).max() <= 1e-6 * np.abs(want).max()


def test_patchify_bit_exact(gpu, rng):
    B, Cc, h, w = 2, 16, 12, 10
    lat = rng.standard_normal((B, Cc, 2 * h, 2 * w)).astype(np.float32)
    tok = M.Dev(lat.nbytes)
    M.call("mk_patchify", dev(lat).p, B, Cc, h, w, tok.p, None)
    M.sync()
    got = fetch(tok, (B, h * w, 4 * Cc))
    for bi in range(B):
        assert np.array_equal(got[bi], R.patchify(lat[bi], h, w))
    back = M.Dev(lat.nbytes)
    M.call("mk_unpatchify", tok.p, B, Cc, h, w, back.p, None)
    M.sync()
    assert np.array_equal(fetch(back, lat.shape), lat)


@pytest.mark.parametrize("dtype", [M.F32, M.BF16])
def test_fill_normal_matches_oracle_rng(gpu, dtype):
    n = 1 << 20
    key = R.tensor_key(0, "transformer_blocks.3.img_mlp.net.0.proj.weight")
    d = M.Dev(n * 4)
    M.call("mk_fill_normal", d.p, n, dtype, key, 0.0, 0.02, None)
    M.sync()
    want = np.empty(n, np.float32)
    R.lib().mkref_fill_normal(R.fp(want), n, key, 0.0, 0.02, int(dtype == M.BF16))
    got = fetch(d, (n,)) if dtype == M.F32 else fetch_bf16(d, (n,))
    assert np.array_equal(got, want)


def test_quantize_fp8_matches_oracle(gpu):
    m = R.Model(R.DUAL, 1, 256, 2, 128, 512, 256, fp8=True, seed=9)
    name = "transformer_blocks.0.img_mlp.net.0.proj.weight"
    q, scale = m.get(name), m.get(name + ".scale")
    rows, cols = q.shape
    # the same bf16 source the oracle quantised: N(0, 0.02) rounded to bf16
    src = R.normal(rows * cols, 9, name, 0.0, 0.02, round_bf16=True).reshape(rows, cols)
    codes, sc = M.Dev(rows * cols), M.Dev(rows * 4)
    M.call("mk_quantize_fp8_rows", bdev(src).p, rows, cols, codes.p, sc.p, None)
    M.sync()
    assert np.array_equal(fetch(sc, (rows,)), scale)
    assert np.array_equal(R.e4m3_table()[fetch(codes, (rows, cols), np.uint8)], q)


def test_quantize_fp8_every_bf16_value_and_zeros(gpu):
    # Every finite bf16 value of magnitude <= 448 (both zeros included), in rows that start with 448 so the row
    # scale is exactly 1 and each code is the encoder's own rounding of the value; then an all-zero row (scale 1,
    # zero codes: exact zeros once came out as code 0xF8, -256 x the scale).
    v = M.bf16_to_f32(np.arange(0x10000, dtype=np.uint32).astype(np.uint16))
    vals = v[np.isfinite(v) & (np.abs(v) <= 448.0)]
    cols = 512
    rows = -(-vals.size // (cols - 1))
    body = np.zeros(rows * (cols - 1), np.float32)
    body[:vals.size] = vals
    mat = np.concatenate([np.full((rows, 1), 448.0, np.float32), body.reshape(rows, cols - 1)], axis=1)
    mat = np.concatenate([mat, np.zeros((1, cols), np.float32)])
    rows += 1
    codes, sc = M.Dev(rows * cols), M.Dev(rows * 4)
    M.call("mk_quantize_fp8_rows", bdev(mat).p, rows, cols, codes.p, sc.p, None)
    M.sync()
    assert np.array_equal(fetch(sc, (rows,)), np.ones(rows, np.float32))
    enc = R.lib().mkref_f32_to_e4m3
    want = np.array([enc(float(x)) for x in mat.ravel()], dtype=np.uint8).reshape(rows, cols)
    got = fetch(codes, (rows, cols), np.uint8)
    assert np.array_equal(got, want), np.argwhere(got != want)[:8]
    assert not got[-1].any()


@pytest.mark.parametrize("d,H,Hkv,scale", [(128, 8, 2, 0.0), (64, 6, 3, 0.125), (128, 4, 1, 0.0)])
def test_attention_grouped_kv_heads(gpu, rng, d, H, Hkv, scale):
    # grouped-query attention (the reference's AttnArgs kv_heads): query head h reads key / value head h / (H / Hkv);
    # the oracle runs plain attention on K / V repeated to every query head
    B, Tq, Tk = 2, 200, 333
    q = R.bf16_round(rng.standard_normal((B, H, Tq, d)).astype(np.float32))
    k = rng.standard_normal((B, Hkv, Tk, d)).astype(np.float32)
    if scale == 0.0:  # K carries the softmax scale in log2 units: softmax(q K'^T ln 2)
        k = k / np.sqrt(d) * np.log2(np.e)
    k = R.bf16_round(k)
    v = R.bf16_round(rng.standard_normal((B, Hkv, Tk, d)).astype(np.float32))
    got = run_attention(q, k, v, scale)
    rep = H // Hkv
    want = R.attention(q, np.repeat(k, rep, axis=1), np.repeat(v, rep, axis=1),
                       float(np.log(2.0)) if scale == 0.0 else scale)
    dd = R.diff(got, want, d)
    assert dd["min_cos"] > 0.9999 and dd["max_rel"] < 1e-2, dd


def test_attention_rejects_kv_heads_not_dividing(gpu):
    z = dev(np.zeros(4096, np.uint16))
    st = M.lib().mk_attention(z.p, z.p, z.p, z.p, M.BF16, 1, 6, 4, 64, 16, 256, 16, 64, 384, 0, 0, 0, 0.125, None,
                              None)
    assert st == 1 and b"kv_heads" in M.lib().mk_last_error()


def test_binding_keeps_dropped_buffers_until_sync(gpu, rng):
    # the pointer of a temporary Dev passed straight to a call stays valid: dropped buffers are freed only after the
    # next device-wide synchronisation
    x = rng.standard_normal(1 << 16).astype(np.float32)
    out = dev(np.zeros(1 << 16, np.uint16))
    M.call("mk_f32_to_bf16", M.Dev.from_array(x).p, x.size, out.p, None)
    assert len(M._pending) >= 1
    M.sync()
    assert not M._pending
    assert np.array_equal(out.to_array(np.uint16, x.shape), M.bf16_bits(x))


# Gated linear units in the projection's epilogue: W = [first F rows; second F rows] (the fused gate|up matrix),
# C [M][F] = silu(first) second (SwiGLU) or first gelu_erf(second) (GEGLU), from the fp32 accumulators. Shapes that
# take 256-wide tiles (8 waves) and 128-wide ones (4 waves); bf16 and fp8 weights; with and without bias.
@pytest.mark.parametrize("epi,Mr,F,K,w8,bias", [(M.EPI_SWIGLU, 4352, 3072, 512, False, False),
                                                (M.EPI_GEGLU, 2048, 2560, 320, False, True),
                                                (M.EPI_SWIGLU, 300, 640, 256, False, True),
                                                (M.EPI_GEGLU, 77, 192, 128, False, True),
                                                (M.EPI_SWIGLU, 1100, 1536, 384, True, False)])
def test_gemm_glu_epilogue(gpu, rng, epi, Mr, F, K, w8, bias):
    N = 2 * F
    A = rng.standard_normal((Mr, K)).astype(np.float32)
    Wf = rng.standard_normal((N, K)).astype(np.float32) * 0.08
    if w8:
        scale = (np.abs(Wf).max(1) / 448).astype(np.float32)
        table = R.e4m3_table()
        mags, a = table[:127], np.abs(Wf / scale[:, None])
        i = np.clip(np.searchsorted(mags, a), 1, 126)
        codes = np.where(a - mags[i - 1] <= mags[i] - a, i - 1, i).astype(np.uint8) | \
            np.where(Wf < 0, 0x80, 0).astype(np.uint8)
        Wv, Wd, sd = table[codes], dev(codes), dev(scale)
    else:
        Wv, Wd, sd, scale = R.bf16_round(Wf), None, None, None
        Wd = bdev(Wv)
    b = rng.standard_normal(N).astype(np.float32) * 0.3 if bias else None
    out = dev(np.zeros(Mr * F, np.uint16))
    gemm(bdev(A), Wd, bias=dev(b) if bias else None, wscale=sd, c=out, c_dtype=M.BF16, epi=epi, M_=(Mr, N, K),
         lda=K, ldc=F, w_dtype=M.FP8 if w8 else M.BF16)
    y = R.gemm(A, Wv, b, wscale=scale)
    want = R.swiglu(y) if epi == M.EPI_SWIGLU else R.geglu(y)
    got = fetch_bf16(out, (Mr, F))
    assert np.abs(got - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6


def test_gemm_glu_equals_separate_glu_kernel(gpu, rng):
    # the fused epilogue against the two-step form (fp32 GEMM output, then mk_swiglu on it): within one bf16 rounding
    Mr, F, K = 512, 1024, 256
    A, W = bdev(rng.standard_normal((Mr, K)).astype(np.float32)), bdev(rng.standard_normal((2 * F, K)) * 0.05)
    fused = dev(np.zeros(Mr * F, np.uint16))
    gemm(A, W, c=fused, c_dtype=M.BF16, epi=M.EPI_SWIGLU, M_=(Mr, 2 * F, K), lda=K, ldc=F)
    gu, m = M.Dev(Mr * 2 * F * 4), dev(np.zeros(Mr * F, np.uint16))
    _live.append(gu)
    gemm(A, W, c=gu, c_dtype=M.F32, M_=(Mr, 2 * F, K), lda=K, ldc=2 * F)
    M.call("mk_swiglu", gu.p, M.F32, Mr, F, m.p, None)
    M.sync()
    a, b = fetch_bf16(fused, (Mr, F)), fetch_bf16(m, (Mr, F))
    assert np.abs(a - b).max() <= 2 ** -8 * np.abs(b).max()
    assert np.mean(a == b) > 0.95


@pytest.mark.parametrize("d,Tq,Tk,holes,scale", [(128, 300, 300, ((41, 64), (64, 64)), 0.0),
                                                 (128, 300, 700, ((5, 200), (100, 101)), 0.0),
                                                 (64, 120, 333, ((1, 64), (30, 97)), 0.125)])
def test_attention_masked_key_range(gpu, rng, d, Tq, Tk, holes, scale):
    # a guidance batch whose shorter prompt is padded: keys [lo, hi) of each batch item are masked; equal to attention
    # over the remaining keys (ranges inside a tile, across tiles, empty, a single key)
    B, H = 2, 3
    q = R.bf16_round(rng.standard_normal((B, H, Tq, d)).astype(np.float32))
    k = rng.standard_normal((B, H, Tk, d)).astype(np.float32)
    if scale == 0.0:
        k = k / np.sqrt(d) * np.log2(np.e)
    k = R.bf16_round(k)
    v = R.bf16_round(rng.standard_normal((B, H, Tk, d)).astype(np.float32))
    got = run_attention(q, k, v, scale, hole=holes)
    eff = float(np.log(2.0)) if scale == 0.0 else scale
    for b, (lo, hi) in enumerate(holes):
        keep = np.r_[0:lo, hi:Tk]
        want = R.attention(q[b:b + 1], np.ascontiguousarray(k[b:b + 1, :, keep]),
                           np.ascontiguousarray(v[b:b + 1, :, keep]), eff)
        dd = R.diff(got[b], want[0], d)
        assert dd["min_cos"] > 0.9999 and dd["max_rel"] < 1e-2, dd


# Launches of at most one tile a CU on 128-channel tiles run deep-staged (4 LDS stages for 128 x 128 tiles, 3 for
# 256 x 128): K of 1 to 20 k steps covers the prologue, whole unrolled rounds and every remainder length.
@pytest.mark.parametrize("K", [64, 128, 192, 256, 320, 448, 1280])
@pytest.mark.parametrize("Mr,N", [(256, 256), (8192, 640)])  # 4 tiles of 128 x 128; 160 of 256 x 128
def test_gemm_deep_staged_lone_tiles(gpu, rng, Mr, N, K):
    A = rng.standard_normal((Mr, K)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.05)
    b = rng.standard_normal(N).astype(np.float32) * 0.3
    out = dev(np.zeros(Mr * N, np.float32))
    gemm(bdev(A), bdev(W), bias=dev(b), c=out, c_dtype=M.F32, epi=M.EPI_STORE, M_=(Mr, N, K), lda=K, ldc=N)
    got = fetch(out, (Mr, N))
    rows = np.sort(rng.choice(Mr, 96, replace=False))
    rows[0], rows[-1] = 0, Mr - 1
    assert maxrel(got[rows], R.gemm(np.ascontiguousarray(A[rows]), W, b)) < 1e-5


# Launches of few tiles take 128 x 128 tiles (two workgroups a CU): the SDXL stage-B shapes (2 x 1024 tokens, 1280
# channels) and a row count that leaves a partial 128-row tile, each epilogue kind against the oracle. The same
# products through 256-row tiles (a grouped launch with an empty second problem plans the same way, so instead the
# rows are split: rows [0, 1024) and [1024, Mr) as two launches) must give the same bits: a tile's k order does not
# depend on its height.
@pytest.mark.parametrize("Mr,N,K,epi", [(2048, 1280, 1280, M.EPI_ADD), (2048, 1280, 5120, M.EPI_GATE_ADD),
                                        (2000, 3840, 1280, M.EPI_STORE), (2048, 2 * 5120, 1280, M.EPI_GEGLU),
                                        (1900, 1280, 640, M.EPI_GELU_TANH)])
def test_gemm_short_tiles_match_oracle(gpu, rng, Mr, N, K, epi):
    A = rng.standard_normal((Mr, K)).astype(np.float32)
    W = R.bf16_round(rng.standard_normal((N, K)).astype(np.float32) * 0.03)
    b = rng.standard_normal(N).astype(np.float32) * 0.3
    glu = epi == M.EPI_GEGLU
    F = N // 2 if glu else N
    resid = epi in (M.EPI_ADD, M.EPI_GATE_ADD)
    bf16_out = epi in (M.EPI_GEGLU, M.EPI_GELU_TANH)
    X = rng.standard_normal((Mr, F)).astype(np.float32) if resid else None
    gate = rng.standard_normal(N).astype(np.float32) if epi == M.EPI_GATE_ADD else None
    out = dev(X) if resid else dev(np.zeros(Mr * F, np.uint16 if bf16_out else np.float32))
    gemm(bdev(A), bdev(W), bias=dev(b), c=out, c_dtype=M.BF16 if bf16_out else M.F32, epi=epi, M_=(Mr, N, K),
         lda=K, ldc=F, gate=dev(gate) if gate is not None else None)
    got = fetch_bf16(out, (Mr, F)) if bf16_out else fetch(out, (Mr, F))
    rows = np.sort(rng.choice(Mr, 96, replace=False))
    rows[-1] = Mr - 1  # the partial tile's last row
    y = R.gemm(np.ascontiguousarray(A[rows]), W, b)
    if epi == M.EPI_ADD:
        want = X[rows].astype(np.float64) + y
    elif epi == M.EPI_GATE_ADD:
        want = X[rows].astype(np.float64) + gate * y
    elif glu:
        want = R.geglu(y)
    elif epi == M.EPI_GELU_TANH:
        want = R.gelu_tanh(y)
    else:
        want = y
    if bf16_out:
        assert np.abs(got[rows] - want).max() <= 2 ** -8 * np.abs(want).max() + 1e-6
    elif resid:
        assert maxrel(got[rows] - X[rows], want - X[rows]) < 1e-5
    else:
        assert maxrel(got[rows], want) < 1e-5
    # the same rows as two launches of a different plan (1024 rows: 256-row tiles where the whole launch took
    # 128-row ones, or the reverse): bit-identical
    out2 = dev(X) if resid else dev(np.zeros(Mr * F, np.uint16 if bf16_out else np.float32))
    esz = 2 if bf16_out else 4
    for r0, r1 in ((0, 1024), (1024, Mr)):
        g = gemm_args(bdev(A[r0:r1]), bdev(W), bias=dev(b), c=out2, c_dtype=M.BF16 if bf16_out else M.F32, epi=epi,
                      M_=(r1 - r0, N, K), lda=K, ldc=F, gate=dev(gate) if gate is not None else None)
        g.c = out2.p + r0 * F * esz
        M.call("mk_gemm", C.byref(g), None)
    M.sync()
    got2 = fetch_bf16(out2, (Mr, F)) if bf16_out else fetch(out2, (Mr, F))
    assert np.array_equal(got, got2)
