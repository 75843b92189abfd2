"""The binding's operand extent checks (mkimage.call): an undersized A, W, C, convolution grid or attention operand
is refused with MkError before the library is called; operands that fit go through. No GPU: the allocations are
fake address ranges registered with the checks, and the library is a stub that records its calls."""
import ctypes as C

import pytest

import mkimage as M


class StubLib:
    def __init__(self):
        self.calls = []

    def __getattr__(self, name):
        def fn(*args):
            self.calls.append(name)
            return 0
        return fn


@pytest.fixture
def stub(monkeypatch):
    lib = StubLib()
    monkeypatch.setattr(M, "lib", lambda: lib)
    monkeypatch.setattr(M, "STRICT", True)
    regions = []

    def alloc(nbytes):
        base = 0x7f0000000000 + 0x100000000 * (len(regions) + 1)
        M.register(base, nbytes)
        regions.append(base)
        return base

    yield lib, alloc
    for r in regions:
        M.unregister(r)


def gemm_args(a, w, c, Mr, N, K, **kw):
    g = M.GemmArgs()
    g.a, g.w, g.c, g.M, g.N, g.K = a, w, c, Mr, N, K
    g.lda, g.ldc, g.batch, g.w_dtype, g.c_dtype, g.epilogue = K, N, 1, M.BF16, M.F32, M.EPI_STORE
    for k, v in kw.items():
        setattr(g, k, v)
    return g


def test_gemm_operands_that_fit_are_launched(stub):
    lib, alloc = stub
    Mr, N, K = 300, 256, 128
    g = gemm_args(alloc(Mr * K * 2), alloc(N * K * 2), alloc(Mr * N * 4), Mr, N, K)
    M.call("mk_gemm", C.byref(g), None)
    assert lib.calls == ["mk_gemm"]


@pytest.mark.parametrize("short", ["a", "w", "c"])
def test_gemm_undersized_operand_is_refused(stub, short):
    lib, alloc = stub
    Mr, N, K = 300, 256, 128
    need = {"a": Mr * K * 2, "w": N * K * 2, "c": Mr * N * 4}
    ptr = {k: alloc(v - (16 if k == short else 0)) for k, v in need.items()}
    g = gemm_args(ptr["a"], ptr["w"], ptr["c"], Mr, N, K)
    with pytest.raises(M.MkError, match=f": {short.upper()}"):
        M.call("mk_gemm", C.byref(g), None)
    assert lib.calls == []


def test_gemm_batch_stride_and_row_stride_count(stub):
    lib, alloc = stub
    # two batch items 1000 rows apart, ldc 512 for N 256: C spans (1000 + 63) rows of 512 plus 256 floats
    Mr, N, K = 64, 256, 64
    a = alloc((1000 + Mr) * K * 2)
    w = alloc(N * K * 2)
    c = alloc(((1000 + Mr - 1) * 512 + N) * 4 - 4)
    g = gemm_args(a, w, c, Mr, N, K, batch=2, stride_a=1000 * K, stride_c=1000 * 512, ldc=512)
    with pytest.raises(M.MkError, match=": C"):
        M.call("mk_gemm", C.byref(g), None)
    M.register(c, ((1000 + Mr - 1) * 512 + N) * 4)
    M.call("mk_gemm", C.byref(g), None)
    assert lib.calls == ["mk_gemm"]


def test_grouped_gemm_checks_every_problem(stub):
    lib, alloc = stub
    Mr, N, K = 128, 256, 64
    g0 = gemm_args(alloc(Mr * K * 2), alloc(N * K * 2), alloc(Mr * N * 4), Mr, N, K)
    g1 = gemm_args(alloc(Mr * K * 2), alloc(N * K * 2 - 2), alloc(Mr * N * 4), Mr, N, K)
    arr = (M.GemmArgs * 2)(g0, g1)
    with pytest.raises(M.MkError, match=r"mk_gemm_grouped\[1\]: W"):
        M.call("mk_gemm_grouped", C.cast(arr, C.c_void_p), 2, None)
    assert lib.calls == []


def test_fp8_weights_heads_and_glu_extents(stub):
    lib, alloc = stub
    # fp8 weights take one byte an element; a GLU's output has N / 2 columns
    Mr, N, K = 64, 512, 64
    g = gemm_args(alloc(Mr * K * 2), alloc(N * K), alloc(Mr * (N // 2) * 2), Mr, N, K, w_dtype=M.FP8,
                  wscale=alloc(N * 4), epilogue=M.EPI_SWIGLU, c_dtype=M.BF16, ldc=N // 2)
    M.call("mk_gemm", C.byref(g), None)
    # the heads epilogue: Q, K, V^T of batch x heads x pad x 128 halves
    B, H, pad = 2, 2, 256
    ha = M.HeadsArgs(alloc(B * H * pad * 128 * 2), alloc(B * H * pad * 128 * 2), alloc(B * H * pad * 128 * 2 - 2),
                     H, 128, pad, pad, 0, 0, None, None, None, 0, 1e-6, 0.0, M.BF16)
    g = gemm_args(alloc((pad + 100) * K * 2), alloc(3 * H * 128 * K * 2), None, 100, 3 * H * 128, K, batch=B,
                  stride_a=pad * K, epilogue=M.EPI_HEADS, heads=C.pointer(ha))
    with pytest.raises(M.MkError, match="heads vt"):
        M.call("mk_gemm", C.byref(g), None)
    assert lib.calls == ["mk_gemm"]


def test_conv_and_attention_extents(stub):
    lib, alloc = stub
    h, w, c, n = 5, 7, 64, 96
    grid = (h + 2) * (w + 2)
    x = alloc((grid + 2 * (w + 3)) * c * 2)
    a = M.ConvArgs(x, alloc(n * 9 * c * 2), 0, alloc(((grid - 1) * n + n) * 4), h, w, c, n, n, M.F32, M.EPI_STORE)
    M.call("mk_conv3x3", C.byref(a), None)
    a.x = alloc((grid + 2 * (w + 3)) * c * 2 - 64)
    with pytest.raises(M.MkError, match="x"):
        M.call("mk_conv3x3", C.byref(a), None)
    B, H, d, T, pad = 2, 4, 128, 100, 128
    q, k, vt = (alloc(B * H * pad * d * 2) for _ in range(3))
    out = alloc(B * T * H * d * 2 - 2)
    with pytest.raises(M.MkError, match="out"):
        M.call("mk_attention", q, k, vt, out, M.BF16, B, H, H, d, T, pad, T, pad, H * d, T * H * d, 0, 0, 0.0, None,
               None)
    # an operand outside every known allocation
    with pytest.raises(M.MkError, match="not inside"):
        M.call("mk_attention", 0x1000, k, vt, out, M.BF16, B, H, H, d, T, pad, T, pad, H * d, T * H * d, 0, 0, 0.0,
               None, None)
    assert lib.calls == ["mk_conv3x3"]


def test_device_buffer_steps_check_their_extents(stub):
    # the engine and VAE entry points on caller device buffers: mk_step_cfg_device (latents of the begun grid),
    # mk_sdxl_forward ([batch][n][c] fp32 in and out) and mk_vae_decode_device (tokens [h w][4 z], RGBA [16 h][16 w][4])
    lib, alloc = stub
    import numpy as np
    e = M.Engine(M.FAMILY_DUAL, blocks=1, dim=256, heads=2, head_dim=128, ffn=512, text_dim=128)
    e.begin(np.zeros((3, 128), np.float32), 4, 6, 0)
    lat = alloc(4 * 6 * 64 * 4)
    e.step_cfg_device(lat, 0.5, 0.4, 4.0, lat)
    with pytest.raises(M.MkError, match="lat_out"):
        e.step_cfg_device(lat, 0.5, 0.4, 4.0, alloc(4 * 6 * 64 * 4 - 4))
    s = M.Engine(M.FAMILY_SDXL, blocks=1, dim=640, heads=10, head_dim=64, ffn=2560, text_dim=2048)
    x, y = alloc(2 * 100 * 640 * 4), alloc(2 * 100 * 640 * 4)
    s.sdxl_forward(x, 2, 100, y)
    with pytest.raises(M.MkError, match="sdxl_forward: x"):
        s.sdxl_forward(x, 2, 101, y)
    v = M.Vae(16)
    tok, rgba = alloc(3 * 5 * 64 * 4), alloc(48 * 80 * 4 * 4)
    v.decode_device(tok, 3, 5, rgba)
    with pytest.raises(M.MkError, match="rgba"):
        v.decode_device(tok, 3, 5, alloc(48 * 80 * 4 * 4 - 16))
    assert lib.calls.count("mk_step_cfg_device") == 1 and lib.calls.count("mk_sdxl_forward") == 1
    assert lib.calls.count("mk_vae_decode_device") == 1
