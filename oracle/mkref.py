"""ctypes binding of the oracle library (oracle/libmkref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, always
as the reference results or the CPU baseline, never as the product path. The product library (mako-image_amd/libmkimage.so)
does not use it.
"""
from __future__ import annotations

import ctypes as C
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
_lib = None

DUAL, Q21, SDXL = 0, 1, 2


class Dims(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("kind", "blocks", "dim", "heads", "head_dim", "ffn", "text_dim", "latent",
                                           "fp8", "f16")]


PROBE = C.CFUNCTYPE(None, C.c_void_p, C.c_char_p, C.c_int, C.POINTER(C.c_float), C.c_size_t)

_F = C.POINTER(C.c_float)
_I64 = C.c_int64


def lib():
    global _lib
    if _lib is None:
        path = HERE / "libmkref.so"
        if not path.exists():
            raise RuntimeError(f"{path} is not built: run `make -C oracle`")
        L = C.CDLL(str(path))
        L.mkref_f32_to_bf16.restype = C.c_uint16
        L.mkref_f32_to_bf16.argtypes = [C.c_float]
        L.mkref_bf16_to_f32.restype = C.c_float
        L.mkref_bf16_to_f32.argtypes = [C.c_uint16]
        L.mkref_round_bf16.argtypes = [_F, C.c_size_t]
        L.mkref_round_f16.argtypes = [_F, C.c_size_t]
        L.mkref_f32_to_e4m3.restype = C.c_uint8
        L.mkref_f32_to_e4m3.argtypes = [C.c_float]
        L.mkref_e4m3_to_f32.restype = C.c_float
        L.mkref_e4m3_to_f32.argtypes = [C.c_uint8]
        L.mkref_tensor_key.restype = C.c_uint64
        L.mkref_tensor_key.argtypes = [C.c_uint64, C.c_char_p]
        L.mkref_fill_normal.argtypes = [_F, C.c_size_t, C.c_uint64, C.c_double, C.c_double, C.c_int]
        L.mkref_gemm.argtypes = [_F, _I64, _I64, _I64, _F, _I64, _F, _F, _F, _I64]
        L.mkref_ln_modulate.argtypes = [_F, _I64, _I64, _F, _F, C.c_float, _F]
        L.mkref_layer_norm.argtypes = [_F, _I64, _I64, _F, _F, C.c_float, _F]
        L.mkref_rms_norm.argtypes = [_F, _I64, _I64, _F, C.c_float, _F]
        L.mkref_group_norm.argtypes = [_F, _I64, _I64, _I64, _F, _F, C.c_float, _F]
        L.mkref_rope_table.argtypes = [_F, C.c_uint32, C.c_uint32, C.c_uint32]
        L.mkref_heads_norm_rope.argtypes = [_F, _I64, _I64, _I64, _I64, _I64, _F, C.c_float, _F, C.c_int, _F, _I64,
                                            _I64]
        L.mkref_attention.argtypes = [_F, _F, _F, _I64, _I64, _I64, _I64, _I64, C.c_float, C.c_uint32, C.c_uint32,
                                      _F]
        L.mkref_vae_create.restype = C.c_void_p
        L.mkref_vae_create.argtypes = [C.c_uint32, C.c_uint32, C.c_uint64, _F, _F]
        L.mkref_vae_destroy.argtypes = [C.c_void_p]
        L.mkref_vae_count.restype = C.c_size_t
        L.mkref_vae_count.argtypes = [C.c_void_p]
        L.mkref_vae_name.restype = C.c_char_p
        L.mkref_vae_name.argtypes = [C.c_void_p, C.c_size_t]
        L.mkref_vae_tensor.restype = _F
        L.mkref_vae_tensor.argtypes = [C.c_void_p, C.c_size_t, C.POINTER(C.c_uint32), C.POINTER(C.c_int64)]
        L.mkref_vae_decode.argtypes = [C.c_void_p, _F, C.c_uint32, C.c_uint32, _F, C.c_void_p, C.c_void_p]
        L.mkref_gelu_tanh.argtypes = [_F, C.c_size_t]
        L.mkref_silu.argtypes = [_F, C.c_size_t]
        L.mkref_swiglu.argtypes = [_F, _I64, _I64, _F]
        L.mkref_geglu.argtypes = [_F, _I64, _I64, _F]
        L.mkref_sinusoid.argtypes = [C.c_float, C.c_uint32, _F]
        L.mkref_sigmas.argtypes = [C.c_uint32, C.c_uint32, C.c_double, C.c_double, C.c_double, C.c_double,
                                   C.c_double, _F]
        L.mkref_patchify.argtypes = [_F, C.c_uint32, C.c_uint32, C.c_uint32, _F]
        L.mkref_unpatchify.argtypes = [_F, C.c_uint32, C.c_uint32, C.c_uint32, _F]
        L.mkref_model_create.restype = C.c_void_p
        L.mkref_model_create.argtypes = [C.POINTER(Dims), C.c_uint64, C.c_double]
        L.mkref_model_destroy.argtypes = [C.c_void_p]
        L.mkref_model_count.restype = C.c_size_t
        L.mkref_model_count.argtypes = [C.c_void_p]
        L.mkref_model_name.restype = C.c_char_p
        L.mkref_model_name.argtypes = [C.c_void_p, C.c_size_t]
        L.mkref_model_tensor.restype = _F
        L.mkref_model_tensor.argtypes = [C.c_void_p, C.c_size_t, C.POINTER(_I64), C.POINTER(_I64),
                                         C.POINTER(C.c_int)]
        L.mkref_model_find.restype = _I64
        L.mkref_model_find.argtypes = [C.c_void_p, C.c_char_p]
        L.mkref_dual_step.restype = C.c_int
        L.mkref_dual_step.argtypes = [C.c_void_p, _I64, _F, _I64, _F, C.c_uint32, C.c_uint32, C.c_float, _F, PROBE,
                                      C.c_void_p]
        L.mkref_q21_step.restype = C.c_int
        L.mkref_q21_step.argtypes = [C.c_void_p, _F, _I64, _F, C.c_uint32, C.c_uint32, C.c_float, _F, PROBE,
                                     C.c_void_p]
        L.mkref_sdxl_trans.restype = C.c_int
        L.mkref_sdxl_trans.argtypes = [C.c_void_p, _F, _I64, _F, _I64, _F]
        L.mkref_dual_block.restype = C.c_int
        L.mkref_dual_block.argtypes = [C.c_void_p, C.c_int, _F, _I64, _F, _I64, _F, _F, _F]
        L.mkref_threads.restype = C.c_int
        _lib = L
    return _lib


def fp(a):
    """float32 C-contiguous numpy array -> float* (None -> NULL)."""
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- formats ----

def bf16_bits(a):
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16), vectorised (same rule as mkref_f32_to_bf16)."""
    u = f32(a).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_round(a):
    return (bf16_bits(a).astype(np.uint32) << 16).view(np.float32)


def f16_round(a):
    """IEEE half rounding (nearest even) of float32 values, the oracle's rule."""
    x = np.array(a, dtype=np.float32, copy=True, order="C")
    lib().mkref_round_f16(fp(x), x.size)
    return x


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


_E4M3 = None


def e4m3_table():
    global _E4M3
    if _E4M3 is None:
        _E4M3 = np.array([lib().mkref_e4m3_to_f32(i) for i in range(256)], dtype=np.float32)
    return _E4M3


def e4m3_encode(a):
    """Vectorised e4m3 encode of values already exactly representable (weights the oracle quantised)."""
    t = e4m3_table()
    a = f32(a).ravel()
    pos = t[:127]
    idx = np.searchsorted(pos, np.abs(a))
    idx = np.clip(idx, 0, 126)
    codes = idx.astype(np.uint8) | np.where(np.signbit(a), 0x80, 0).astype(np.uint8)
    assert np.array_equal(t[codes], a), "value not representable in e4m3"
    return codes


def tensor_key(seed, name):
    return lib().mkref_tensor_key(seed, name.encode())


def normal(n, seed, name, mean=0.0, std=1.0, round_bf16=False):
    out = np.empty(n, dtype=np.float32)
    lib().mkref_fill_normal(fp(out), n, tensor_key(seed, name), mean, std, int(round_bf16))
    return out


# ---- primitives ----

def gemm(A, W, bias=None, wscale=None):
    A, W = f32(A), f32(W)
    M, K = A.shape
    N = W.shape[0]
    out = np.empty((M, N), dtype=np.float32)
    lib().mkref_gemm(fp(A), K, M, K, fp(W), N, fp(None if wscale is None else f32(wscale)),
                     fp(None if bias is None else f32(bias)), fp(out), N)
    return out


def ln_modulate(x, scale, shift=None, eps=1e-6):
    x = f32(x)
    y = np.empty_like(x)
    lib().mkref_ln_modulate(fp(x), x.shape[0], x.shape[1], fp(None if shift is None else f32(shift)), fp(f32(scale)),
                            eps, fp(y))
    return y


def layer_norm(x, g, b, eps=1e-5):
    x = f32(x)
    y = np.empty_like(x)
    lib().mkref_layer_norm(fp(x), x.shape[0], x.shape[1], fp(f32(g)), fp(f32(b)), eps, fp(y))
    return y


def rms_norm(x, w, eps=1e-6):
    x = f32(x)
    y = np.empty_like(x)
    lib().mkref_rms_norm(fp(x), x.shape[0], x.shape[1], fp(None if w is None else f32(w)), eps, fp(y))
    return y


def group_norm(x, g, b, groups=32, eps=1e-6):
    x = f32(x)
    y = np.empty_like(x)
    lib().mkref_group_norm(fp(x), x.shape[0], x.shape[1], groups, fp(f32(g)), fp(f32(b)), eps, fp(y))
    return y


def rope_table(S, h, w):
    cs = np.empty((S + h * w, 64, 2), dtype=np.float32)
    lib().mkref_rope_table(fp(cs), S, h, w)
    return cs


def heads_norm_rope(x, heads, d, col0=0, w=None, eps=1e-6, cs=None, rope=0, out_rows=None, out_row0=0, out=None):
    x = f32(x)
    rows, ld = x.shape
    out_rows = rows if out_rows is None else out_rows
    if out is None:
        out = np.zeros((heads, out_rows, d), dtype=np.float32)
    lib().mkref_heads_norm_rope(fp(x), rows, ld, col0, heads, d, fp(None if w is None else f32(w)), eps,
                                fp(None if cs is None else f32(cs)), rope, fp(out), out_rows, out_row0)
    return out


def attention(q, k, v, scale, q_pos0=0, block=0):
    """q [B][H][Tq][d], k, v [B][H][Tk][d] -> [B][Tq][H*d]."""
    q, k, v = f32(q), f32(k), f32(v)
    B, H, Tq, d = q.shape
    Tk = k.shape[2]
    out = np.empty((B, Tq, H * d), dtype=np.float32)
    lib().mkref_attention(fp(q), fp(k), fp(v), B, H, Tq, Tk, d, scale, q_pos0, block, fp(out))
    return out


def gelu_tanh(x):
    x = f32(x).copy()
    lib().mkref_gelu_tanh(fp(x), x.size)
    return x


def silu(x):
    x = f32(x).copy()
    lib().mkref_silu(fp(x), x.size)
    return x


def swiglu(gu):
    gu = f32(gu)
    rows, F2 = gu.shape
    m = np.empty((rows, F2 // 2), dtype=np.float32)
    lib().mkref_swiglu(fp(gu), rows, F2 // 2, fp(m))
    return m


def geglu(hg):
    hg = f32(hg)
    rows, F2 = hg.shape
    m = np.empty((rows, F2 // 2), dtype=np.float32)
    lib().mkref_geglu(fp(hg), rows, F2 // 2, fp(m))
    return m


def sinusoid(v, dim=256):
    out = np.empty(dim, dtype=np.float32)
    lib().mkref_sinusoid(v, dim, fp(out))
    return out


def sigmas(steps, tokens, base_seq=256, max_seq=4096, base_shift=0.5, max_shift=1.15, terminal=0.0):
    out = np.empty(steps + 1, dtype=np.float32)
    lib().mkref_sigmas(steps, tokens, base_seq, max_seq, base_shift, max_shift, terminal, fp(out))
    return out


_MASK64 = (1 << 64) - 1


def mt19937_64(seed):
    """std::mt19937_64 (the C++ standard's [rand.predef] parameters: w 64, n 312, m 156, r 31, a 0xB5026F5AA96619E9,
    u 29 d 0x5555555555555555, s 17 b 0x71D67FFFEDA60000, t 37 c 0xFFF7EEE000000000, l 43, f 6364136223846793005):
    a generator of its outputs, pure Python."""
    n, m = 312, 156
    mt = [seed & _MASK64]
    for i in range(1, n):
        mt.append((6364136223846793005 * (mt[-1] ^ (mt[-1] >> 62)) + i) & _MASK64)
    upper, lower = _MASK64 ^ 0x7FFFFFFF, 0x7FFFFFFF
    while True:
        for i in range(n):
            x = (mt[i] & upper) | (mt[(i + 1) % n] & lower)
            xa = (x >> 1) ^ (0xB5026F5AA96619E9 if x & 1 else 0)
            mt[i] = mt[(i + m) % n] ^ xa
        for i in range(n):
            y = mt[i]
            y ^= (y >> 29) & 0x5555555555555555
            y ^= (y << 17) & 0x71D67FFFEDA60000
            y ^= (y << 37) & 0xFFF7EEE000000000
            y ^= y >> 43
            yield y


def _u64_to_f32(v):
    """An unsigned 64-bit integer rounded to the nearest float32 (ties to even), exactly as a C++ conversion does."""
    if v.bit_length() <= 24:
        return np.float32(v)
    sh = v.bit_length() - 24
    mant, rem, half = v >> sh, v & ((1 << sh) - 1), 1 << (sh - 1)
    if rem > half or (rem == half and mant & 1):
        mant += 1
    return np.float32(float(mant) * 2.0 ** sh)


def noise(seed, n):
    """The start noise of Engine::generate (engine.cpp:398-408): n draws of std::normal_distribution<float> over
    std::mt19937_64(seed), as libstdc++ computes them: generate_canonical<float, 24> is one 64-bit draw rounded to
    float over 2^64 (a result of 1 becomes the float below 1), then Marsaglia's polar method: x, y = 2 u - 1
    (float(2) u in float, minus the double 1.0, back to float), r2 = x x + y y in float, redrawn while r2 > 1 or
    r2 == 0, mult = sqrt(-2 logf(r2) / r2); the call returns y mult and keeps x mult for the next call."""
    logf = C.CDLL("libm.so.6").logf
    logf.restype, logf.argtypes = C.c_float, [C.c_float]
    gen = mt19937_64(seed)
    one_below = np.nextafter(np.float32(1), np.float32(0))

    def canonical():
        u = _u64_to_f32(next(gen)) / np.float32(2.0 ** 64)
        return one_below if u >= 1 else u

    out = np.empty(n, np.float32)
    saved = None
    for i in range(n):
        if saved is not None:
            out[i], saved = saved, None
            continue
        while True:
            x = np.float32(float(np.float32(2) * canonical()) - 1.0)
            y = np.float32(float(np.float32(2) * canonical()) - 1.0)
            r2 = x * x + y * y
            if not (r2 > 1.0 or r2 == 0.0):
                break
        mult = np.sqrt(np.float32(-2) * np.float32(logf(r2)) / r2)
        saved = x * mult
        out[i] = y * mult
    return out


def patchify(lat, h, w):
    lat = f32(lat)
    C_ = lat.shape[0]
    out = np.empty((h * w, C_ * 4), dtype=np.float32)
    lib().mkref_patchify(fp(lat), C_, h, w, fp(out))
    return out


def unpatchify(tokens, C_, h, w):
    tokens = f32(tokens)
    out = np.empty((C_, 2 * h, 2 * w), dtype=np.float32)
    lib().mkref_unpatchify(fp(tokens), C_, h, w, fp(out))
    return out


# ---- models ----

class Model:
    """Synthetic weights by name (counter RNG), and the oracle's graphs over them."""

    def __init__(self, kind, blocks, dim, heads, head_dim, ffn, text_dim, latent=64, fp8=False, seed=0, wstd=0.02,
                 f16=False):
        self.dims = Dims(kind, blocks, dim, heads, head_dim, ffn, text_dim, latent, int(bool(fp8)), int(bool(f16)))
        self.seed = seed
        self.h = lib().mkref_model_create(C.byref(self.dims), seed, wstd)
        if not self.h:
            raise ValueError("bad model kind")

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.mkref_model_destroy(self.h)
            self.h = None

    def tensors(self):
        """Yields (name, float32 array [rows][cols] or [rows], kind)."""
        L = lib()
        for i in range(L.mkref_model_count(self.h)):
            rows, cols, kind = _I64(), _I64(), C.c_int()
            p = L.mkref_model_tensor(self.h, i, C.byref(rows), C.byref(cols), C.byref(kind))
            n = rows.value * cols.value
            a = np.ctypeslib.as_array(p, shape=(n,)).copy()
            a = a.reshape(rows.value, cols.value) if kind.value else a
            yield L.mkref_model_name(self.h, i).decode(), a, kind.value

    def get(self, name):
        L = lib()
        i = L.mkref_model_find(self.h, name.encode())
        if i < 0:
            raise KeyError(name)
        rows, cols, kind = _I64(), _I64(), C.c_int()
        p = L.mkref_model_tensor(self.h, i, C.byref(rows), C.byref(cols), C.byref(kind))
        a = np.ctypeslib.as_array(p, shape=(rows.value * cols.value,)).copy()
        return a.reshape(rows.value, cols.value) if kind.value else a

    def _probe(self, probes):
        if probes is None:
            return PROBE(), None

        def cb(_u, name, layer, data, n):
            probes[(name.decode(), layer)] = np.ctypeslib.as_array(data, shape=(n,)).copy()

        return PROBE(cb), None

    def dual_step(self, prompt, latents, h, w, sigma, probes=None):
        prompt, latents = f32(prompt), f32(latents)
        B, S, _ = prompt.shape
        out = np.empty((B, h * w, self.dims.latent), dtype=np.float32)
        cb, _ = self._probe(probes)
        rc = lib().mkref_dual_step(self.h, B, fp(prompt), S, fp(latents), h, w, sigma, fp(out), cb, None)
        if rc:
            raise RuntimeError("mkref_dual_step failed")
        return out

    def q21_step(self, prompt, latents, h, w, sigma, probes=None):
        prompt, latents = f32(prompt), f32(latents)
        S = prompt.shape[0]
        out = np.empty((h * w, self.dims.latent), dtype=np.float32)
        cb, _ = self._probe(probes)
        rc = lib().mkref_q21_step(self.h, fp(prompt), S, fp(latents), h, w, sigma, fp(out), cb, None)
        if rc:
            raise RuntimeError("mkref_q21_step failed")
        return out

    def sdxl_trans(self, x, ctx):
        x, ctx = f32(x), f32(ctx)
        y = np.empty_like(x)
        rc = lib().mkref_sdxl_trans(self.h, fp(x), x.shape[0], fp(ctx), ctx.shape[0], fp(y))
        if rc:
            raise RuntimeError("mkref_sdxl_trans failed")
        return y

    def dual_block(self, block, img, txt, mod_img, mod_txt, cs):
        rc = lib().mkref_dual_block(self.h, block, fp(img), img.shape[0], fp(txt), txt.shape[0], fp(f32(mod_img)),
                                    fp(f32(mod_txt)), fp(f32(cs)))
        if rc:
            raise RuntimeError("mkref_dual_block failed")


class Vae:
    """The VAE decoder (src/image/engine.cpp:862-954) with counter-RNG weights by checkpoint name."""

    def __init__(self, base, z=16, seed=0, mean=None, std=None):
        self.base, self.z = base, z
        self.mean = f32(np.zeros(z) if mean is None else mean)
        self.std = f32(np.ones(z) if std is None else std)
        self.h = lib().mkref_vae_create(base, z, seed, fp(self.mean), fp(self.std))
        if not self.h:
            raise ValueError("bad VAE configuration")

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.mkref_vae_destroy(self.h)
            self.h = None

    def tensors(self):
        """Yields (name, float32 array in PyTorch layout)."""
        L = lib()
        for i in range(L.mkref_vae_count(self.h)):
            nd, dims = C.c_uint32(), (C.c_int64 * 4)()
            p = L.mkref_vae_tensor(self.h, i, C.byref(nd), dims)
            shape = tuple(dims[k] for k in range(nd.value))
            yield L.mkref_vae_name(self.h, i).decode(), np.ctypeslib.as_array(p, shape=(int(np.prod(shape)),)).copy(
            ).reshape(shape)

    def decode(self, tokens, h, w, probes=None):
        tokens = f32(tokens)
        out = np.empty((16 * h, 16 * w, 4), dtype=np.float32)
        cb = None
        if probes is not None:
            def _cb(_u, name, layer, data, n):
                probes[(name.decode(), layer)] = np.ctypeslib.as_array(data, shape=(n,)).copy()
            cb = PROBE(_cb)
        rc = lib().mkref_vae_decode(self.h, fp(tokens), h, w, fp(out), C.cast(cb, C.c_void_p) if cb else None, None)
        if rc:
            raise RuntimeError("mkref_vae_decode failed")
        return out


def diff(got, want, width):
    """The reference's Diff (tests/image_ref_test.cpp:55-78): relative RMS error and the lowest row cosine; plus
    cosine over everything and max-rel = max|g - w| / max|w|."""
    g = np.asarray(got, dtype=np.float64).reshape(-1, width)
    w_ = np.asarray(want, dtype=np.float64).reshape(-1, width)
    rel = float(np.sqrt(((g - w_) ** 2).sum() / (w_ ** 2).sum()))
    cos_rows = (g * w_).sum(1) / np.sqrt((g * g).sum(1) * (w_ * w_).sum(1))
    cos = float((g * w_).sum() / np.sqrt((g * g).sum() * (w_ * w_).sum()))
    max_rel = float(np.abs(g - w_).max() / np.abs(w_).max())
    return {"rel": rel, "min_cos": float(cos_rows.min()), "cos": cos, "max_rel": max_rel}
