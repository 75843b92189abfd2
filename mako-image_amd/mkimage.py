"""ctypes binding of libmkimage.so, the C ABI of include/mkimage.h.

Device memory, streams and events come from the library itself, so a process needs no other GPU runtime. The
library must be built (`make -C mako-image_amd`); nothing here falls back to a CPU path.
"""
from __future__ import annotations

import bisect
import ctypes as C
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "libmkimage.so"

F32, BF16, FP8, F16, DTYPE_OTHER = 0, 1, 2, 3, 255
EPI_STORE, EPI_GELU_TANH, EPI_GATE_ADD, EPI_GATE_TANH, EPI_SILU, EPI_ADD, EPI_HEADS, EPI_SWIGLU, EPI_GEGLU, \
    EPI_PAIR_SUM = range(10)
FAMILY_DUAL, FAMILY_Q21, FAMILY_SDXL = 0, 1, 2

_vp, _sz, _u32, _u64, _i64, _f, _d, _i = (C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint64, C.c_int64, C.c_float,
                                          C.c_double, C.c_int)
_fp = C.POINTER(C.c_float)


class MkError(RuntimeError):
    pass


class HeadsArgs(C.Structure):
    _fields_ = [("q", _vp), ("k", _vp), ("vt", _vp), ("heads", _u32), ("head_dim", _u32), ("q_pad", _u32),
                ("k_pad", _u32), ("row0", _u32), ("q_row0", _u32), ("norm_q", _vp), ("norm_k", _vp), ("rope", _vp),
                ("rope_mode", _u32), ("eps", _f), ("k_scale", _f), ("dtype", _u32), ("rope_stride", _i64)]


class GemmArgs(C.Structure):
    _fields_ = [("a", _vp), ("w", _vp), ("wscale", _vp), ("bias", _vp), ("c", _vp), ("gate", _vp),
                ("gate_alt", _i64), ("split", _u32), ("seg_rows", _u32), ("M", _u32), ("N", _u32), ("K", _u32),
                ("lda", _i64), ("ldc", _i64), ("stride_a", _i64), ("stride_c", _i64), ("batch", _u32),
                ("w_dtype", _u32), ("c_dtype", _u32), ("epilogue", _u32), ("heads", C.POINTER(HeadsArgs))]


class Config(C.Structure):
    _fields_ = [(n, _u32) for n in ("family", "blocks", "dim", "heads", "head_dim", "ffn", "text_dim", "latent",
                                     "weight_dtype", "max_batch")]


class Schedule(C.Structure):
    _fields_ = [("base_seq", _d), ("max_seq", _d), ("base_shift", _d), ("max_shift", _d), ("terminal", _d),
                ("has_mu", _i), ("mu", _d)]


class StTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype_name", C.c_char_p), ("dtype", _u32), ("ndim", _u32),
                ("dims", _u64 * 8), ("file", _u32), ("offset", _u64), ("bytes", _u64)]


class ConvArgs(C.Structure):
    _fields_ = [("x", _vp), ("w", _vp), ("bias", _vp), ("y", _vp), ("h", _u32), ("width", _u32), ("c", _u32),
                ("n", _u32), ("ldy", _i64), ("y_dtype", _u32), ("epilogue", _u32)]


class VaeConfig(C.Structure):
    _fields_ = [("base", _u32), ("z", _u32), ("mean", _fp), ("std", _fp)]


PROBE = C.CFUNCTYPE(None, _vp, C.c_char_p, _i, _fp, _sz)

_SIGS = {
    "mk_last_error": (C.c_char_p, []),
    "mk_version": (C.c_char_p, []),
    "mk_device_count": (_i, [C.POINTER(_i)]),
    "mk_set_device": (_i, [_i]),
    "mk_device_info": (_i, [_i, C.c_char_p, _sz, C.POINTER(_i), C.POINTER(_i), C.c_char_p, _sz]),
    "mk_malloc": (_i, [C.POINTER(_vp), _sz]),
    "mk_free": (_i, [_vp]),
    "mk_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "mk_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "mk_memset": (_i, [_vp, _i, _sz]),
    "mk_synchronize": (_i, []),
    "mk_stream_create": (_i, [C.POINTER(_vp)]),
    "mk_stream_destroy": (_i, [_vp]),
    "mk_stream_synchronize": (_i, [_vp]),
    "mk_event_create": (_i, [C.POINTER(_vp)]),
    "mk_event_destroy": (_i, [_vp]),
    "mk_event_record": (_i, [_vp, _vp]),
    "mk_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(_f)]),
    "mk_gemm": (_i, [C.POINTER(GemmArgs), _vp]),
    "mk_gemm_grouped": (_i, [_vp, _u32, _vp]),
    "mk_gemm_set_wait_limit": (_i, [_u32]),
    "mk_gemv": (_i, [_vp, _u32, _u32, _vp, _vp, _u32, _vp, _i, _vp]),
    "mk_ln_modulate": (_i, [_vp, _u32, _u32, _vp, _vp, _i64, _u32, _u32, _f, _vp, _vp]),
    "mk_gate_add": (_i, [_vp, _vp, _u32, _u32, _u32, _vp, _i64, _u32, _u32, _i, _vp]),
    "mk_heads": (_i, [_vp, _u32, _u32, _i64, _i64, _u32, _u32, _u32, _vp, _f, _vp, _u32, _vp, _u32, _u32, _i, _u32,
                      _vp]),
    "mk_attention": (_i, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _i64, _i64, _u32,
                          _u32, _f, _vp, _vp]),
    "mk_silu": (_i, [_vp, _sz, _vp]),
    "mk_gelu_tanh": (_i, [_vp, _sz, _vp]),
    "mk_swiglu": (_i, [_vp, _u32, _u32, _u32, _vp, _vp]),
    "mk_geglu": (_i, [_vp, _u32, _u32, _u32, _vp, _vp]),
    "mk_rms_norm": (_i, [_vp, _u32, _u32, _vp, _f, _f, _vp, _vp]),
    "mk_layer_norm": (_i, [_vp, _u32, _u32, _vp, _vp, _f, _vp, _vp]),
    "mk_group_norm": (_i, [_vp, _u32, _u32, _u32, _u32, _vp, _vp, _f, _vp, _vp]),
    "mk_group_norm_noalloc": (_i, [_vp, _u32, _u32, _u32, _u32, _vp, _vp, _f, _vp, _vp]),
    "mk_cfg_euler": (_i, [_vp, _vp, _vp, _sz, _f, _f, _vp, _vp]),
    "mk_rope_table": (_i, [_u32, _u32, _u32, _vp]),
    "mk_patchify": (_i, [_vp, _u32, _u32, _u32, _u32, _vp, _vp]),
    "mk_unpatchify": (_i, [_vp, _u32, _u32, _u32, _u32, _vp, _vp]),
    "mk_fill_normal": (_i, [_vp, _sz, _u32, _u64, _d, _d, _vp]),
    "mk_tensor_key": (_u64, [_u64, C.c_char_p]),
    "mk_quantize_fp8_rows": (_i, [_vp, _u64, _u64, _vp, _vp, _vp]),
    "mk_f32_to_bf16": (_i, [_vp, _sz, _vp, _vp]),
    "mk_bf16_to_f32": (_i, [_vp, _sz, _vp, _vp]),
    "mk_engine_create": (_i, [C.POINTER(Config), C.POINTER(_vp)]),
    "mk_engine_destroy": (_i, [_vp]),
    "mk_engine_load": (_i, [_vp, C.c_char_p, _vp, _u32, _u64, _u64]),
    "mk_engine_init_random": (_i, [_vp, _u64]),
    "mk_engine_weight_bytes": (_i, [_vp, C.POINTER(_u64)]),
    "mk_begin": (_i, [_vp, _vp, _sz, _u32, _u32, _u32]),
    "mk_step": (_i, [_vp, _vp, _sz, _f, _u32, _vp]),
    "mk_step_cfg": (_i, [_vp, _vp, _sz, _f, _f, _f, _vp]),
    "mk_step_cfg_device": (_i, [_vp, _vp, _f, _f, _f, _vp, _vp]),
    "mk_engine_stream": (_i, [_vp, C.POINTER(_vp)]),
    "mk_noise": (_i, [_u64, _vp, _sz]),
    "mk_sigmas": (_i, [_u32, _u32, C.POINTER(Schedule), _vp]),
    "mk_generate": (_i, [_vp, _vp, _sz, _vp, _u32, _f, _vp]),
    "mk_engine_set_probe": (_i, [_vp, PROBE, _vp]),
    "mk_engine_set_timing": (_i, [_vp, _i]),
    "mk_engine_timing": (_i, [_vp, _u32, C.POINTER(C.c_char_p), C.POINTER(_f), C.POINTER(_u32), C.POINTER(_d)]),
    "mk_sdxl_forward": (_i, [_vp, _vp, _u32, _u32, _vp, _vp]),
    "mk_lora_merge": (_i, [_vp, _u32, _vp, _u64, _u64, _vp, _vp, _u32, _f, _vp]),
    "mk_st_open": (_i, [C.c_char_p, C.POINTER(_vp)]),
    "mk_st_close": (_i, [_vp]),
    "mk_st_count": (_i, [_vp, C.POINTER(_sz), C.POINTER(_u32)]),
    "mk_st_file_path": (C.c_char_p, [_vp, _u32]),
    "mk_st_at": (_i, [_vp, _sz, C.POINTER(StTensor)]),
    "mk_st_find": (_i, [_vp, C.c_char_p, C.POINTER(StTensor)]),
    "mk_st_read": (_i, [_vp, C.c_char_p, _vp, _sz]),
    "mk_engine_load_safetensors": (_i, [_vp, C.c_char_p, C.POINTER(_u64)]),
    "mk_engine_load_safetensors_at": (_i, [_vp, C.c_char_p, C.c_char_p, C.POINTER(_u64)]),
    "mk_engine_add_lora": (_i, [_vp, C.c_char_p, _f, C.POINTER(_u64), C.POINTER(_u64)]),
    "mk_engine_tensor_count": (_i, [_vp, C.POINTER(_sz)]),
    "mk_engine_tensor_at": (_i, [_vp, _sz, C.POINTER(C.c_char_p), C.POINTER(_u32), C.POINTER(_u64),
                                 C.POINTER(_u64)]),
    "mk_engine_fetch": (_i, [_vp, C.c_char_p, _vp, _sz]),
    "mk_conv3x3": (_i, [C.POINTER(ConvArgs), _vp]),
    "mk_vae_create": (_i, [C.POINTER(VaeConfig), C.POINTER(_vp)]),
    "mk_vae_destroy": (_i, [_vp]),
    "mk_vae_load": (_i, [_vp, C.c_char_p, _vp, C.POINTER(_i64), _u32]),
    "mk_vae_load_safetensors": (_i, [_vp, C.c_char_p, C.POINTER(_u64)]),
    "mk_vae_init_random": (_i, [_vp, _u64]),
    "mk_vae_decode": (_i, [_vp, _vp, _sz, _u32, _u32, _vp]),
    "mk_vae_decode_device": (_i, [_vp, _vp, _u32, _u32, _vp]),
    "mk_vae_stream": (_i, [_vp, C.POINTER(_vp)]),
    "mk_vae_set_probe": (_i, [_vp, PROBE, _vp]),
}

EXPORTS = tuple(_SIGS)
_lib = None


def lib():
    """The loaded library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise MkError(f"{LIB_PATH} is not built: run `make -C mako-image_amd` (or __graft_entry__.build())")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status, what=""):
    if status != 0:
        raise MkError(f"{what}: status {status}: {lib().mk_last_error().decode()}")


def call(name, *args):
    chk = _EXTENT_CHECKS.get(name)
    if chk is not None:
        chk(*args)
    check(getattr(lib(), name)(*args), name)


# ---------------------------------------------------------------------------------------------------------------
# device memory
# ---------------------------------------------------------------------------------------------------------------

_NP = {F32: np.float32, BF16: np.uint16, FP8: np.uint8, F16: np.uint16}


# Device memory of dropped Dev objects: freed only after a device-wide synchronisation, so a pointer taken from a
# temporary (`Dev.from_array(x).p` passed to a call) stays valid for every kernel queued before the object went away.
_pending = []
_pending_bytes = 0
_pending_status = 0
_PENDING_LIMIT = 1 << 30


def _free_pending():
    global _pending_bytes
    while _pending:
        _lib.mk_free(_pending.pop())
    _pending_bytes = 0


def _release(p, nbytes):
    global _pending_bytes, _pending_status
    unregister(p)
    _pending.append(p)
    _pending_bytes += nbytes
    if _pending_bytes >= _PENDING_LIMIT:
        # a finaliser cannot raise: a failed synchronisation is kept for the next sync() to report
        st = _lib.mk_synchronize()
        if st != 0 and not _pending_status:
            _pending_status = st
        if st == 0:
            _free_pending()


# ---------------------------------------------------------------------------------------------------------------
# operand extents: call() checks every device operand of a GEMM, convolution or attention launch against the
# allocation it points into before the launch, so an undersized buffer is refused (MkError) instead of overrun
# ---------------------------------------------------------------------------------------------------------------

_starts = []      # sorted start addresses of the known allocations
_extent = {}      # start -> bytes
STRICT = False    # True: an operand outside every known allocation is refused as well (the tests set it)


def register(p, nbytes):
    """Makes device memory not allocated through Dev (e.g. another library's tensor) known to the checks."""
    p, nbytes = int(p), int(nbytes)
    if p not in _extent:
        bisect.insort(_starts, p)
    _extent[p] = nbytes


def unregister(p):
    p = int(p)
    if _extent.pop(p, None) is not None:
        del _starts[bisect.bisect_left(_starts, p)]


def check_extent(p, nbytes, what):
    """Raises MkError unless bytes [p, p + nbytes) lie inside one known allocation (p None/0 or nbytes <= 0: nothing
    to check; an unknown p passes unless STRICT)."""
    if not p or nbytes <= 0:
        return
    p = int(p)
    i = bisect.bisect_right(_starts, p) - 1
    if i < 0 or p >= _starts[i] + _extent[_starts[i]]:
        if STRICT:
            raise MkError(f"{what}: {p:#x} is not inside any known device allocation")
        return
    end = _starts[i] + _extent[_starts[i]]
    if p + nbytes > end:
        raise MkError(f"{what}: needs {nbytes} bytes from {p:#x}, its allocation holds {end - p}")


def _struct(arg, cls):
    """The structure a byref() / pointer() / address argument points at."""
    if isinstance(arg, cls):
        return arg
    obj = getattr(arg, "_obj", None)   # C.byref(x)
    if isinstance(obj, cls):
        return obj
    if hasattr(arg, "contents"):       # C.pointer(x)
        return arg.contents
    addr = arg.value if isinstance(arg, C.c_void_p) else int(arg)
    return cls.from_address(addr)


def gemm_extents(g, what="mk_gemm"):
    """The bytes each operand of one mk_gemm_args problem spans, checked (include/mkimage.h)."""
    if g.M == 0 or g.N == 0:
        return
    b = max(int(g.batch), 1)
    glu = g.epilogue in (EPI_SWIGLU, EPI_GEGLU, EPI_PAIR_SUM)
    check_extent(g.a, ((b - 1) * g.stride_a + (g.M - 1) * g.lda + g.K) * 2, what + ": A")
    check_extent(g.w, g.N * g.K * (1 if g.w_dtype == FP8 else 2), what + ": W")
    check_extent(g.wscale, g.N * 4, what + ": wscale")
    check_extent(g.bias, g.N * 4, what + ": bias")
    if g.epilogue in (EPI_GATE_ADD, EPI_GATE_TANH):
        check_extent(g.gate, (g.N + (max(int(g.gate_alt), 0) if g.split else 0)) * 4, what + ": gate")
    if g.epilogue == EPI_HEADS:
        if not g.heads:
            return
        h = g.heads.contents
        d = h.head_dim
        check_extent(h.q, b * h.heads * h.q_pad * d * 2, what + ": heads q")
        check_extent(h.k, b * h.heads * h.k_pad * d * 2, what + ": heads k")
        check_extent(h.vt, b * h.heads * d * h.k_pad * 2, what + ": heads vt")
        check_extent(h.norm_q, d * 4, what + ": norm_q")
        check_extent(h.norm_k, d * 4, what + ": norm_k")
        if h.rope_mode:
            check_extent(h.rope, ((b - 1) * h.rope_stride + (h.row0 + g.M) * 128) * 4, what + ": rope")
    else:
        cols = g.N // 2 if glu else g.N
        check_extent(g.c, ((b - 1) * g.stride_c + (g.M - 1) * g.ldc + cols) * (4 if g.c_dtype == F32 else 2),
                     what + ": C")


def _check_gemm(args, stream=None):
    gemm_extents(_struct(args, GemmArgs))


def _check_gemm_grouped(args, count, stream=None):
    addr = args.value if isinstance(args, C.c_void_p) else int(C.cast(args, C.c_void_p).value)
    for i, g in enumerate((GemmArgs * int(count)).from_address(addr)):
        gemm_extents(g, f"mk_gemm_grouped[{i}]")


def _check_conv(args, stream=None):
    a = _struct(args, ConvArgs)
    grid = (a.h + 2) * (a.width + 2)
    check_extent(a.x, (grid + 2 * (a.width + 3)) * a.c * 2, "mk_conv3x3: x (padded grid with slack rows)")
    check_extent(a.w, a.n * 9 * a.c * 2, "mk_conv3x3: w")
    check_extent(a.bias, a.n * 4, "mk_conv3x3: bias")
    check_extent(a.y, ((grid - 1) * a.ldy + a.n) * (4 if a.y_dtype == F32 else 2), "mk_conv3x3: y")


def _check_attention(q, k, vt, out, dtype, batch, heads, kv_heads, d, n_q, q_pad, n_k, k_pad, ldo, stride_o, *rest):
    check_extent(q, batch * heads * q_pad * d * 2, "mk_attention: q")
    check_extent(k, batch * kv_heads * k_pad * d * 2, "mk_attention: k")
    check_extent(vt, batch * kv_heads * d * k_pad * 2, "mk_attention: vt")
    if n_q:
        check_extent(out, ((batch - 1) * stride_o + (n_q - 1) * ldo + heads * d) * 2, "mk_attention: out")


_EXTENT_CHECKS = {"mk_gemm": _check_gemm, "mk_gemm_grouped": _check_gemm_grouped, "mk_conv3x3": _check_conv,
                  "mk_attention": _check_attention}


class Dev:
    """A device allocation (zero-filled). Dropping the object releases it after the next device-wide
    synchronisation (sync()), never before work already queued on it has run."""

    def __init__(self, nbytes):
        p = _vp()
        call("mk_malloc", C.byref(p), max(int(nbytes), 16))
        self.p = p.value
        self.nbytes = int(nbytes)
        register(self.p, self.nbytes)

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        call("mk_memcpy_h2d", d.p, a.ctypes.data, a.nbytes)
        return d

    def to_array(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        call("mk_memcpy_d2h", out.ctypes.data, self.p, out.nbytes)
        return out

    def write(self, a, offset=0):
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        call("mk_memcpy_h2d", self.p + offset, a.ctypes.data, a.nbytes)

    def __del__(self):
        if getattr(self, "p", None) and _lib is not None:
            _release(self.p, self.nbytes)
            self.p = None

    def __int__(self):
        return self.p


def sync():
    """Waits for all device work, then frees the memory of dropped Dev objects."""
    global _pending_status
    call("mk_synchronize")
    _free_pending()
    if _pending_status:
        st, _pending_status = _pending_status, 0
        check(st, "mk_synchronize (from a release)")


def device_info(dev=0):
    name = C.create_string_buffer(256)
    arch = C.create_string_buffer(256)
    cus, clk = _i(), _i()
    call("mk_device_info", dev, name, 256, C.byref(cus), C.byref(clk), arch, 256)
    return {"name": name.value.decode(), "arch": arch.value.decode(), "cus": cus.value, "clock_khz": clk.value}


def device_count():
    n = _i()
    check(lib().mk_device_count(C.byref(n)), "mk_device_count")
    return n.value


class Event:
    def __init__(self):
        p = _vp()
        call("mk_event_create", C.byref(p))
        self.p = p.value

    def record(self, stream=None):
        call("mk_event_record", self.p, stream)

    def elapsed_ms(self, end):
        ms = _f()
        call("mk_event_elapsed_ms", self.p, end.p, C.byref(ms))
        return ms.value

    def __del__(self):
        if getattr(self, "p", None) and _lib is not None:
            _lib.mk_event_destroy(self.p)


# ---------------------------------------------------------------------------------------------------------------
# engine
# ---------------------------------------------------------------------------------------------------------------

def vt_col(k):
    """Column of key k in a V^T buffer (MK_VT_COL): bits 2 and 3 of the key swapped within groups of 16."""
    k = np.asarray(k)
    return (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1)


def bf16_bits(a):
    """float32 -> bf16 bit patterns, round to nearest even (the library's rule)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits(a):
    """float32 -> IEEE half bit patterns, round to nearest even."""
    return np.ascontiguousarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(b):
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


class SafeTensors:
    """A safetensors file or shard directory through the library's reader (host only, no device needed)."""

    def __init__(self, path):
        p = _vp()
        call("mk_st_open", str(path).encode(), C.byref(p))
        self.h = p.value

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.mk_st_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __len__(self):
        n = _sz()
        call("mk_st_count", self.h, C.byref(n), None)
        return n.value

    def files(self):
        f = _u32()
        call("mk_st_count", self.h, None, C.byref(f))
        return [lib().mk_st_file_path(self.h, i).decode() for i in range(f.value)]

    @staticmethod
    def _info(t):
        return {"name": t.name.decode(), "dtype": t.dtype, "dtype_name": t.dtype_name.decode(),
                "dims": [t.dims[i] for i in range(t.ndim)], "file": t.file, "offset": t.offset, "bytes": t.bytes}

    def tensors(self):
        out = []
        for i in range(len(self)):
            t = StTensor()
            call("mk_st_at", self.h, i, C.byref(t))
            out.append(self._info(t))
        return out

    def find(self, name):
        t = StTensor()
        call("mk_st_find", self.h, name.encode(), C.byref(t))
        return self._info(t)

    def read(self, name):
        """The tensor's raw bytes."""
        info = self.find(name)
        buf = np.empty(info["bytes"], dtype=np.uint8)
        call("mk_st_read", self.h, name.encode(), buf.ctypes.data, buf.nbytes)
        return buf


class Vae:
    """The VAE decoder (mk_vae_*): tokens [h * w][4 z] -> RGBA [16 h][16 w][4]."""

    def __init__(self, base=96, z=16, mean=None, std=None):
        self.z = z
        self._mean = np.ascontiguousarray(np.zeros(z) if mean is None else mean, dtype=np.float32)
        self._std = np.ascontiguousarray(np.ones(z) if std is None else std, dtype=np.float32)
        if self._mean.size != z or self._std.size != z:
            raise MkError(f"vae: mean and std need {z} values each (one a latent channel)")
        cfg = VaeConfig(base, z, self._mean.ctypes.data_as(_fp), self._std.ctypes.data_as(_fp))
        p = _vp()
        call("mk_vae_create", C.byref(cfg), C.byref(p))
        self.h = p.value
        self._probe_cb = None

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.mk_vae_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def init_random(self, seed):
        call("mk_vae_init_random", self.h, seed)

    def load(self, name, array):
        a = np.ascontiguousarray(array, dtype=np.float32)
        dims = (_i64 * max(a.ndim, 1))(*a.shape)
        call("mk_vae_load", self.h, name.encode(), a.ctypes.data, dims, a.ndim)

    def load_safetensors(self, path):
        n = _u64()
        call("mk_vae_load_safetensors", self.h, str(path).encode(), C.byref(n))
        return n.value

    def decode(self, tokens, h, w):
        t = np.ascontiguousarray(tokens, dtype=np.float32)
        out = np.empty((16 * h, 16 * w, 4), dtype=np.float32)
        call("mk_vae_decode", self.h, t.ctypes.data, t.size, h, w, out.ctypes.data)
        return out

    def decode_device(self, tokens_dev, h, w, rgba_dev):
        check_extent(tokens_dev, int(h) * int(w) * 4 * self.z * 4, "mk_vae_decode_device: tokens")
        check_extent(rgba_dev, 16 * int(h) * 16 * int(w) * 4 * 4, "mk_vae_decode_device: rgba")
        call("mk_vae_decode_device", self.h, int(tokens_dev), h, w, int(rgba_dev))

    def stream(self):
        s = _vp()
        call("mk_vae_stream", self.h, C.byref(s))
        return s.value

    def set_probe(self, probes):
        if probes is None:
            self._probe_cb = None
            call("mk_vae_set_probe", self.h, PROBE(), None)
            return

        def cb(_u, name, layer, data, n):
            probes[(name.decode(), layer)] = np.ctypeslib.as_array(data, shape=(n,)).copy()

        self._probe_cb = PROBE(cb)
        call("mk_vae_set_probe", self.h, self._probe_cb, None)


class Engine:
    def __init__(self, family, blocks, dim, heads, head_dim, ffn, text_dim, latent=64, weight_dtype=BF16,
                 max_batch=2):
        self.cfg = Config(family, blocks, dim, heads, head_dim, ffn, text_dim, latent, weight_dtype, max_batch)
        p = _vp()
        call("mk_engine_create", C.byref(self.cfg), C.byref(p))
        self.h = p.value
        self._probe_cb = None
        self._grid = None  # (h, w) of the last begin: the latent extent of the device-buffer steps

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.mk_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def load(self, name, array, dtype):
        a = np.ascontiguousarray(array, dtype=_NP[dtype])
        rows = a.shape[0] if a.ndim else 1
        cols = a.size // max(rows, 1)
        call("mk_engine_load", self.h, name.encode(), a.ctypes.data, dtype, rows, cols)

    def init_random(self, seed):
        call("mk_engine_init_random", self.h, seed)

    def load_safetensors(self, path, prefix=None):
        """Every weight from a safetensors file or shard directory; returns the number of tensors read. `prefix`: the
        names are looked up under it first (an SDXL spatial transformer's path inside a UNet checkpoint)."""
        n = _u64()
        if prefix:
            call("mk_engine_load_safetensors_at", self.h, str(path).encode(), prefix.encode(), C.byref(n))
        else:
            call("mk_engine_load_safetensors", self.h, str(path).encode(), C.byref(n))
        return n.value

    def add_lora(self, path, scale=1.0):
        """Merges a LoRA file into the weights; returns (modules merged, modules skipped)."""
        m, k = _u64(), _u64()
        call("mk_engine_add_lora", self.h, str(path).encode(), scale, C.byref(m), C.byref(k))
        return m.value, k.value

    def tensors(self):
        """[(name, dtype, rows, cols)] of the engine's weights."""
        n = _sz()
        call("mk_engine_tensor_count", self.h, C.byref(n))
        out = []
        for i in range(n.value):
            name, dt, r, c = C.c_char_p(), _u32(), _u64(), _u64()
            call("mk_engine_tensor_at", self.h, i, C.byref(name), C.byref(dt), C.byref(r), C.byref(c))
            out.append((name.value.decode(), dt.value, r.value, c.value))
        return out

    def fetch(self, name, dtype, rows, cols):
        """A weight as stored (float32, bf16 or half bits as uint16, e4m3 codes as uint8); name + ".scale": fp32
        scales."""
        if name.endswith(".scale"):
            a = np.empty(rows, dtype=np.float32)
        else:
            a = np.empty((rows, cols) if cols > 1 else rows, dtype=_NP[dtype])
        call("mk_engine_fetch", self.h, name.encode(), a.ctypes.data, a.nbytes)
        return a

    def weight_bytes(self):
        b = _u64()
        call("mk_engine_weight_bytes", self.h, C.byref(b))
        return b.value

    def begin(self, prompt, h, w, slot=0):
        """prompt: S rows of text_dim embeddings, in any shape holding S x text_dim floats (the reference takes a flat
        span and refuses one that is empty or not whole rows, qwen_image.cpp:117-118)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.float32)
        td = int(self.cfg.text_dim)
        if prompt.size == 0 or prompt.size % td:
            raise MkError(f"prompt embeddings must be rows of {td}")
        call("mk_begin", self.h, prompt.ctypes.data, prompt.size // td, h, w, slot)
        self._grid = (int(h), int(w))

    def step(self, latents, sigma, slot=0):
        latents = np.ascontiguousarray(latents, dtype=np.float32)
        out = np.empty_like(latents)
        call("mk_step", self.h, latents.ctypes.data, latents.size, sigma, slot, out.ctypes.data)
        return out

    def step_cfg(self, latents, sigma, sigma_next, guidance):
        latents = np.ascontiguousarray(latents, dtype=np.float32)
        out = np.empty_like(latents)
        call("mk_step_cfg", self.h, latents.ctypes.data, latents.size, sigma, sigma_next, guidance, out.ctypes.data)
        return out

    def step_cfg_device(self, lat, sigma, sigma_next, guidance, lat_out, stream=None):
        if self._grid:
            nb = self._grid[0] * self._grid[1] * int(self.cfg.latent) * 4
            check_extent(lat, nb, "mk_step_cfg_device: lat")
            check_extent(lat_out, nb, "mk_step_cfg_device: lat_out")
        call("mk_step_cfg_device", self.h, int(lat), sigma, sigma_next, guidance, int(lat_out), stream)

    def generate(self, noise, sigmas, guidance):
        """The Euler loop over `sigmas` (len steps + 1) from `noise` [h*w][latent]; returns the final latents."""
        noise = np.ascontiguousarray(noise, dtype=np.float32)
        sigmas = np.ascontiguousarray(sigmas, dtype=np.float32)
        if sigmas.ndim != 1 or sigmas.size < 2:
            raise MkError("generate: sigmas must hold steps + 1 >= 2 noise levels")
        out = np.empty_like(noise)
        call("mk_generate", self.h, noise.ctypes.data, noise.size, sigmas.ctypes.data, sigmas.size - 1, guidance,
             out.ctypes.data)
        return out

    def stream(self):
        s = _vp()
        call("mk_engine_stream", self.h, C.byref(s))
        return s.value

    def set_probe(self, probes):
        """Collect probes into the dict `probes` ((name, layer) -> array); None turns probing off."""
        if probes is None:
            self._probe_cb = None
            call("mk_engine_set_probe", self.h, PROBE(), None)
            return

        def cb(_u, name, layer, data, n):
            probes[(name.decode(), layer)] = np.ctypeslib.as_array(data, shape=(n,)).copy()

        self._probe_cb = PROBE(cb)
        call("mk_engine_set_probe", self.h, self._probe_cb, None)

    def set_timing(self, on):
        call("mk_engine_set_timing", self.h, int(on))

    def timing(self):
        out = {}
        i = 0
        while True:
            name, ms, n, fl = C.c_char_p(), _f(), _u32(), _d()
            if lib().mk_engine_timing(self.h, i, C.byref(name), C.byref(ms), C.byref(n), C.byref(fl)) != 0:
                break
            out[name.value.decode()] = {"ms": ms.value, "launches": n.value, "flops": fl.value}
            i += 1
        return out

    def sdxl_forward(self, x_dev, batch, n, y_dev):
        nb = int(batch) * int(n) * int(self.cfg.dim) * 4
        check_extent(x_dev, nb, "mk_sdxl_forward: x")
        check_extent(y_dev, nb, "mk_sdxl_forward: y")
        call("mk_sdxl_forward", self.h, int(x_dev), batch, n, int(y_dev), None)


def sigmas(steps, tokens, terminal=0.0, mu=None, base_seq=256.0, max_seq=4096.0, base_shift=0.5, max_shift=1.15):
    """The schedule of Engine::sigmas (engine.cpp:335-365): `steps` noise levels for `tokens` latent tokens, then 0."""
    sc = Schedule(base_seq, max_seq, base_shift, max_shift, terminal, mu is not None, 0.0 if mu is None else mu)
    out = np.empty(steps + 1, np.float32)
    call("mk_sigmas", steps, tokens, C.byref(sc), out.ctypes.data)
    return out


def noise(seed, n):
    """The start noise Engine::generate draws for a seed (engine.cpp:398-408): n floats of
    std::normal_distribution<float> over std::mt19937_64(seed) (mk_noise)."""
    out = np.empty(int(n), np.float32)
    call("mk_noise", int(seed), out.ctypes.data, int(n))
    return out


def rope_table(S, h, w):
    """The RoPE table mk_begin uploads: [S + h*w][64][2] float32 (cos, sin)."""
    out = np.empty((S + h * w, 64, 2), np.float32)
    call("mk_rope_table", S, h, w, out.ctypes.data)
    return out


def upload_model(engine, tensors):
    """Upload (name, float32 array, kind) triples (kind 0 vector, 1 bf16 matrix, 2 fp8 matrix whose values are exact
    e4m3 and whose scale is the tensor name + '.scale', 3 half matrix)."""
    table = None
    for name, a, kind in tensors:
        if kind == 0:
            engine.load(name, a, F32)
        elif kind == 1:
            engine.load(name, bf16_bits(a), BF16)
        elif kind == 3:
            engine.load(name, f16_bits(a), F16)
        else:
            if table is None:
                table = _e4m3_table()
            engine.load(name, _e4m3_codes(a, table), FP8)


def _e4m3_table():
    t = np.zeros(256, dtype=np.float32)
    for b in range(256):
        s, e, m = b >> 7, (b >> 3) & 15, b & 7
        if e == 15 and m == 7:
            v = np.nan
        elif e == 0:
            v = m * 2.0 ** -9
        else:
            v = (1 + m / 8) * 2.0 ** (e - 7)
        t[b] = -v if s else v
    return t


def _e4m3_codes(a, table):
    a = np.asarray(a, dtype=np.float32)
    mags = table[:127]
    idx = np.clip(np.searchsorted(mags, np.abs(a)), 0, 126).astype(np.uint8)
    codes = idx | np.where(np.signbit(a), 0x80, 0).astype(np.uint8)
    if not np.array_equal(table[codes], a):
        raise ValueError("fp8 weights are not exact e4m3 values")
    return codes
