"""Writes tests/golden/golden.npz: inputs and expected outputs of the textbook pieces of the hot path, computed by
PyTorch's CPU library routines in float64 (layer_norm, rms_norm, group_norm, gelu, silu, scaled_dot_product_attention,
the bfloat16 and float8_e4m3fn casts). They pin the oracle (oracle/mkref.cpp) independently of its own code.

The reference (mako-image) holds no vectors for this path: its model tests compare against tensors kept outside the
repository (tests/image_ref_test.cpp:1-8), so these come from library routines instead.

Run: python tests/golden/make_golden.py   (CPU only; deterministic)
"""
import pathlib

import numpy as np
import torch
import torch.nn.functional as F

OUT = pathlib.Path(__file__).resolve().parent / "golden.npz"


def bf16(x):
    return torch.as_tensor(x).to(torch.bfloat16).to(torch.float64)


def main():
    g = torch.Generator().manual_seed(1234)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    out = {}

    # LayerNorm (no affine) then (1 + scale) + shift
    x, sc, sh = r(9, 96) * 3 + 0.5, r(96) * 0.3, r(96) * 0.3
    out["ln_x"], out["ln_scale"], out["ln_shift"] = x, sc, sh
    out["ln_y"] = F.layer_norm(x, (96,), eps=1e-6) * (1 + sc) + sh
    # LayerNorm with gamma / beta, eps 1e-5
    gm, bt = 1 + r(96) * 0.1, r(96) * 0.1
    out["lna_g"], out["lna_b"] = gm, bt
    out["lna_y"] = F.layer_norm(x, (96,), weight=gm, bias=bt, eps=1e-5)
    # RMSNorm with weight
    w = 1 + r(96) * 0.1
    out["rms_w"] = w
    out["rms_y"] = F.rms_norm(x, (96,), weight=w, eps=1e-6)
    # GroupNorm, 32 groups over channels-last rows [rows][c]
    gx, gg, gb = r(50, 64), 1 + r(64) * 0.1, r(64) * 0.1
    out["gn_x"], out["gn_g"], out["gn_b"] = gx, gg, gb
    out["gn_y"] = F.group_norm(gx.t().unsqueeze(0), 32, gg, gb, eps=1e-6)[0].t()
    # activations
    a = r(1000) * 4
    out["act_x"] = a
    out["gelu_tanh"] = F.gelu(a, approximate="tanh")
    out["silu"] = F.silu(a)
    hg = r(7, 2 * 40) * 2
    out["geglu_x"] = hg
    out["geglu_y"] = hg[:, :40] * F.gelu(hg[:, 40:])
    out["swiglu_y"] = F.silu(hg[:, :40]) * hg[:, 40:]
    # GEMM with bf16 operands, fp64 accumulate: y = bf16(A) bf16(W)^T + b
    A, W, b = r(37, 128), r(80, 128) * 0.02, r(80) * 0.02
    out["gemm_a"], out["gemm_w"], out["gemm_b"] = A, bf16(W), b
    out["gemm_y"] = bf16(A) @ bf16(W).t() + b
    # attention: bf16-exact q, k, v; [B][H][T][d]
    for name, (T, d, kind) in {"attn": (37, 128, "none"), "attn64": (29, 64, "none"), "attnc": (33, 128, "causal"),
                               "attnp": (40, 128, "prefix")}.items():
        q, k, v = bf16(r(1, 2, T, d)), bf16(r(1, 2, T, d)), bf16(r(1, 2, T, d))
        mask = None
        if kind == "causal":
            mask = torch.ones(T, T, dtype=torch.bool).tril()
        elif kind == "prefix":  # the first 12 rows (text) causal among themselves; the rest see every key
            mask = torch.ones(T, T, dtype=torch.bool)
            mask[:12, :] = torch.ones(12, T, dtype=torch.bool).tril()
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=1 / np.sqrt(d))
        out[name + "_q"], out[name + "_k"], out[name + "_v"] = q, k, v
        out[name + "_o"] = o.permute(0, 2, 1, 3).reshape(1, T, 2 * d)
    # bf16 round-to-nearest-even of tricky values (torch's cast is the independent rule)
    vals = np.concatenate([
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 1.0078125, 3.4e38, -3.4e38, 1e-40, -1e-40, np.inf, -np.inf],
                 dtype=np.float32),
        np.frombuffer(np.random.default_rng(5).integers(0, 2**32, 4000, dtype=np.uint64).astype(np.uint32).tobytes(),
                      dtype=np.float32)])
    vals = vals[np.isfinite(vals) | np.isinf(vals)]
    out["bf16_in"] = vals
    out["bf16_bits"] = torch.from_numpy(vals.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    # e4m3: every code's value, and encodings of in-range values (torch's float8_e4m3fn cast)
    codes = torch.arange(256, dtype=torch.int16).to(torch.uint8)
    out["e4m3_decode"] = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    ev = np.concatenate([np.linspace(-448, 448, 2001), np.random.default_rng(6).standard_normal(3000) * 20,
                         np.random.default_rng(7).standard_normal(1000) * 0.01]).astype(np.float32)
    out["e4m3_in"] = ev
    out["e4m3_codes"] = torch.from_numpy(ev).to(torch.float8_e4m3fn).view(torch.uint8).numpy()

    arrays = {k: (v.numpy() if isinstance(v, torch.Tensor) else v) for k, v in out.items()}
    arrays = {k: (v.astype(np.float32) if v.dtype == np.float64 else v) for k, v in arrays.items()}
    # expected values are kept in float64 where the precision matters
    for k in ("ln_y", "lna_y", "rms_y", "gn_y", "gelu_tanh", "silu", "geglu_y", "swiglu_y", "gemm_y", "attn_o",
              "attn64_o", "attnc_o", "attnp_o"):
        arrays[k] = out[k].numpy()
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
