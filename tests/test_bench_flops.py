"""The algorithmic FLOP counts bench.py divides by (the roofline and MFMA fractions it reports), checked against
independent counts: the step's per-block linear and attention work and the step totals of the 1024² bf16 and 2048²
fp8 workloads, the SDXL blocks' work, and the VAE decode counted from the oracle decoder's own weight shapes."""
import re

import pytest

import bench
import mkref as R


def test_step_flops():
    total, lin, attn = bench.step_flops()
    # per block and sample at 4096 image + 256 text tokens: linear 985.7 GFLOP, attention 232.7 GFLOP (as stated, to
    # four significant digits)
    assert lin / 120 == pytest.approx(985.7e9, rel=5e-4)
    assert attn / 120 == pytest.approx(232.7e9, rel=5e-4)
    assert total == pytest.approx(146.26e12, rel=1e-3)
    # 2048x2048: 16384 image + 512 text tokens
    total5, lin5, attn5 = bench.step_flops(N=16384, S=512)
    assert lin5 / 120 == pytest.approx(3826.8e9, rel=5e-4)
    assert attn5 / 120 == pytest.approx(3507.9e9, rel=5e-4)
    assert total5 == pytest.approx(880.24e12, rel=1e-3)


def test_sdxl_flops():
    # per block (batch 2): stage A (4096 tokens, 640 channels) 208.3 GFLOP, stage B (1024, 1280) 132.3 GFLOP;
    # proj_in and proj_out (2 C^2 n each) once a forward
    for n, C, want in ((4096, 640, 208.3e9), (1024, 1280, 132.3e9)):
        f1, _ = bench.sdxl_flops(n, C, 1)
        f2, _ = bench.sdxl_flops(n, C, 2)
        assert f2 - f1 == pytest.approx(want, rel=1e-3)
        assert f1 - (f2 - f1) == pytest.approx(2 * 2 * 2 * C * C * n, rel=1e-9)


@pytest.mark.parametrize("base, th, tw", [(16, 3, 5), (96, 64, 64)])
def test_vae_flops_from_the_decoders_weights(base, th, tw):
    # 2 x pixels x (out x in x k x k) for every conv weight of the decoder, at the level it runs at, plus the mid
    # block's attention 4 n^2 c; the level of a tensor follows from its name
    vae = R.Vae(base, seed=0) if base == 16 else None
    if vae is None:
        # the 96-channel decoder's shapes: the 16-channel one's scaled (same names, every channel count x 6, except
        # the latent's 16 and the 3 output channels)
        shapes = {n: a.shape for n, a in R.Vae(16, seed=0).tensors()}

        def scale(n, s):
            if len(s) != 4:
                return s
            o, i = s[0], s[1]
            o = o if n.startswith("post_quant") or n.startswith("decoder.conv_out") else o * 6
            i = i if n.startswith("post_quant") or n.startswith("decoder.conv_in") else i * 6
            return (o, i) + tuple(s[2:])
        shapes = {n: scale(n, s) for n, s in shapes.items()}
    else:
        shapes = {n: a.shape for n, a in vae.tensors()}
    n0 = 4 * th * tw
    total = 0
    for name, s in shapes.items():
        if len(s) != 4:
            continue
        m = re.match(r"decoder\.up_blocks\.(\d+)\.(resnets|upsamplers)", name)
        if m:
            level = int(m.group(1)) + (1 if m.group(2) == "upsamplers" else 0)
        elif name.startswith("decoder.conv_out"):
            level = 3
        else:
            level = 0
        total += 2 * n0 * 4 ** level * s[0] * s[1] * s[2] * s[3]
    d0 = 4 * base
    total += 4 * n0 * n0 * d0
    got, attn = bench.vae_flops(th, tw, b=base)
    assert attn == 4 * n0 * n0 * d0
    assert got == total


def test_kernel_names_follow_the_profiled_launches():
    # the kernel each timing class names (and whose traffic bench.py reports) is one the profiled step launches:
    # a renamed or re-templated kernel would otherwise leave the roofline's traffic figure silently empty
    prof = (bench.ROOT / "profiles" / "mmdit_step_1024_kernels.md").read_text()
    for cls, name in bench.KERNEL_OF.items():
        assert name in prof, (cls, name)
        assert bench.kernel_traffic(name) is not None, (cls, name)
    prof21 = (bench.ROOT / "profiles" / "q21_step_1024_kernels.md").read_text()
    for cls, name in bench.KERNEL_OF_Q21.items():
        assert name.split(" (")[0] in prof21, (cls, name)
