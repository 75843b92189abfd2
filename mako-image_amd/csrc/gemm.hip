// proj: C = A W^T on gfx950 bf16 MFMA, fp32 accumulation, with fused epilogues.
//
// Roles: the weight tile is the MFMA A operand (its M = output channels) and the activation tile the B operand (its
// N = tokens), so each lane's accumulators hold 4 consecutive channels of one token: the epilogues stage a wave's
// 32-token slice through LDS and write whole row segments.
//
// Tiling: BM = 256 (or 128) tokens x BN channels x 64 k per workgroup; 256- and 192-wide tiles run 8 waves (two a
// SIMD: 2 along channels x 4 along tokens) on v_mfma_f32_16x16x32_bf16, 128- and 64-wide ones 4 waves (2 x 2) on
// v_mfma_f32_32x32x16_bf16, 96-wide ones (convolutions) 4 waves of whole 96-channel rows on 16x16x32; 128-token tiles
// run two workgroups a CU. Both tiles are K-contiguous and staged in LDS with a 16-byte-chunk XOR swizzle
// (chunk ^ ((row >> 1) & 7)) so the fragment reads of 16 or 32 rows at one k offset are bank-conflict free. Two LDS
// buffers, one barrier per k step: buffer loads write a later k step straight into LDS while the current one's
// MFMAs run (128-channel tiles stage it through registers instead). The main loop's instruction order is fixed by
// hand (every MFMA, fragment read and load fenced): loads and reads spread over the MFMAs, each read issued in the
// order its MFMA needs it. Workgroups map to tiles XCD-aware (consecutive tiles on one XCD share its L2) and grouped
// along M.
#include "common.hpp"

#include <memory>
#include <mutex>
#include <type_traits>
#include <vector>

namespace mk {

namespace gemm_detail {

struct HeadsP {
    uint16_t *q, *k, *vt;
    uint32_t heads, q_pad, k_pad, row0, q_row0, rope_mode, dim;
    const float *norm_q, *norm_k, *rope;
    float eps, k_scale;
    uint32_t f16;     // Q, K, V^T as IEEE half (else bf16)
    int64_t rope_bs;  // floats between the batch items' RoPE tables
    uint32_t hd;      // head dim: 128 (a wave slice of 128 channels is one head) or 64 (128-channel tiles)
};

struct GemmP {
    const uint16_t* a;
    const void* w;
    const float* wscale;
    const float* bias;
    void* c;
    const float* gate;
    int64_t gate_alt;
    uint32_t split, seg_rows, M, N, K;
    int64_t lda, ldc, sa, sc;
    uint32_t epi, c_bf16, c_f16; // 16-bit outputs (c_bf16), as IEEE half (c_f16) rather than bf16
    uint32_t tiles_m, tiles_n, batch;
    HeadsP hp;
    // 3 x 3 convolution (EK_CONV): the padded grid's row width w + 2, k tiles a tap (channels / 64), and
    // ceil(2^16 / conv_tpt) for the tap index by multiply-shift; with EK_CONVQ conv_tpt counts 8-channel chunks
    uint32_t conv_pw, conv_tpt, conv_inv;
    // With conv_w (the image width, a multiple of BM) the tiles cover the conv_pix = h w pixels only, BM of one image
    // row each (tile tm: pixel tm BM, grid row (y + 1) pw + x + 1), so no tile is spent on ring rows and the launch
    // holds whole rounds where h w does; the ring's output rows are then not written.
    uint32_t conv_w, conv_pix;
    // gated linear unit (EK_GLU): the weights' rows are [first part F; second part F], the output [M][F]
    uint32_t glu_f;
    // EK_NORM / EK_RMWN: the RMS norm's per-channel gain; EK_RMWN: the normed rows' 16-bit output and its row stride
    // (EK_RMWUP: the 2x grid's 16-bit buffer, from its first row, and row stride)
    const float* norm_g;
    uint16_t* norm_out;
    uint32_t norm_ld;
    // EK_RMWUP: the 2x grid's row width (2 w + 2) and slack rows (2 w + 3)
    uint32_t up_pw, up_slack;
    // EK_RMWN: the fp32 rows are not stored, only their norm
    uint32_t norm_only;
};

// One launch of up to two GEMMs of equal N, K and epilogue kind (the dual-stream blocks' image and text
// projections): workgroups [0, tiles0 * ...) take problem 0, the rest problem 1 (grid z = the larger batch).
struct GemmG {
    GemmP g[2];
    uint32_t tiles0;
};

constexpr int BK = 64;


// LDS tile rows are 64 bf16 (128 bytes, 8 chunks of 16). gfx950's LDS has 64 banks (256 bytes a cycle): a 16-byte read
// serves 16 lanes a cycle, here 16 consecutive rows at one logical chunk. Rows r and r + 1 fall in opposite halves of
// the banks, so the chunk is XOR-ed with (row >> 1) & 7: the 8 rows of each half get 8 distinct chunks.
__device__ inline int swz_chunk(int row, int kc) { return kc ^ ((row >> 1) & 7); }
__device__ inline int swz(int row, int kc) { return row * 64 + (swz_chunk(row, kc) << 3); }

// fp8 e4m3 (16 values in a u32x4) -> two bf16x8 chunks, exact (every e4m3 value is a bf16 value): gfx950's
// conversion instruction, two values each.
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
__device__ inline void f8x16_to_bf16(const u32x4& v, u32x4& lo, u32x4& hi)
{
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t x = v[i];
        const bf16x2v a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, false); // bytes 0, 1
        const bf16x2v b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, true);  // bytes 2, 3
        o[2 * i] = __builtin_bit_cast(uint32_t, a);
        o[2 * i + 1] = __builtin_bit_cast(uint32_t, b);
    }
    lo = u32x4{o[0], o[1], o[2], o[3]};
    hi = u32x4{o[4], o[5], o[6], o[7]};
}

// Epilogue kinds (template): a plain store, an activation, a read-modify-write of the fp32 residual, the q/k/v heads,
// a gated linear unit (SwiGLU / GEGLU: each output channel from two weight rows F apart).
// EK_NORM: a 96-channel convolution's rows RMS-normed and SiLU-ed into the next convolution's 16-bit input grid;
// EK_RMWN: the rows stored (or added into the fp32 residual) and their RMS norm + SiLU written besides; EK_RMWUP: the
// rows added into the residual and written, 16-bit, to the four pixels each becomes in the nearest 2x grid. (A
// convolution's 16-bit grids are IEEE half, like its operands.)
enum { EK_STORE = 0, EK_ACT = 1, EK_RMW = 2, EK_HEADS = 3, EK_GLU = 4, EK_NORM = 5, EK_RMWN = 6, EK_RMWUP = 7 };
// Flag on the epilogue kind: the A operand is a 3 x 3 convolution's input (implicit im2col, see conv_koff).
constexpr int EK_CONV = 8;
// With EK_CONV: input channels not a multiple of 64 (dense K = 9 c rounded up to 64, k = tap c + channel): a k step
// spans taps, so each 16-byte chunk (8 channels) takes its own tap's row shift (conv3x3_dense).
constexpr int EK_CONVQ = 32;
// Flag on the epilogue kind: the operands are IEEE half (v_mfma_f32_*_f16): the VAE's convolutions and products, whose
// reference multiplies F16 weights with half activations (docs/performance.md:13, engine.cpp:766-773).
constexpr int EK_F16 = 64;
// Flag on the epilogue kind: a launch of at most one tile a CU (each workgroup alone on its CU) on 4-wave 128-channel
// tiles. The operands go global -> LDS by direct loads through NSTG stages (4 for 128-token tiles, 3 for 256), each
// k step's loads issued NSTG - 1 steps ahead of its use; the two-workgroup form stages them through registers three
// substeps ahead, a latency a workgroup alone on its CU cannot hide.
constexpr int EK_DEEP = 128;
// s_waitcnt immediate (gfx9 layout): vmcnt vm (0-63: bits 3:0 and 15:14), expcnt not waited for, lgkmcnt lgkm (0-15)
constexpr int waitcnt_bits(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8); }
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));

// A pair of 16-bit outputs: IEEE half (H) or bf16, round to nearest even either way. The type is a template
// argument: the epilogues test the run-time flag once and run a copy of their store code for each type (with the flag
// tested at every pair the compiler emits a uniform branch, a scalar reload of the flag and an LDS wait per pair).
template <bool H> __device__ inline uint32_t pack16(float a, float b) { return H ? pack_f16x2(a, b) : pack_bf16x2(a, b); }
// f(std::bool_constant<flag>{}): one branch on a uniform flag around code specialised for each value
template <class F> __device__ inline void with_flag(bool flag, F&& f)
{
    if (flag)
        f(std::true_type{});
    else
        f(std::false_type{});
}

// Per-tile channel constants of a lane's 4 channels (the same for every token row it writes).
struct EpiCh {
    f32x4 scale, bias, g0, g1; // g0: the gate row, g1: the alternate gate row (rows r % seg_rows < split)
};

// MK_EPI_GATE_TANH: the gates through tanh (apart from the loads, so the residual's loads can go out in between: the
// tanh waits for the gate loads only)
__device__ inline void epi_gate_tanh(const GemmP& p, EpiCh& c)
{
    if (p.gate && p.epi == MK_EPI_GATE_TANH)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            c.g0[e] = tanh_f(c.g0[e]);
            c.g1[e] = tanh_f(c.g1[e]);
        }
}

__device__ inline EpiCh epi_channels(const GemmP& p, int ch, bool tanh_now = true)
{
    EpiCh c;
    c.scale = p.wscale ? *reinterpret_cast<const f32x4*>(p.wscale + ch) : f32x4{1, 1, 1, 1};
    c.bias = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + ch) : f32x4{0, 0, 0, 0};
    if (p.gate) {
        // without a split the alternate row is the gate row itself, loaded again: a copy of g0 would wait for g0's
        // load right here, before the loads that follow could go out
        c.g0 = *reinterpret_cast<const f32x4*>(p.gate + ch);
        c.g1 = *reinterpret_cast<const f32x4*>(p.gate + (p.split ? p.gate_alt : 0) + ch);
    }
    if (tanh_now)
        epi_gate_tanh(p, c);
    return c;
}

// Epilogue of a wave's staged slice: 32 token rows x WC channels in LDS (row stride ld floats), rows tok0 .. of the
// GEMM, channels from chw. Lanes run along the channels (4 each, WC/4 lanes a row), so LDS reads are conflict free and
// every store instruction writes whole row segments. For the residual the rows' x loads go out together before the
// stores (vmcnt also counts stores: a load among the stores would wait for all of them).
// With SW the slice is 32 x 32 in unpadded 32-float rows whose 16-byte chunks are XOR-swizzled (stage_sw).
template <int EK, int WC, bool SW = false>
__device__ inline void epi_slice(const GemmP& p, const float* st, int ld, int tok0, int chw, int lane, int64_t zc,
                                 const EpiCh& k)
{
    constexpr int LPR = WC / 4, RPI = 64 / LPR, NI = 32 / RPI; // lanes a row, rows an instruction, rows a lane
    static_assert(!SW || WC == 32, "swizzled staging holds 32 channels");
    const int c = lane % LPR, r0 = lane / LPR, ch = chw + 4 * c;
    f32x4 v[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = r0 + RPI * i;
        v[i] = *reinterpret_cast<const f32x4*>(SW ? st + row * 32 + 4 * (c ^ ((row >> 1) & 7)) : st + row * ld + 4 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            v[i][e] = v[i][e] * k.scale[e] + k.bias[e];
    }
    if constexpr (EK == EK_RMWUP) {
        // x + v (the convolution's ADD) goes to the four pixels (2 y + dy, 2 x + dx) of the nearest 2x grid, 16-bit;
        // the residual itself is not stored (its next reader is the upsampling). Tiles over the pixels only: every
        // row of the slice is a pixel of image row y.
        const float* c = static_cast<const float*>(p.c) + ch;
        const uint32_t pw = p.conv_pw, y = uint32_t(tok0) / pw - 1, ld2 = p.norm_ld;
        uint16_t* up = p.norm_out + ch;
        f32x4 xs[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i)
            xs[i] = *reinterpret_cast<const f32x4*>(c + int64_t(min(tok0 + r0 + RPI * i, int(p.M) - 1)) * p.ldc);
        with_flag(p.c_f16, [&](auto h_c) {
            constexpr bool H = decltype(h_c)::value;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int t = tok0 + r0 + RPI * i;
                const f32x4& x = xs[i];
                if (t < int(p.M)) {
                    const uint32_t xx = uint32_t(t) - (y + 1) * pw - 1;
                    const uint64_t r = p.up_slack + uint64_t(2 * y + 1) * p.up_pw + 2 * xx + 1;
                    const u32x2 o{pack16<H>(x[0] + v[i][0], x[1] + v[i][1]), pack16<H>(x[2] + v[i][2], x[3] + v[i][3])};
                    *reinterpret_cast<u32x2*>(up + r * ld2) = o;
                    *reinterpret_cast<u32x2*>(up + (r + 1) * ld2) = o;
                    *reinterpret_cast<u32x2*>(up + (r + p.up_pw) * ld2) = o;
                    *reinterpret_cast<u32x2*>(up + (r + p.up_pw + 1) * ld2) = o;
                }
            }
        });
        return;
    }
    if constexpr (EK == EK_RMW) {
        // rows past M read (and leave) the last valid row
        float* c = static_cast<float*>(p.c) + zc + ch;
        f32x4 x[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i)
            x[i] = *reinterpret_cast<const f32x4*>(c + int64_t(min(tok0 + r0 + RPI * i, int(p.M) - 1)) * p.ldc);
        const bool add = p.epi == MK_EPI_ADD;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int t = tok0 + r0 + RPI * i;
            const f32x4& g = (uint32_t(t) % p.seg_rows) < p.split ? k.g1 : k.g0;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                x[i][e] += (add ? 1.0f : g[e]) * v[i][e];
        }
        const int64_t step = int64_t(RPI) * p.ldc;
        float* c0 = c + int64_t(tok0 + r0) * p.ldc;
        if (tok0 + 32 <= int(p.M)) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
                *reinterpret_cast<f32x4*>(c0 + i * step) = x[i];
        } else {
            for (int i = 0; i < NI && tok0 + r0 + RPI * i < int(p.M); ++i)
                *reinterpret_cast<f32x4*>(c0 + i * step) = x[i];
        }
        return;
    }
    if constexpr (EK == EK_ACT) {
        // GELU or SiLU for the whole slice (one branch)
        with_flag(p.epi == MK_EPI_GELU_TANH, [&](auto g_c) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[i][e] = decltype(g_c)::value ? gelu_tanh_f(v[i][e]) : silu_f(v[i][e]);
        });
    }
    // the stores: straight-line when the slice is whole (row-guard branches between stores make the compiler wait
    // for each store before the next)
    const bool whole = tok0 + 32 <= int(p.M);
    const int64_t off0 = zc + int64_t(tok0 + r0) * p.ldc + ch, step = int64_t(RPI) * p.ldc;
    if (p.c_bf16) {
        u32x2 o[NI];
        with_flag(p.c_f16, [&](auto h_c) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
                o[i] = u32x2{pack16<decltype(h_c)::value>(v[i][0], v[i][1]),
                             pack16<decltype(h_c)::value>(v[i][2], v[i][3])};
        });
        uint16_t* c = static_cast<uint16_t*>(p.c) + off0;
        if (whole) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
                *reinterpret_cast<u32x2*>(c + i * step) = o[i];
        } else {
            for (int i = 0; i < NI && tok0 + r0 + RPI * i < int(p.M); ++i)
                *reinterpret_cast<u32x2*>(c + i * step) = o[i];
        }
    } else {
        float* c = static_cast<float*>(p.c) + off0;
        if (whole) {
#pragma unroll
            for (int i = 0; i < NI; ++i)
                *reinterpret_cast<f32x4*>(c + i * step) = v[i];
        } else {
            for (int i = 0; i < NI && tok0 + r0 + RPI * i < int(p.M); ++i)
                *reinterpret_cast<f32x4*>(c + i * step) = v[i];
        }
    }
}

// The residual epilogue in two halves, so a tile's slices can overlap: rmw_load issues the loads of a slice's x rows
// (rows past M read the last valid row), rmw_finish adds gate * (acc scale + bias) to them and stores the rows; the
// next slice's loads go out before this slice's stores (epi_slice's lane mapping: WC / 4 lanes a row).
template <int WC>
__device__ inline void rmw_load(const GemmP& p, int tok0, int chw, int lane, int64_t zc, f32x4 (&x)[WC / 8])
{
    constexpr int LPR = WC / 4, RPI = 64 / LPR, NI = 32 / RPI;
    const int c = lane % LPR, r0 = lane / LPR;
    const float* cp = static_cast<const float*>(p.c) + zc + chw + 4 * c;
#pragma unroll
    for (int i = 0; i < NI; ++i)
        x[i] = *reinterpret_cast<const f32x4*>(cp + int64_t(min(tok0 + r0 + RPI * i, int(p.M) - 1)) * p.ldc);
}
template <int WC>
__device__ inline void rmw_finish(const GemmP& p, const float* st, int ld, int tok0, int chw, int lane, int64_t zc,
                                  const EpiCh& k, f32x4 (&x)[WC / 8])
{
    constexpr int LPR = WC / 4, RPI = 64 / LPR, NI = 32 / RPI;
    const int c = lane % LPR, r0 = lane / LPR;
    const bool add = p.epi == MK_EPI_ADD;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(st + (r0 + RPI * i) * ld + 4 * c);
        const int t = tok0 + r0 + RPI * i;
        const f32x4& g = (uint32_t(t) % p.seg_rows) < p.split ? k.g1 : k.g0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            x[i][e] += (add ? 1.0f : g[e]) * (v[e] * k.scale[e] + k.bias[e]);
    }
    float* c0 = static_cast<float*>(p.c) + zc + chw + 4 * c + int64_t(tok0 + r0) * p.ldc;
    const int64_t step = int64_t(RPI) * p.ldc;
    if (tok0 + 32 <= int(p.M)) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
            *reinterpret_cast<f32x4*>(c0 + i * step) = x[i];
    } else {
        for (int i = 0; i < NI && tok0 + r0 + RPI * i < int(p.M); ++i)
            *reinterpret_cast<f32x4*>(c0 + i * step) = x[i];
    }
}

// The q / k / v epilogue from a wave's staged slice: 32 tokens x 128 channels (one head of q, k or v) in LDS, row
// stride ld floats, tokens tok0 .. tok0 + 31 (GEMM rows).
//  - q, k: lanes along the head's channels (4 each, 32 lanes a row, rows r0 + 2i for i < 16): per-head RMSNorm * w
//    (the row's sum of squares reduced across its 32 lanes), RoPE, 16-bit rows to [batch][heads][pad][128]. Every
//    global load (channel constants, RoPE factors) is issued before the first store: vmcnt also counts stores, so a
//    load behind stores would wait for all of them.
//  - v: each lane two head dims across the 32 tokens, 16-bit to V^T [batch][heads][128][k_pad] rows (keys in the
//    vt_col order).
// (F16: the output type; MODE: the RoPE mode, 0 none, 1 half-split pairs, 2 interleaved pairs; both template
// arguments, so the code a launch runs has no per-row tests of them)
template <bool F16, int MODE>
__device__ inline void epi_heads(const GemmP& p, const float* st, int ld, int tok0, int nw0, int lane, uint32_t z)
{
    const HeadsP& h = p.hp;
    const int which = nw0 / int(h.dim), head = (nw0 % int(h.dim)) / 128;
    const int64_t bh = int64_t(z) * h.heads + head;
    if (which == 2) {
        float sc[2], bi[2];
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
            sc[dd] = p.wscale ? p.wscale[nw0 + 2 * lane + dd] : 1.0f;
            bi[dd] = p.bias ? p.bias[nw0 + 2 * lane + dd] : 0.0f;
        }
        const uint32_t k0 = h.row0 + tok0;
        const bool full = k0 % 16 == 0 && tok0 + 32 <= int(p.M);
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
            const int d = 2 * lane + dd;
            uint16_t* dst = h.vt + (bh * 128 + d) * int64_t(h.k_pad);
            auto v = [&](int j) { return st[j * ld + d] * sc[dd] + bi[dd]; };
            if (full) {
#pragma unroll
                for (int g = 0; g < 2; ++g) {
                    // physical columns 16g + 0..15 hold keys 16g + {0..3, 8..11, 4..7, 12..15}
                    const int j0 = 16 * g;
                    *reinterpret_cast<u32x4*>(dst + k0 + j0) =
                        u32x4{pack_x2(v(j0 + 0), v(j0 + 1), F16), pack_x2(v(j0 + 2), v(j0 + 3), F16),
                              pack_x2(v(j0 + 8), v(j0 + 9), F16), pack_x2(v(j0 + 10), v(j0 + 11), F16)};
                    *reinterpret_cast<u32x4*>(dst + k0 + j0 + 8) =
                        u32x4{pack_x2(v(j0 + 4), v(j0 + 5), F16), pack_x2(v(j0 + 6), v(j0 + 7), F16),
                              pack_x2(v(j0 + 12), v(j0 + 13), F16), pack_x2(v(j0 + 14), v(j0 + 15), F16)};
                }
            } else {
                for (int t = 0; t < 32 && tok0 + t < int(p.M); ++t)
                    dst[vt_col(k0 + t)] = F16 ? f2h_bits(v(t)) : f2bf_bits(v(t));
            }
        }
        return;
    }
    const float* nw = which == 0 ? h.norm_q : h.norm_k;
    const int c = lane & 31, r0 = lane >> 5, ch = 4 * c;
    const f32x4 sc = p.wscale ? *reinterpret_cast<const f32x4*>(p.wscale + nw0 + ch) : f32x4{1, 1, 1, 1};
    const f32x4 bi = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + nw0 + ch) : f32x4{0, 0, 0, 0};
    // the norm weights, with K's scale folded in (norm, RoPE and the scale are all linear in the row)
    const float ks = which == 1 ? h.k_scale : 1.0f;
    f32x4 wn = nw ? *reinterpret_cast<const f32x4*>(nw + ch) : f32x4{1, 1, 1, 1};
#pragma unroll
    for (int e = 0; e < 4; ++e)
        wn[e] *= ks;
    constexpr int mode = MODE;
    const int last = int(p.M) - 1;
    // RoPE factors of a row (clamped to the last valid row): mode 2, pairs (2c, 2c + 1) -> (cos, sin, cos, sin) of
    // the lane's 4 channels; mode 1, channel d and d + 64 pair at angle d -> cos / sin of angles 4 (c % 16) .. + 3
    auto rope_lo = [&](int i) {
        const int t = min(tok0 + r0 + 2 * i, last);
        const float* cs = h.rope + int64_t(z) * h.rope_bs + (int64_t(h.row0) + t) * 128;
        return *reinterpret_cast<const f32x4*>(cs + (mode == 2 ? ch : 8 * (c & 15)));
    };
    auto rope_hi = [&](int i) {
        const int t = min(tok0 + r0 + 2 * i, last);
        return *reinterpret_cast<const f32x4*>(h.rope + int64_t(z) * h.rope_bs + (int64_t(h.row0) + t) * 128 +
                                               8 * (c & 15) + 4);
    };
    auto val = [&](int i) {
        f32x4 x = *reinterpret_cast<const f32x4*>(st + (r0 + 2 * i) * ld + ch);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            x[e] = x[e] * sc[e] + bi[e];
        return x;
    };
    // the RoPE factors go out before anything else: mode 2 all 16 rows' (one f32x4 a row), mode 1 the first half's
    // (two a row; the second half's after the first half is written)
    f32x4 ra[16], rb[8];
    if (mode == 2)
#pragma unroll
        for (int i = 0; i < 16; ++i)
            ra[i] = rope_lo(i);
    else if (mode == 1)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ra[i] = rope_lo(i);
            rb[i] = rope_hi(i);
        }
    // per-row 1 / rms over the head: partial sums of squares, then a reduce across the row's 32 lanes
    float inv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
        inv[i] = 1.0f;
    if (nw) {
        float ss[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const f32x4 x = val(i);
            ss[i] = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i)
            ss[i] = half_sum(ss[i]); // lanes 0-31 hold row 2i, lanes 32-63 row 2i + 1
#pragma unroll
        for (int i = 0; i < 16; ++i)
            inv[i] = rsqrtf(ss[i] * (1.0f / 128.0f) + h.eps);
    }
    const int64_t pad = which == 0 ? h.q_pad : h.k_pad;
    uint16_t* base = (which == 0 ? h.q : h.k) + (bh * pad + (which == 0 ? h.q_row0 : h.row0)) * 128 + ch;
    auto emit = [&](int i, const f32x4& r_lo, const f32x4& r_hi) {
        f32x4 x = val(i);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            x[e] *= inv[i] * wn[e];
        if (mode == 2) {
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                const float co = r_lo[e], si = r_lo[e + 1], a = x[e], b = x[e + 1];
                x[e] = a * co - b * si;
                x[e + 1] = a * si + b * co;
            }
        } else if (mode == 1) {
            // lanes c and c + 16 hold channels d and d + 64 (d = 4 (c % 16) + e): the partner's value by one swap
            const bool lo = c < 16;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float other = __shfl_xor(x[e], 16, 64);
                const float co = e < 2 ? r_lo[2 * e] : r_hi[2 * e - 4];
                const float si = e < 2 ? r_lo[2 * e + 1] : r_hi[2 * e - 3];
                x[e] = lo ? x[e] * co - other * si : other * si + x[e] * co;
            }
        }
        // a row past M stores into the last row: its A row was read as the last row's (the loads clamp), so every
        // value it computes is the last row's, bit for bit. No row guard, so the rows' code is one straight block in
        // which the next rows' LDS reads can go out ahead of this row's store.
        const int t = min(tok0 + r0 + 2 * i, last);
        *reinterpret_cast<u32x2*>(base + int64_t(t) * 128) = u32x2{pack_x2(x[0], x[1], F16), pack_x2(x[2], x[3], F16)};
    };
#pragma unroll
    for (int i = 0; i < 8; ++i)
        emit(i, ra[i], rb[i]);
    if (mode == 1)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            ra[i] = rope_lo(8 + i);
            rb[i] = rope_hi(8 + i);
        }
#pragma unroll
    for (int i = 0; i < 8; ++i)
        emit(8 + i, mode == 2 ? ra[8 + i] : ra[i], rb[i]);
}

// The heads epilogue for 64-dim heads (the SDXL form: no norm, no RoPE) on 128-channel tiles, whose wave slice of
// 32 tokens x 64 channels is one head: Q / K rows [bh][row][64] (16 lanes a row, 4 channels each), V^T rows
// [bh][d][k_pad] (a lane per dim, 32 keys in the vt_col order). Q-only launches (k == NULL) write Q alone, k|v-only
// launches (q == NULL: the cross attention's context, heads_half from the fp32 projection, sdxl.cpp:697-708) K and
// V^T, each rounded once from the fp32 accumulators.
template <bool F16>
__device__ inline void epi_heads64(const GemmP& p, const float* st, int ld, int tok0, int nw0, int lane, uint32_t z)
{
    const HeadsP& h = p.hp;
    // 0 q, 1 k, 2 v (a k|v-only launch, q NULL, starts at k)
    const int which = nw0 / int(h.dim) + (h.q ? 0 : 1), head = (nw0 % int(h.dim)) / 64;
    const int64_t bh = int64_t(z) * h.heads + head;
    const int last = int(p.M) - 1;
    if (which == 2) {
        const int d = lane;
        const float sc = p.wscale ? p.wscale[nw0 + d] : 1.0f, bi = p.bias ? p.bias[nw0 + d] : 0.0f;
        const uint32_t k0 = h.row0 + tok0;
        uint16_t* dst = h.vt + (bh * 64 + d) * int64_t(h.k_pad);
        auto v = [&](int j) { return st[j * ld + d] * sc + bi; };
        if (k0 % 16 == 0 && tok0 + 32 <= int(p.M)) {
#pragma unroll
            for (int g = 0; g < 2; ++g) {
                // physical columns 16g + 0..15 hold keys 16g + {0..3, 8..11, 4..7, 12..15}
                const int j0 = 16 * g;
                *reinterpret_cast<u32x4*>(dst + k0 + j0) =
                    u32x4{pack_x2(v(j0 + 0), v(j0 + 1), F16), pack_x2(v(j0 + 2), v(j0 + 3), F16),
                          pack_x2(v(j0 + 8), v(j0 + 9), F16), pack_x2(v(j0 + 10), v(j0 + 11), F16)};
                *reinterpret_cast<u32x4*>(dst + k0 + j0 + 8) =
                    u32x4{pack_x2(v(j0 + 4), v(j0 + 5), F16), pack_x2(v(j0 + 6), v(j0 + 7), F16),
                          pack_x2(v(j0 + 12), v(j0 + 13), F16), pack_x2(v(j0 + 14), v(j0 + 15), F16)};
            }
        } else {
            for (int t = 0; t < 32 && tok0 + t <= last; ++t)
                dst[vt_col(k0 + t)] = F16 ? f2h_bits(v(t)) : f2bf_bits(v(t));
        }
        return;
    }
    const int c = lane & 15, r0 = lane >> 4, ch = 4 * c;
    const f32x4 sc = p.wscale ? *reinterpret_cast<const f32x4*>(p.wscale + nw0 + ch) : f32x4{1, 1, 1, 1};
    const f32x4 bi = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + nw0 + ch) : f32x4{0, 0, 0, 0};
    const float ks = which == 1 ? h.k_scale : 1.0f;
    const int64_t pad = which == 0 ? h.q_pad : h.k_pad;
    uint16_t* base = (which == 0 ? h.q : h.k) + (bh * pad + (which == 0 ? h.q_row0 : h.row0)) * 64 + ch;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // a row past M stores into the last row, with the last row's bits (its A row was read as the last row's)
        const int r = r0 + 4 * i, t = min(tok0 + r, last);
        f32x4 x = *reinterpret_cast<const f32x4*>(st + r * ld + ch);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            x[e] = (x[e] * sc[e] + bi[e]) * ks;
        *reinterpret_cast<u32x2*>(base + int64_t(t) * 64) = u32x2{pack_x2(x[0], x[1], F16), pack_x2(x[2], x[3], F16)};
    }
}

// Stream-K state of a persistent launch: the tail tiles are split into k ranges over the whole grid; a workgroup
// whose range ends inside a tile publishes its partial accumulators, the workgroup holding the tile's last k steps
// adds them (in a fixed order) and runs the epilogue.
struct SkP {
    float* ws;          // [2 grid][threads * accumulators] partials, two slots a workgroup (its first and last tile)
    uint32_t* flags;    // [2 grid]: set to epoch when the slot holds this launch's partial
    uint32_t* err;      // host-visible word: set to 1 when a wait for a partial gave up (the host reports it)
    uint32_t epoch;
    uint32_t polls;     // bound of a wait for a partial's flag (polls of ~128 cycles each)
    uint32_t total;     // tiles over both problems
    uint32_t dp;        // tiles done whole, round robin over the grid (a multiple of it)
    uint32_t kt;        // k steps a tile
    uint64_t units;     // (total - dp) * kt: the tail's k steps, split evenly over the grid
};

// Stream-K tail partition: range i (a virtual workgroup index) holds tail units [units i / grid, units (i+1) / grid).
// Its segment of tail tile tt publishes to slot 2 i (its first tile) or 2 i + 1 (its last).
__device__ inline uint64_t sk_begin(const SkP& sk, uint32_t i) { return sk.units * i / gridDim.x; }
__device__ inline int sk_slot(const SkP& sk, uint32_t i, uint64_t tt)
{
    return int(2 * i + (tt == sk_begin(sk, i) / sk.kt ? 0 : 1));
}
// The physical workgroup of virtual index i: virtual order gives each XCD (workgroups w = x mod 8) a contiguous run
// of tail tiles, which then share panels in its L2.
__device__ inline uint32_t sk_phys(uint32_t i)
{
    const uint32_t per = gridDim.x / 8;
    return gridDim.x % 8 ? i : (i % per) * 8 + i / per;
}

// XCD-aware order of n tiles (n a multiple of 8): round-robin dispatch puts workgroup i on XCD i % 8; give each
// XCD a contiguous run of tiles.
__device__ inline uint32_t xcd_order(uint32_t t, uint32_t n) { return n % 8 ? t : (t % 8) * (n / 8) + t / 8; }

// Tile t of a launch (problem 0's tiles, then problem 1's; batch-major within a problem) -> problem, batch and tile
// coordinates, grouped 8 token tiles at a time so consecutive tiles share weight columns.
__device__ inline const GemmP& locate(const GemmG& G, uint32_t t, uint32_t& z, uint32_t& tm, uint32_t& tn)
{
    const bool second = t >= G.tiles0;
    const GemmP& p = G.g[second];
    const uint32_t per = p.tiles_m * p.tiles_n;
    uint32_t pid = second ? t - G.tiles0 : t;
    z = pid / per;
    pid %= per;
    const uint32_t GM = 8, in_group = GM * p.tiles_n;
    const uint32_t first_m = (pid / in_group) * GM;
    const uint32_t gsize = min(p.tiles_m - first_m, GM);
    tm = first_m + (pid % in_group) % gsize;
    tn = (pid % in_group) / gsize;
    return p;
}

// 16-byte accumulator groups a stream-K fixup pass brings into LDS: the largest divisor of the qn groups that fits
// the cap the operand buffers allow.
constexpr int fixup_groups(int qn, int cap)
{
    int q = qn < cap ? qn : cap;
    while (qn % q)
        --q;
    return q;
}

// The norm epilogues of a wave's staged slice (32 rows x 96 channels from chw, row stride ld floats; rows tok0 .. of
// the padded grid, M = (h + 2) pw of them). v = the conv's value + bias; EK_NORM: y = n(v) (16-bit) where n(v) =
// silu(v rsqrt(mean(v^2) + 1e-24 / C) g) over the row's C channels, the VAE's RMS norm + SiLU (engine.cpp:725-727);
// EK_RMWN: y = v or y += v (fp32) and norm_out = n(y) (16-bit). Normed ring rows are zero. 8 lanes a row (4 channels of
// each 32-channel third), 8 rows an instruction, 4 rows a lane; a row's sum of squares over its 8 lanes by DPP. With
// C = 192 (PAIR) the row's other 96 channels are the partner wave's (wave ^ 1): the partial sums meet in xch (32
// floats a wave) across one barrier that waits for LDS operations only, not for the stores in flight.
template <int EKE, bool PAIR, bool H>
__device__ inline void epi_norm_silu(const GemmP& p, const float* st, int ld, int tok0, int chw, int lane, float* xch,
                                     int wave)
{
    constexpr float kInvC = PAIR ? 1.0f / 192.0f : 1.0f / 96.0f;
    const int c = lane % 8, r0 = lane / 8;
    f32x4 bias[3], gm[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        bias[j] = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + chw + 32 * j + 4 * c) : f32x4{0, 0, 0, 0};
        gm[j] = *reinterpret_cast<const f32x4*>(p.norm_g + chw + 32 * j + 4 * c);
    }
    const uint32_t pw = p.conv_pw, gh = p.M / pw;
    const bool add = EKE == EK_RMWN && p.epi == MK_EPI_ADD;
    f32x4 v[4][3];
    if (add) {
        // the residual rows first, all in flight together (rows past M read the last row and are not stored)
        const float* x = static_cast<const float*>(p.c) + chw;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 3; ++j)
                v[i][j] = *reinterpret_cast<const f32x4*>(x + int64_t(min(tok0 + r0 + 8 * i, int(p.M) - 1)) * p.ldc +
                                                          32 * j + 4 * c);
    }
    float ss[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = r0 + 8 * i;
        ss[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(st + row * ld + 32 * j + 4 * c);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[i][j][e] = add ? v[i][j][e] + (a[e] + bias[j][e]) : a[e] + bias[j][e];
                ss[i] = fmaf(v[i][j][e], v[i][j][e], ss[i]);
            }
        }
        ss[i] = oct_sum(ss[i]);
    }
    if constexpr (PAIR) {
        if (c == 0)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                xch[wave * 32 + r0 + 8 * i] = ss[i];
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(0xc07f); // lgkmcnt(0): this wave's LDS writes done
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ss[i] += xch[(wave ^ 1) * 32 + r0 + 8 * i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int row = r0 + 8 * i, t = tok0 + row;
        // (v_rsq_f32: the mean of squares plus 1e-24 / C is never a denormal)
        const float sc = __builtin_amdgcn_rsqf(ss[i] * kInvC + 1e-24f * kInvC);
        // (tiles over the pixels hold pixel rows only; else the row's ring test, an integer division). Ring rows are
        // zeroed by a mask on the bits, so a ring value that is not finite still comes out 0.
        uint32_t keep = ~0u;
        if (!p.conv_w) {
            const uint32_t gy = uint32_t(t) / pw, gx = uint32_t(t) - gy * pw;
            keep = gy >= 1 && gy + 1 < gh && gx >= 1 && gx + 1 < pw ? ~0u : 0u;
        }
        uint32_t o[3][2];
#pragma unroll
        for (int j = 0; j < 3; ++j) {
            float u[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                u[e] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, silu_f(v[i][j][e] * sc * gm[j][e])) & keep);
            o[j][0] = pack16<H>(u[0], u[1]);
            o[j][1] = pack16<H>(u[2], u[3]);
        }
        if (t < int(p.M)) {
            uint16_t* y = EKE == EK_RMWN ? p.norm_out + int64_t(t) * p.norm_ld + chw + 4 * c
                                         : static_cast<uint16_t*>(p.c) + int64_t(t) * p.ldc + chw + 4 * c;
            float* x = static_cast<float*>(p.c) + int64_t(t) * p.ldc + chw + 4 * c;
#pragma unroll
            for (int j = 0; j < 3; ++j) {
                if (EKE == EK_RMWN && !p.norm_only)
                    *reinterpret_cast<f32x4*>(x + 32 * j) = v[i][j];
                *reinterpret_cast<u32x2*>(y + 32 * j) = u32x2{o[j][0], o[j][1]};
            }
        }
    }
}

// One tile's k steps [kb, ke): the pipelined main loop, then either the partial published to stream-K slot
// `publish`, or the partials of the tile's other ranges (virtual indices fix_lo .. fix_hi except `self`, tail tile
// tt) added in index order, and the epilogue.
template <int BM, int BN, bool kF8, int EK, int NW>
__device__ __forceinline__ void gemm_tile(const GemmP& p, uint32_t z, uint32_t tm, uint32_t tn, int kb, int ke,
                                          uint16_t* smem, const SkP* sk, int publish, int fix_lo = 0,
                                          int fix_hi = -1, int self = -1, uint64_t tt = 0)
{
    static_assert(((EK & 7) != EK_HEADS && (EK & 7) != EK_GLU) || !(EK & EK_CONV),
                  "a convolution has no heads or GLU epilogue");
    constexpr bool kConv = (EK & EK_CONV) != 0, kConvQ = (EK & EK_CONVQ) != 0, kF16 = (EK & EK_F16) != 0;
    constexpr bool kDeep = (EK & EK_DEEP) != 0;
    static_assert(!kDeep || (NW == 4 && BN == 128 && !kF8 && !kConv), "deep stages: 4-wave 128-channel tiles");
    constexpr int NSTG = kDeep ? (BM == 128 ? 4 : 3) : 2; // LDS stages of the operand tiles
    constexpr int EKE = EK & 7;                 // the epilogue kind
    constexpr int NT = 64 * NW;                 // threads
    // waves: 2 along channels x NW/2 along tokens; the 96-channel tiles 1 x NW (a wave holds whole rows)
    constexpr int WCH = BN == 96 ? 1 : 2;
    constexpr int WM = BM / (NW / WCH);         // tokens per wave
    constexpr int WC = BN / WCH;                // channels per wave
    // 8-wave tiles run v_mfma_f32_16x16x32_bf16 (16 x 16 output blocks, 32-deep substeps: 3-4% faster than the
    // 32 x 32 x 16 form on the step's shapes, where the matrix cores are held by the power limit; bit-identical
    // results), 4-wave tiles v_mfma_f32_32x32x16_bf16, except the 96-channel ones (six 16-row blocks a wave).
    constexpr bool M16 = NW == 8 || BN == 96;
    constexpr int MB = M16 ? 16 : 32;
    constexpr int TB = WM / MB, CB = WC / MB;   // MFMA blocks per wave along tokens / channels
    constexpr int RA = BM * 8 / NT;             // direct-load rounds for the activation tile (64 chunks per wave)
    constexpr int RW = BN * 8 / NT;             // ... for a bf16 weight tile
    constexpr int LW = BN * 4 / NT;             // 16-byte fp8 weight chunks per thread (register staged)
    constexpr int ND = RA + (kF8 ? 0 : RW);     // direct loads a thread issues per k step
    constexpr int LDW = WC + 4;                 // epilogue staging: a wave's 32 tokens x WC channels, padded rows
    uint16_t(*sW)[BN * 64] = reinterpret_cast<uint16_t(*)[BN * 64]>(smem);
    uint16_t(*sA)[BM * 64] = reinterpret_cast<uint16_t(*)[BM * 64]>(smem + NSTG * BN * 64);

    // the wave index is uniform: readfirstlane keeps it (and the LDS bases of the direct loads) in scalar registers
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = WCH == 2 ? wave & 1 : 0, wm = WCH == 2 ? wave >> 1 : wave;
    int m0 = int(tm) * BM;
    if constexpr (kConv) {
        if (p.conv_w) {
            const int y = m0 / int(p.conv_w), x = m0 - y * int(p.conv_w);
            m0 = (y + 1) * int(p.conv_pw) + x + 1;
        }
    }
    const int n0 = int(tn) * BN;

    // Direct loads: wave w's round i fills LDS chunks P = (i * NW + w) * 64 + lane of the tile; chunk P holds
    // row P / 8 and logical k-chunk swz_chunk(row, P % 8), so the lane loads that one. Buffer loads: the resource
    // spans the tile's rows (base = its first row), the lane's 32-bit byte offset selects row and chunk, the k
    // offset is a scalar; activation rows past M read the last row.
    const char* gA = reinterpret_cast<const char*>(p.a + int64_t(z) * p.sa + int64_t(m0) * p.lda);
    // GLU: the tile computes output channels tn BN/2 .. + BN/2; each wave's WC rows are WC/2 rows of the first part
    // and the same channels' rows of the second part (F rows further on), so one lane's accumulator blocks cb and
    // cb + CB/2 hold the two operands of the same output. wrow: the tile's local weight row -> row offset from gW.
    constexpr bool kGlu = EKE == EK_GLU;
    const int nw0 = kGlu ? int(tn) * (BN / 2) : n0;
    const char* gW = static_cast<const char*>(p.w) + int64_t(nw0) * p.K * (kF8 ? 1 : 2);
    auto wrow = [&](int r) -> int {
        if constexpr (kGlu)
            return (r / WC) * (WC / 2) + (r % WC) % (WC / 2) + ((r % WC) >= WC / 2 ? int(p.glu_f) : 0);
        else
            return r;
    };
    // a convolution's tile reads up to 2 (w + 2) + 2 rows past its own (the taps' shifts), all inside the input
    const BufRes rsA = buf_res(
        gA, uint32_t(kConv ? (min(int(p.M) - m0, BM) + 2 * int64_t(p.conv_pw) + 2) * p.lda * 2
                           : ((min(int(p.M) - m0, BM) - 1) * int64_t(p.lda) + p.K) * 2));
    // A's byte offset of k step kt. Convolution: k = tap * lda + channel, tap = 3 dy + dx reads the row shifted by
    // dy (w + 2) + dx; the k step lies inside one tap (lda is a multiple of 64). tap = kt / tpt by multiply-shift
    // (exact for kt < 2^16 / tpt), dy = tap / 3 likewise (exact for tap < 9).
    auto koffA = [&](int kt) -> uint32_t {
        if constexpr (kConv) {
            const uint32_t tap = (uint32_t(kt) * p.conv_inv) >> 16;
            const uint32_t dy = (tap * 21846u) >> 16, dx = tap - 3 * dy;
            const uint32_t ch = (uint32_t(kt) - tap * p.conv_tpt) * BK;
            return ((dy * p.conv_pw + dx) * uint32_t(p.lda) + ch) * 2;
        } else {
            return uint32_t(kt * BK * 2);
        }
    };
    const BufRes rsW = buf_res(gW, uint32_t((kGlu ? int64_t(p.glu_f) + BN / 2 : int64_t(BN)) * p.K * 2));
    uint32_t oa[RA], kq[kConvQ ? RA : 1];
#pragma unroll
    for (int i = 0; i < RA; ++i) {
        const int P = (i * NW + wave) * 64 + lane, row = P >> 3, kc = swz_chunk(row, P & 7);
        oa[i] = uint32_t(min(row, int(p.M) - 1 - m0) * int(p.lda) + (kConvQ ? 0 : kc * 8)) * 2;
        if constexpr (kConvQ)
            kq[i] = uint32_t(kc);
    }
    // EK_CONVQ: the lane's A byte offset (beyond its row) for chunk kq[i] of k step kt: global chunk q = 8 kt + kc,
    // tap = q / cq, channel chunk q - tap cq (multiply-shift, exact for q < 2^16 / cq: cq <= 64); the tail past
    // 9 cq (zero weights) reads tap 8's rows
    auto koffq = [&](int kt, int i) -> uint32_t {
        const uint32_t q = uint32_t(kt) * 8 + kq[i];
        uint32_t tap = (q * p.conv_inv) >> 16;
        const uint32_t ch8 = q - tap * p.conv_tpt;
        tap = min(tap, 8u);
        const uint32_t dy = (tap * 21846u) >> 16, dx = tap - 3 * dy;
        return ((dy * p.conv_pw + dx) * uint32_t(p.lda) + ch8 * 8) * 2;
    };
    uint32_t ow[kF8 ? 1 : RW];
    const uint8_t* gw8[kF8 ? LW : 1];
    if constexpr (!kF8) {
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int P = (i * NW + wave) * 64 + lane, row = P >> 3, kc = swz_chunk(row, P & 7);
            ow[i] = uint32_t(wrow(row) * int(p.K) + kc * 8) * 2;
        }
    } else {
#pragma unroll
        for (int i = 0; i < LW; ++i) {
            const int c = tid + NT * i, row = c >> 2, kc = c & 3;
            gw8[i] = reinterpret_cast<const uint8_t*>(gW) + int64_t(wrow(row)) * p.K + kc * 16;
        }
    }
    u32x4 rw[kF8 ? LW : 1];
    // direct load i (activation rounds first, then bf16 weight rounds) of k step kt into buffer buf
    auto dma1 = [&](int kt, int buf, int i) {
        if (i < RA) {
            if constexpr (kConvQ)
                buf_load_lds16(rsA, (lds_void*)&sA[buf][(i * NW + wave) * 64 * 8], oa[i] + koffq(kt, i), 0);
            else
                buf_load_lds16(rsA, (lds_void*)&sA[buf][(i * NW + wave) * 64 * 8], oa[i], koffA(kt));
        }
        else if constexpr (!kF8)
            buf_load_lds16(rsW, (lds_void*)&sW[buf][((i - RA) * NW + wave) * 64 * 8], ow[i - RA],
                           uint32_t(kt * BK * 2));
    };
    auto load_f8 = [&](int kt) {
        if constexpr (kF8) {
#pragma unroll
            for (int i = 0; i < LW; ++i)
                rw[i] = *reinterpret_cast<const u32x4*>(gw8[i] + kt * BK);
        }
    };
    auto issue = [&](int kt, int buf) {
#pragma unroll
        for (int i = 0; i < ND; ++i)
            dma1(kt, buf, i);
        load_f8(kt);
    };
    auto commit_f8 = [&](int buf) {
        if constexpr (kF8) {
#pragma unroll
            for (int i = 0; i < LW; ++i) {
                const int c = tid + NT * i, row = c >> 2, kc = c & 3;
                u32x4 lo, hi;
                f8x16_to_bf16(rw[i], lo, hi);
                *reinterpret_cast<u32x4*>(&sW[buf][swz(row, 2 * kc)]) = lo;
                *reinterpret_cast<u32x4*>(&sW[buf][swz(row, 2 * kc + 1)]) = hi;
            }
        }
    };

    std::conditional_t<M16, f32x4, f32x16> acc[CB][TB];
#pragma unroll
    for (int i = 0; i < CB; ++i)
#pragma unroll
        for (int j = 0; j < TB; ++j)
            acc[i][j] = {};

    // v_mfma_f32_32x32x16_bf16: lane (r32, hk) supplies row r32 of a 32-row block and k values 8 hk .. 8 hk + 7 of
    // a 16-wide substep, and holds output rows (channels) 8 i + 4 hk .. + 3 (i < 4) of column r32 (token).
    // v_mfma_f32_16x16x32_bf16: lane (r16, g4) supplies row r16 of a 16-row block and k values 8 g4 .. 8 g4 + 7 of
    // a 32-wide substep, and holds output rows 4 g4 .. 4 g4 + 3 of column r16.
    const int r32 = lane & 31, hk = lane >> 5, r16 = lane & 15, g4 = lane >> 4;
    // fragment j of a substep in first-use order (the MFMAs run channel-block-major): weight block 0, the token
    // blocks, then weight blocks 1 ..
    // the matrix-core products in the operands' type (the fragments are 16-bit lanes either way)
    auto mfma16 = [](const bf16x8& w, const bf16x8& a, const f32x4& c) -> f32x4 {
        if constexpr (kF16)
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8v, w), __builtin_bit_cast(f16x8v, a),
                                                          c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, a, c, 0, 0, 0);
    };
    auto mfma32 = [](const bf16x8& w, const bf16x8& a, const f32x16& c) -> f32x16 {
        if constexpr (kF16)
            return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8v, w), __builtin_bit_cast(f16x8v, a),
                                                          c, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_32x32x16_bf16(w, a, c, 0, 0, 0);
    };
    auto frag = [&](int buf, int ks, int j, bf16x8(&wf)[CB], bf16x8(&af)[TB]) {
        const int kc = ks * 2 + hk;
        if (j == 0 || j > TB) {
            const int cb = j == 0 ? 0 : j - TB;
            wf[cb] = *reinterpret_cast<const bf16x8*>(&sW[buf][swz(wn * WC + cb * 32 + r32, kc)]);
        } else {
            af[j - 1] = *reinterpret_cast<const bf16x8*>(&sA[buf][swz(wm * WM + (j - 1) * 32 + r32, kc)]);
        }
    };
    // 16 x 16 x 32 fragments: weight block cb, token block tb of substep ks
    auto rdw = [&](int buf, int ks, int cb, bf16x8(&wf)[CB]) {
        wf[cb] = *reinterpret_cast<const bf16x8*>(&sW[buf][swz(wn * WC + cb * 16 + r16, ks * 4 + g4)]);
    };
    auto rda = [&](int buf, int ks, int tb, bf16x8(&af)[TB]) {
        af[tb] = *reinterpret_cast<const bf16x8*>(&sA[buf][swz(wm * WM + tb * 16 + r16, ks * 4 + g4)]);
    };
    // 128-channel tiles (4 waves, one a SIMD) with bf16 weights stage the operands through registers: a thread
    // loads its ND 16-byte chunks of a k step into registers (buffer loads) and later writes each to the LDS chunk a
    // direct load would have filled (measured: 6-13% faster than direct loads there on K of 3072-5120; 2-8% slower
    // for the 8-wave 256-wide tiles and 5-15% for 64-channel tiles, which keep the direct loads). fp8 weights: the
    // activation chunks go by direct load, the weight chunks through registers (converted to bf16, commit_f8).
    constexpr bool kStage = !kF8 && NW == 4 && BN == 128 && !kDeep;
    u32x4 stg[kStage ? ND : 1];
    auto gload = [&](int kt, int i) {
        if constexpr (kStage) {
            if (i < RA)
                stg[i] = kConvQ ? buf_load16(rsA, oa[i] + koffq(kt, i), 0) : buf_load16(rsA, oa[i], koffA(kt));
            else
                stg[i] = buf_load16(rsW, ow[i - RA], uint32_t(kt * BK * 2));
        }
    };
    auto swrite = [&](int buf, int i) {
        if constexpr (kStage) {
            if (i < RA)
                *reinterpret_cast<u32x4*>(&sA[buf][((i * NW + wave) * 64 + lane) * 8]) = stg[i];
            else
                *reinterpret_cast<u32x4*>(&sW[buf][(((i - RA) * NW + wave) * 64 + lane) * 8]) = stg[i];
        }
    };
    // One substep's MFMAs from fragments wf / af in a fixed order (every instruction fenced): one read of the next
    // substep's fragments (buffer nbuf, substep nks; none if nks < 0) after each of the first MFMAs, then operand
    // moves for later k steps likewise: loads g0 .. g1 - 1 of step gkt (staged: into registers; otherwise direct
    // loads into buffer gbuf) and, staged only, register writes w0 .. w1 - 1 into buffer wbuf (what is left after the
    // last MFMA follows it). (The ranges are compile-time: register and offset array indices then are constants.)
    auto group = [&](const bf16x8(&wf)[CB], const bf16x8(&af)[TB], int nbuf, int nks, bf16x8(&nwf)[CB],
                     bf16x8(&naf)[TB], int gkt, int gbuf, auto g0_c, auto g1_c, int wbuf, auto w0_c, auto w1_c) {
        constexpr int g0 = decltype(g0_c)::value, g1 = decltype(g1_c)::value;
        constexpr int w0 = decltype(w0_c)::value, w1 = decltype(w1_c)::value;
        auto move = [&](int i) {
            if (g0 + i < g1) {
                if constexpr (!kStage)
                    dma1(gkt, gbuf, g0 + i);
                else
                    gload(gkt, g0 + i);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (w0 + i < w1) {
                swrite(wbuf, w0 + i);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
#pragma unroll
        for (int i = 0; i < CB * TB; ++i) {
            const int cb = i / TB, tb = i % TB;
            if constexpr (!M16)
                acc[cb][tb] = mfma32(wf[cb], af[tb], acc[cb][tb]);
            __builtin_amdgcn_sched_barrier(0);
            if (nks >= 0 && i < CB + TB) {
                frag(nbuf, nks, i, nwf, naf);
                __builtin_amdgcn_sched_barrier(0);
            }
            move(i);
        }
        // narrow tiles have fewer MFMAs a substep than reads or moves
        if (nks >= 0) {
#pragma unroll
            for (int j = CB * TB; j < CB + TB; ++j)
                frag(nbuf, nks, j, nwf, naf);
        }
#pragma unroll
        for (int i = CB * TB; i < (g1 - g0 > w1 - w0 ? g1 - g0 : w1 - w0); ++i)
            move(i);
    };

    // 16 x 16 x 32 substep (32 MFMAs for a 64 x 128 wave tile): the weight fragments are single-buffered, each
    // next-substep fragment read into its register right after the MFMA that last uses it; the token fragments of
    // the next substep go to the other buffer (naf) with the first channel block; direct loads g0 .. g1 - 1 of step
    // gkt into buffer gbuf follow the MFMAs one each.
    auto group16 = [&](bf16x8(&wf)[CB], const bf16x8(&af)[TB], int nbuf, int nks, bf16x8(&naf)[TB], int gkt,
                       int gbuf, auto g0_c, auto g1_c) {
        constexpr int g0 = decltype(g0_c)::value, g1 = decltype(g1_c)::value;
#pragma unroll
        for (int i = 0; i < CB * TB; ++i) {
            const int cb = i / TB, tb = i % TB;
            if constexpr (M16)
                acc[cb][tb] = mfma16(wf[cb], af[tb], acc[cb][tb]);
            __builtin_amdgcn_sched_barrier(0);
            if (nks >= 0 && cb == 0) {
                rda(nbuf, nks, tb, naf);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (nks >= 0 && tb == TB - 1) {
                rdw(nbuf, nks, cb, wf);
                __builtin_amdgcn_sched_barrier(0);
            }
            if (g0 + i < g1) {
                dma1(gkt, gbuf, g0 + i);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int i = CB * TB; i < g1 - g0; ++i)
            dma1(gkt, gbuf, g0 + i);
    };

    using C0 = std::integral_constant<int, 0>;
    using CH = std::integral_constant<int, ND / 2>;
    using CN = std::integral_constant<int, ND>;
    bf16x8 wf0[CB], af0[TB], wf1[CB], af1[TB]; // (16 x 16 x 32: wf0 is the single weight buffer)
    if constexpr (kDeep) {
        // steps kb .. kb + NSTG - 2 into stages 0 .. NSTG - 2 (past-the-end steps clamped: a reload of the last);
        // step kb landed (this wave's later loads may stay in flight), then every wave's
        static_assert(NSTG == 3 || NSTG == 4, "deep stages: 3 or 4");
        issue(min(kb, ke - 1), 0);
        issue(min(kb + 1, ke - 1), 1);
        if constexpr (NSTG == 4)
            issue(min(kb + 2, ke - 1), 2);
        __builtin_amdgcn_s_waitcnt(waitcnt_bits((NSTG - 2) * ND, 0));
        __builtin_amdgcn_s_barrier();
    } else if constexpr (!kStage) {
        // Software pipeline over k steps of four 16-wide substeps: step t is in LDS buffer t & 1; step t + 1 lands
        // in the other buffer during step t (the first half of its direct loads goes out with the last substep of
        // step t - 1, right after the barrier frees the buffer, the second half with the first substep of step t);
        // each substep reads the next one's fragments. Past-the-end steps are clamped (they reload the last step).
        issue(kb, 0);
        commit_f8(0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // step kb + 1: 32 x 32 x 16, its first half (each step issues the next one's second half); 16 x 16 x 32,
        // all of it (each step issues the whole step after next)
#pragma unroll
        for (int i = 0; i < (M16 ? ND : ND / 2); ++i)
            dma1(min(kb + 1, ke - 1), 1, i);
        load_f8(min(kb + 1, ke - 1));
    } else {
        // Software pipeline over k steps of four 16-wide substeps: step t is in LDS buffer t & 1. During step t the
        // registers take step t + 2 (first half with substep 0, second half with substep 1) and go to LDS once that
        // buffer is free: the first half with substep 3 (after the barrier that ends the reads of step t), the
        // second half with substep 0 of step t + 1; a load has three substeps to arrive. The barrier itself waits
        // for the LDS writes only, not for loads in flight. Past-the-end steps are clamped (they reload the last
        // step into a buffer nobody reads any more).
#pragma unroll
        for (int i = 0; i < ND; ++i)
            gload(kb, i);
#pragma unroll
        for (int i = 0; i < ND; ++i)
            swrite(0, i);
#pragma unroll
        for (int i = 0; i < ND; ++i)
            gload(min(kb + 1, ke - 1), i);
        __syncthreads();
#pragma unroll
        for (int i = 0; i < ND / 2; ++i)
            swrite(1, i);
    }
    if constexpr (M16) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
            rdw(0, 0, cb, wf0);
#pragma unroll
        for (int tb = 0; tb < TB; ++tb)
            rda(0, 0, tb, af0);
    } else {
#pragma unroll
        for (int j = 0; j < CB + TB; ++j)
            frag(0, 0, j, wf0, af0);
    }
    // one k step from buffer `buf` (a constant: the loop is unrolled by two, so every LDS address is a register
    // base plus an immediate offset)
    auto step = [&](int kt, auto buf_c) {
        constexpr int buf = decltype(buf_c)::value;
        if constexpr (M16) {
            // two 32-deep substeps: the second substep's fragments are read during the first; after the barrier
            // (step kt + 1 complete in the other buffer, every wave done with this one) the second substep reads
            // the next step's first fragments and loads step kt + 2 into this buffer
            group16(wf0, af0, buf, 1, af1, 0, 0, C0{}, C0{});
            commit_f8(buf ^ 1);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            load_f8(min(kt + 2, ke - 1));
            group16(wf0, af1, buf ^ 1, 0, af0, min(kt + 2, ke - 1), buf, C0{}, CN{});
        } else if constexpr (kDeep) {
            // step kt in stage buf; its first three substeps issue step kt + NSTG - 1 into the stage step kt - 1
            // left (freed by the previous barrier); then step kt + 1 landed (this wave's loads of the steps after it
            // may stay in flight), the barrier (every wave's loads of it visible, every wave done reading stage buf),
            // and the last substep reads step kt + 1's first fragments
            constexpr int lb = (buf + NSTG - 1) % NSTG, nb = (buf + 1) % NSTG;
            const int kl = min(kt + NSTG - 1, ke - 1);
            group(wf0, af0, buf, 1, wf1, af1, kl, lb, C0{}, CH{}, 0, C0{}, C0{});
            group(wf1, af1, buf, 2, wf0, af0, kl, lb, CH{}, CN{}, 0, C0{}, C0{});
            group(wf0, af0, buf, 3, wf1, af1, 0, 0, C0{}, C0{}, 0, C0{}, C0{});
            __builtin_amdgcn_s_waitcnt(waitcnt_bits((NSTG - 2) * ND, 0));
            __builtin_amdgcn_s_barrier();
            group(wf1, af1, nb, 0, wf0, af0, 0, 0, C0{}, C0{}, 0, C0{}, C0{});
        } else if constexpr (!kStage) {
            group(wf0, af0, buf, 1, wf1, af1, min(kt + 1, ke - 1), buf ^ 1, CH{}, CN{}, 0, C0{}, C0{});
            group(wf1, af1, buf, 2, wf0, af0, 0, 0, C0{}, C0{}, 0, C0{}, C0{});
            group(wf0, af0, buf, 3, wf1, af1, 0, 0, C0{}, C0{}, 0, C0{}, C0{});
            // step kt + 1 complete in the other buffer, every wave done reading this one
            commit_f8(buf ^ 1);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            load_f8(min(kt + 2, ke - 1));
            group(wf1, af1, buf ^ 1, 0, wf0, af0, min(kt + 2, ke - 1), buf, C0{}, CH{}, 0, C0{}, C0{});
        } else {
            const int k2 = min(kt + 2, ke - 1);
            // substep 0: second half of step kt + 1 to LDS, first half of step kt + 2 into registers
            group(wf0, af0, buf, 1, wf1, af1, k2, 0, C0{}, CH{}, buf ^ 1, CH{}, CN{});
            group(wf1, af1, buf, 2, wf0, af0, k2, 0, CH{}, CN{}, 0, C0{}, C0{});
            group(wf0, af0, buf, 3, wf1, af1, 0, 0, C0{}, C0{}, 0, C0{}, C0{});
            // step kt + 1 complete in the other buffer, every wave done reading this one
            __syncthreads();
            group(wf1, af1, buf ^ 1, 0, wf0, af0, 0, 0, C0{}, C0{}, buf, C0{}, CH{});
        }
    };
    int kt = kb;
    if constexpr (kDeep) {
        // unrolled by NSTG: step kb + j of each round in stage j (constant LDS offsets)
        for (; kt + NSTG - 1 < ke; kt += NSTG) {
            step(kt, std::integral_constant<int, 0>{});
            step(kt + 1, std::integral_constant<int, 1>{});
            step(kt + 2, std::integral_constant<int, 2>{});
            if constexpr (NSTG == 4)
                step(kt + 3, std::integral_constant<int, 3 % NSTG>{});
        }
        if (kt < ke)
            step(kt, std::integral_constant<int, 0>{});
        if (kt + 1 < ke)
            step(kt + 1, std::integral_constant<int, 1>{});
        if constexpr (NSTG == 4)
            if (kt + 2 < ke)
                step(kt + 2, std::integral_constant<int, 2>{});
    } else {
        for (; kt + 1 < ke; kt += 2) {
            step(kt, std::integral_constant<int, 0>{});
            step(kt + 1, std::integral_constant<int, 1>{});
        }
        if (kt < ke)
            step(kt, std::integral_constant<int, 0>{});
    }
    __builtin_amdgcn_s_waitcnt(0); // the last (unused) prefetch must land before the LDS is reused
    __syncthreads();

    // ---- stream-K: publish this range's partial, or add the earlier ranges' partials ----
    constexpr int NACC = CB * TB * (M16 ? 4 : 16);
    // The workspace is uncached (not held in any XCD's L2): a partial is plain 16-byte stores, complete at the memory
    // once acknowledged; the flag store follows every wave's acknowledgements. Slot layout: 16-byte groups
    // q = 4 * block + j / 4 of the accumulators as [q][thread][4 floats], so one group of a wave is 1 KB contiguous
    // (whole-line writes; the fixup's direct-to-LDS loads take it whole).
    if (publish >= 0) {
        f32x4* w = reinterpret_cast<f32x4*>(sk->ws + size_t(publish) * NT * NACC) + tid;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                if constexpr (M16)
                    w[size_t(cb * TB + tb) * NT] = acc[cb][tb];
                else
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        w[size_t((cb * TB + tb) * 4 + m) * NT] = f32x4{acc[cb][tb][4 * m], acc[cb][tb][4 * m + 1],
                                                                      acc[cb][tb][4 * m + 2], acc[cb][tb][4 * m + 3]};
            }
        __builtin_amdgcn_s_waitcnt(0); // every store acknowledged at the coherent level
        __syncthreads();
        if (tid == 0)
            __hip_atomic_store(sk->flags + publish, sk->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    if (fix_hi >= fix_lo) {
        if (tid == 0)
            for (int i = fix_lo; i <= fix_hi; ++i) {
                if (i == self)
                    continue;
                // every other range of the tile belongs to a workgroup dispatched before this one (the owner is
                // the tile's highest workgroup), and a workgroup publishes before it waits on anything; the bound
                // only keeps a broken launch from spinning forever
                const int slot = sk_slot(*sk, uint32_t(i), tt);
                bool seen = false;
                for (uint32_t n = 0; n < sk->polls; ++n) {
                    if (__hip_atomic_load(sk->flags + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == sk->epoch) {
                        seen = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(2);
                }
                // gave up: the tile is finished from what the slot holds, and the host turns the word into an error
                if (!seen)
                    __hip_atomic_store(sk->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        __syncthreads();
        // The other ranges' partials, in index order, each in passes of QL 16-byte groups: every wave streams its
        // own groups into its own region of the (now free) operand buffers with direct-to-LDS loads (device-coherent,
        // sc1), many in flight, then adds them from LDS.
        constexpr int QN = NACC / 4, QL = fixup_groups(QN, (2 * (BN + BM) * 64 * 2) / (NT * 16));
        const f32x4* mine = reinterpret_cast<const f32x4*>(smem) + wave * QL * 64 + lane;
        for (int i = fix_lo; i <= fix_hi; ++i) {
            if (i == self)
                continue;
            const float* src = sk->ws + size_t(sk_slot(*sk, uint32_t(i), tt)) * NT * NACC + 4 * tid;
#pragma unroll
            for (int pass = 0; pass < QN / QL; ++pass) {
#pragma unroll
                for (int q = 0; q < QL; ++q)
                    __builtin_amdgcn_global_load_lds(src + size_t(pass * QL + q) * NT * 4,
                                                     (lds_void*)(reinterpret_cast<f32x4*>(smem) + (wave * QL + q) * 64),
                                                     16, 0, 16 /* sc1 */);
                __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
                for (int q = 0; q < QL; ++q) {
                    const int g = pass * QL + q, b = M16 ? g : g / 4, j0 = M16 ? 0 : (g % 4) * 4;
                    const f32x4 v = mine[q * 64];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[b / TB][b % TB][j0 + e] += v[e];
                }
                __builtin_amdgcn_s_waitcnt(0); // this pass's LDS reads done before the next pass's loads land
            }
        }
        __syncthreads(); // the epilogue's staging regions span other waves' fixup regions
    }

    // ---- epilogue through LDS: per 32-token block, each wave stages its 32 x WC slice (fp32, padded rows) in a
    // region of its own, then reads it back with the lanes along the channels. A wave's LDS operations complete in
    // order, so the slices need no barrier (a __syncthreads() here would also wait for every global store in flight:
    // its release fence waits for vmcnt 0) ----
    float* st = reinterpret_cast<float*>(smem) + wave * 32 * LDW;
    const int64_t zc = int64_t(z) * p.sc;
    // the wave's 32-token slice s (token blocks s for 32 x 32 x 16, 2 s and 2 s + 1 for 16 x 16 x 32) into st
    auto stage = [&](int s) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            if constexpr (M16) {
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    *reinterpret_cast<f32x4*>(st + (16 * h + r16) * LDW + cb * 16 + 4 * g4) = acc[cb][2 * s + h];
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    *reinterpret_cast<f32x4*>(st + r32 * LDW + cb * 32 + 8 * i + 4 * hk) =
                        f32x4{acc[cb][s][4 * i], acc[cb][s][4 * i + 1], acc[cb][s][4 * i + 2], acc[cb][s][4 * i + 3]};
            }
        }
    };
    constexpr int NS = WM / 32, RB = TB / NS; // 32-token slices of a wave, MFMA token blocks a slice
    if constexpr (EKE == EK_GLU) {
        // out = silu(first) second (SwiGLU, swiglu_rows), first gelu_erf(second) (GEGLU, geglu_rows) or first +
        // second (a product split in two weight halves, MK_EPI_PAIR_SUM), computed
        // into blocks cb < CB/2 from blocks cb and cb + CB/2 (each with its rows' scale and bias), then stored as a
        // slice of WC/2 channels
        constexpr int CH2 = CB / 2, NQ = M16 ? 1 : 4; // groups of 4 consecutive channels a lane holds in a block
        const int oc0 = int(tn) * (BN / 2) + wn * (WC / 2);
        // one copy of the products for each kind (one branch a tile)
        auto glu = [&](auto kind_c) {
            constexpr int KIND = decltype(kind_c)::value; // 0 pair sum, 1 SwiGLU, 2 GEGLU
#pragma unroll
            for (int cb = 0; cb < CH2; ++cb)
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int c1 = oc0 + cb * MB + (M16 ? 4 * g4 : 8 * q + 4 * hk), c2 = c1 + int(p.glu_f);
                    const f32x4 s1 = p.wscale ? *reinterpret_cast<const f32x4*>(p.wscale + c1) : f32x4{1, 1, 1, 1};
                    const f32x4 s2 = p.wscale ? *reinterpret_cast<const f32x4*>(p.wscale + c2) : f32x4{1, 1, 1, 1};
                    const f32x4 b1 = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + c1) : f32x4{0, 0, 0, 0};
                    const f32x4 b2 = p.bias ? *reinterpret_cast<const f32x4*>(p.bias + c2) : f32x4{0, 0, 0, 0};
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float a = acc[cb][tb][4 * q + e] * s1[e] + b1[e];
                            const float g = acc[cb + CH2][tb][4 * q + e] * s2[e] + b2[e];
                            acc[cb][tb][4 * q + e] = KIND == 0   ? a + g
                                                     : KIND == 1 ? silu_f(a) * g
                                                                 : a * (0.5f * g * (1.0f + erf_fit(g * 0.70710678f)));
                        }
                }
        };
        if (p.epi == MK_EPI_PAIR_SUM)
            glu(std::integral_constant<int, 0>{});
        else if (p.epi == MK_EPI_SWIGLU)
            glu(std::integral_constant<int, 1>{});
        else
            glu(std::integral_constant<int, 2>{});
        constexpr int WH = WC / 2, LDH = WH + 4;
        float* sh = reinterpret_cast<float*>(smem) + wave * 32 * LDH;
        const EpiCh unit{f32x4{1, 1, 1, 1}, f32x4{0, 0, 0, 0}, f32x4{}, f32x4{}};
#pragma unroll
        for (int s2 = 0; s2 < NS; ++s2) {
#pragma unroll
            for (int cb = 0; cb < CH2; ++cb) {
                if constexpr (M16) {
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        *reinterpret_cast<f32x4*>(sh + (16 * h + r16) * LDH + cb * 16 + 4 * g4) = acc[cb][2 * s2 + h];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        *reinterpret_cast<f32x4*>(sh + r32 * LDH + cb * 32 + 8 * i + 4 * hk) =
                            f32x4{acc[cb][s2][4 * i], acc[cb][s2][4 * i + 1], acc[cb][s2][4 * i + 2],
                                  acc[cb][s2][4 * i + 3]};
                }
            }
            epi_slice<EK_STORE, WH>(p, sh, LDH, m0 + wm * WM + s2 * 32, oc0, lane, zc, unit);
        }
        return;
    }
    if constexpr (EKE == EK_NORM || EKE == EK_RMWN) {
        static_assert(kConv && kF16, "the norm epilogues follow half convolutions");
        // 96-channel tiles: a wave holds whole rows; 192-channel tiles: a row's channels are a wave pair's
        static_assert(WC == 96 && M16 && (BN == 96 || BN == 192), "the norm epilogues take 96- or 192-channel rows");
        constexpr bool PAIR = BN == 192;
        // the exchange of partial sums (192: two slices' worth, by parity) after the staging regions
        static_assert(!PAIR || (NW * 32 * LDW + 2 * NW * 32) * 4 <= 2 * (BN + BM) * 64 * 2, "exchange area in LDS");
        float* xch = reinterpret_cast<float*>(smem) + NW * 32 * LDW;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            stage(s);
            // (a convolution's 16-bit grids are IEEE half, like its operands)
            epi_norm_silu<EKE, PAIR, true>(p, st, LDW, m0 + wm * WM + s * 32, wn * WC, lane, xch + (s & 1) * NW * 32,
                                           wave);
        }
        return;
    }
    if constexpr (EKE == EK_HEADS) {
        // the heads epilogue is large: one copy of it for each output type and RoPE mode (a launch runs one) in a
        // rolled loop over the 32-token slices, which always stages slice 0 of the accumulators and then rotates the
        // next slice into its place (static register indices, so the accumulators stay in registers)
#pragma unroll 1
        for (int s = 0; s < NS; ++s) {
            stage(0);
            with_flag(p.hp.f16, [&](auto h_c) {
                constexpr bool H = decltype(h_c)::value;
                const int tok = m0 + wm * WM + s * 32, nw = n0 + wn * WC;
                if constexpr (WC == 64)
                    epi_heads64<H>(p, st, LDW, tok, nw, lane, z);
                else if (p.hp.rope_mode == 2)
                    epi_heads<H, 2>(p, st, LDW, tok, nw, lane, z);
                else if (p.hp.rope_mode == 1)
                    epi_heads<H, 1>(p, st, LDW, tok, nw, lane, z);
                else
                    epi_heads<H, 0>(p, st, LDW, tok, nw, lane, z);
            });
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                for (int t = 0; t + RB < TB; ++t)
                    acc[cb][t] = acc[cb][t + RB];
        }
        return;
    }
    if constexpr (WC == 96) {
        // 192- and 96-channel tiles: the wave's 96 staged channels go out as three 32-channel slices
        EpiCh kch[3];
#pragma unroll
        for (int j = 0; j < 3; ++j)
            kch[j] = epi_channels(p, n0 + wn * WC + 32 * j + 4 * (lane % 8));
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            stage(s);
#pragma unroll
            for (int j = 0; j < 3; ++j)
                epi_slice<EKE, 32>(p, st + 32 * j, LDW, m0 + wm * WM + s * 32, n0 + wn * WC + 32 * j, lane, zc,
                                   kch[j]);
        }
    } else {
        EpiCh kch = epi_channels(p, n0 + wn * WC + 4 * (lane % (WC / 4)), EKE != EK_RMW);
        if constexpr (EKE == EK_RMW) {
            // the residual rows of slice s + 1 load while slice s is staged, added and stored; slice 0's go out
            // with the channel constants, before the gates' tanh waits for those
            f32x4 xr[2][WC / 8];
            rmw_load<WC>(p, m0 + wm * WM, n0 + wn * WC, lane, zc, xr[0]);
            epi_gate_tanh(p, kch);
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                stage(s);
                if (s + 1 < NS)
                    rmw_load<WC>(p, m0 + wm * WM + (s + 1) * 32, n0 + wn * WC, lane, zc, xr[(s + 1) & 1]);
                rmw_finish<WC>(p, st, LDW, m0 + wm * WM + s * 32, n0 + wn * WC, lane, zc, kch, xr[s & 1]);
            }
        } else {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                stage(s);
                epi_slice<EKE, WC>(p, st, LDW, m0 + wm * WM + s * 32, n0 + wn * WC, lane, zc, kch);
            }
        }
    }
}


template <int BM, int BN, int NW, bool DEEP = false>
constexpr int gemm_smem()
{
    constexpr int LDW = BN / 2 + 4, NSTG = DEEP ? (BM == 128 ? 4 : 3) : 2;
    return NSTG * (BN + BM) * 64 * 2 > NW * 32 * LDW * 4 ? NSTG * (BN + BM) * 64 * 2 : NW * 32 * LDW * 4;
}

// One tile a workgroup.
// Waves a SIMD: 8-wave tiles two (one workgroup a CU), 4-wave 128 x 128 tiles two (two workgroups a CU, 64 KB of LDS
// each) unless deep-staged (EK_DEEP: one workgroup a CU), other 4-wave tiles one.
template <int BM, int NW, int EK> constexpr int gemm_waves_per_eu()
{
    return NW == 8 || (BM == 128 && !(EK & EK_DEEP)) ? 2 : 1;
}

template <int BM, int BN, bool kF8, int EK, int NW>
__global__ __launch_bounds__(64 * NW, BM == 128 && !(EK & EK_DEEP) ? 2 : 1) __attribute__((
    amdgpu_waves_per_eu(gemm_waves_per_eu<BM, NW, EK>(), gemm_waves_per_eu<BM, NW, EK>()))) void gemm_kernel(GemmG G)
{
    __shared__ __attribute__((aligned(16))) uint16_t smem[gemm_smem<BM, BN, NW, (EK & EK_DEEP) != 0>() / 2];
    uint32_t z, tm, tn;
    const GemmP& p = locate(G, xcd_order(blockIdx.x, gridDim.x), z, tm, tn);
    gemm_tile<BM, BN, kF8, EK, NW>(p, z, tm, tn, 0, int(p.K) / BK, smem, nullptr, -1);
}

// Persistent stream-K: a grid of one workgroup a CU takes the first sk.dp tiles whole (round robin), then splits
// the rest's k steps evenly into one range a workgroup. A tile split over several ranges is finished by the one
// held by the highest workgroup: it adds the partials the others publish. Waits thus only ever point at workgroups
// dispatched earlier, which publish before they wait on anything, so the launch always completes.
template <int BM, int BN, bool kF8, int EK, int NW>
__global__ __launch_bounds__(64 * NW, 1) __attribute__((amdgpu_waves_per_eu(NW / 4, NW / 4))) void gemm_sk_kernel(
    GemmG G, SkP sk)
{
    __shared__ __attribute__((aligned(16))) uint16_t smem[gemm_smem<BM, BN, NW>() / 2];
    const uint32_t w = blockIdx.x, grid = gridDim.x;
    for (uint32_t t = w; t < sk.dp; t += grid) {
        uint32_t z, tm, tn;
        const GemmP& p = locate(G, xcd_order(t, sk.dp), z, tm, tn);
        __syncthreads(); // the previous tile's epilogue is done with the LDS
        gemm_tile<BM, BN, kF8, EK, NW>(p, z, tm, tn, 0, int(sk.kt), smem, nullptr, -1);
    }
    // the tail: this workgroup's range (virtual index v), two passes over its tiles: first the ranges it publishes,
    // then the tiles it owns (the tile's range held by its highest workgroup, which adds the others' partials)
    const uint32_t per = grid / 8;
    const uint32_t v = grid % 8 ? w : (w % 8) * per + w / 8;
    const uint64_t b = sk_begin(sk, v), e = sk_begin(sk, v + 1);
    if (b < e) {
        const uint64_t t0 = b / sk.kt, t1 = (e - 1) / sk.kt;
        for (int pass = 0; pass < 2; ++pass)
            for (uint64_t tt = t1 + 1; tt-- > t0;) {
                const uint64_t ts = tt * sk.kt, lo = ts > b ? ts : b, hi = ts + sk.kt < e ? ts + sk.kt : e;
                // the ranges of this tile: virtual indices lo_i .. hi_i
                uint32_t lo_i = v, hi_i = v;
                while (lo_i > 0 && sk_begin(sk, lo_i) > ts)
                    --lo_i;
                while (hi_i + 1 < grid && sk_begin(sk, hi_i + 1) < ts + sk.kt)
                    ++hi_i;
                uint32_t owner = lo_i;
                for (uint32_t i = lo_i + 1; i <= hi_i; ++i)
                    if (sk_phys(i) > sk_phys(owner))
                        owner = i;
                const bool own = owner == v;
                if (own != (pass == 1))
                    continue;
                uint32_t z, tm, tn;
                const GemmP& p = locate(G, sk.dp + uint32_t(tt), z, tm, tn);
                __syncthreads();
                if (own)
                    gemm_tile<BM, BN, kF8, EK, NW>(p, z, tm, tn, int(lo - ts), int(hi - ts), smem, &sk, -1,
                                                   int(lo_i), int(hi_i), int(v), tt);
                else
                    gemm_tile<BM, BN, kF8, EK, NW>(p, z, tm, tn, int(lo - ts), int(hi - ts), smem, &sk,
                                                   sk_slot(sk, v, tt));
            }
    }
}

// Stream-K workspaces: two partial slots and flags per workgroup of a one-a-CU grid, and the launch epoch the flags
// are compared with (so they never need clearing). A workspace serves one launch at a time: a launch takes the
// workspace its stream used last (stream order keeps the two apart), else one whose last launch has completed (its
// event), else a new one, and past kSkPool workspaces a device's least recently used one after its last launch (the
// stream waits for that launch's event). Streams of one device thus never share partials in flight.
// The memory is uncached: a partial written by a CU of one XCD is read by a CU of another, whose L2 is not coherent
// with the writer's for ordinary allocations. Allocated at the full size and never freed (uncached memory a kernel has
// read stays allocated until the process ends). A launch that gives up a wait sets its stream's error word (pinned host
// memory, one a stream: the error belongs to the launch's stream, whichever workspace it used); a stream's word is
// checked and cleared when that stream is synchronised through the library or launches again, every word by a
// device-wide synchronisation.
struct SkWork {
    float* ws = nullptr;
    size_t ws_bytes = 0;
    uint32_t* flags = nullptr;
    uint32_t nflags = 0, epoch = 0;
    hipStream_t last = nullptr;
    hipEvent_t done = nullptr;
    uint64_t used = 0; // launch counter at its last use (least recently used first)
};
struct SkDevice {
    uint32_t cus = 0;
    uint64_t launches = 0;
    std::vector<std::unique_ptr<SkWork>> pool;
    // the error words of the streams that launched stream-K work on this device (kept until the process ends)
    std::vector<std::pair<hipStream_t, uint32_t*>> errs;
};
constexpr int kMaxDevices = 64;
constexpr size_t kSkPool = 4;
constexpr uint32_t kSkPollsDefault = 1u << 26;
std::mutex g_sk_mutex;
SkDevice g_sk[kMaxDevices];
uint32_t g_sk_polls = kSkPollsDefault;

// A workspace for one stream-K launch of `need` partial bytes on stream s (g_sk_mutex held).
mk_status sk_acquire(SkDevice& D, hipStream_t s, size_t need, uint32_t nflags, SkWork*& out)
{
    SkWork* pick = nullptr;
    for (auto& w : D.pool)
        if (w->last == s && w->ws_bytes >= need && w->nflags >= nflags)
            pick = w.get();
    if (!pick)
        for (auto& w : D.pool)
            if (w->ws_bytes >= need && w->nflags >= nflags && hipEventQuery(w->done) == hipSuccess) {
                pick = w.get();
                break;
            }
    if (!pick && D.pool.size() < kSkPool) {
        auto w = std::make_unique<SkWork>();
        MK_HIP(hipExtMallocWithFlags(reinterpret_cast<void**>(&w->ws), need, hipDeviceMallocUncached));
        w->ws_bytes = need;
        MK_HIP(hipExtMallocWithFlags(reinterpret_cast<void**>(&w->flags), nflags * sizeof(uint32_t),
                                     hipDeviceMallocUncached));
        MK_HIP(hipMemset(w->flags, 0, nflags * sizeof(uint32_t)));
        MK_HIP(hipStreamSynchronize(nullptr)); // cleared before the launch's stream reads them
        w->nflags = nflags;
        MK_HIP(hipEventCreateWithFlags(&w->done, hipEventDisableTiming));
        pick = w.get();
        D.pool.push_back(std::move(w));
    }
    if (!pick) {
        for (auto& w : D.pool)
            if (w->ws_bytes >= need && w->nflags >= nflags && (!pick || w->used < pick->used))
                pick = w.get();
        if (!pick)
            return fail(MK_ERR_UNSUPPORTED, "gemm: stream-K workspaces smaller than this launch needs");
        MK_HIP(hipStreamWaitEvent(s, pick->done, 0));
    }
    out = pick;
    return MK_OK;
}

// The error word of stream s on a device (g_sk_mutex held), made on its first stream-K launch.
mk_status sk_err_word(SkDevice& D, hipStream_t s, uint32_t*& out)
{
    for (auto& e : D.errs)
        if (e.first == s) {
            out = e.second;
            return MK_OK;
        }
    uint32_t* w = nullptr;
    MK_HIP(hipHostMalloc(reinterpret_cast<void**>(&w), sizeof(uint32_t), hipHostMallocCoherent));
    *w = 0;
    D.errs.emplace_back(s, w);
    out = w;
    return MK_OK;
}

// A stream-K wait that gave up in a launch on stream s (all: on any stream) of a device (g_sk_mutex held):
// MK_ERR_DEVICE once, then cleared.
mk_status sk_check(SkDevice& D, hipStream_t s, bool all)
{
    for (auto& e : D.errs)
        if ((all || e.first == s) && __atomic_exchange_n(e.second, 0u, __ATOMIC_RELAXED))
            return fail(MK_ERR_DEVICE, "gemm: a stream-K launch gave up waiting for a partial tile; its output is wrong");
    return MK_OK;
}

template <int BM, int BN, bool kF8, int EK, int NW = 4>
mk_status launch(GemmP* p, uint32_t count, const GemmPlan& plan, hipStream_t s)
{
    constexpr int NT = 64 * NW, NACC = (BN / 64) * (BM / (NW / 2) / 32) * 16;
    GemmG G{};
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < count; ++i) {
        p[i].tiles_m = p[i].conv_w ? p[i].conv_pix / BM : cdiv(p[i].M, BM);
        p[i].tiles_n = p[i].N / BN;
        G.g[i] = p[i];
        tiles += p[i].tiles_m * p[i].tiles_n * p[i].batch;
    }
    G.tiles0 = count > 1 ? p[0].tiles_m * p[0].tiles_n * p[0].batch : tiles;
    const uint32_t kt = p[0].K / BK;
    if constexpr (BN == 256 && BM == 256) {
        int dev = 0;
        MK_HIP(hipGetDevice(&dev));
        if (dev < 0 || dev >= kMaxDevices)
            return fail(MK_ERR_DEVICE, "gemm: device index out of range");
        std::lock_guard<std::mutex> lock(g_sk_mutex);
        SkDevice& D = g_sk[dev];
        if (!D.cus) {
            int n = 0;
            MK_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
            D.cus = n > 0 ? uint32_t(n) : 1;
        }
        const uint32_t grid = D.cus;
        if (plan.sk && plan.dp % grid == 0 && plan.dp < tiles) {
            MK_TRY(sk_check(D, s, false));
            SkP sk{};
            sk.total = tiles;
            sk.dp = uint32_t(plan.dp);
            sk.kt = kt;
            sk.units = uint64_t(tiles - sk.dp) * kt;
            SkWork* W = nullptr;
            MK_TRY(sk_acquire(D, s, size_t(2) * grid * NT * NACC * sizeof(float), 2 * grid, W));
            if (++W->epoch == 0)
                W->epoch = 1;
            sk.ws = W->ws;
            sk.flags = W->flags;
            MK_TRY(sk_err_word(D, s, sk.err));
            sk.epoch = W->epoch;
            sk.polls = g_sk_polls;
            gemm_sk_kernel<BM, BN, kF8, EK, NW><<<grid, NT, 0, s>>>(G, sk);
            MK_HIP(hipGetLastError());
            MK_HIP(hipEventRecord(W->done, s));
            W->last = s;
            W->used = ++D.launches;
            return MK_OK;
        }
    }
    gemm_kernel<BM, BN, kF8, EK, NW><<<tiles, NT, 0, s>>>(G);
    MK_HIP(hipGetLastError());
    return MK_OK;
}

// The epilogue kind of an mk_epilogue.
int epi_kind(uint32_t e)
{
    return e == MK_EPI_HEADS                             ? EK_HEADS
           : e == MK_EPI_STORE                           ? EK_STORE
           : (e == MK_EPI_GELU_TANH || e == MK_EPI_SILU) ? EK_ACT
           : (e == MK_EPI_SWIGLU || e == MK_EPI_GEGLU || e == MK_EPI_PAIR_SUM) ? EK_GLU
                                                         : EK_RMW;
}

// Checks one problem's arguments and fills its kernel parameters.
// conv: a 3 x 3 convolution's GEMM, whose N may also be a multiple of 96 (128 x 96 tiles)
mk_status prepare(const mk_gemm_args* a, GemmP& p, bool conv = false)
{
    if (!a || !a->a || !a->w || (!a->c && a->epilogue != MK_EPI_HEADS))
        return fail(MK_ERR_ARG, "gemm: null argument");
    if (a->K % 64 || (a->N % 64 && !(conv && a->N % 96 == 0)) || a->K == 0 || a->N == 0)
        return fail(MK_ERR_ARG, "gemm: K and N must be nonzero multiples of 64 (K " + std::to_string(a->K) + ", N " +
                                    std::to_string(a->N) + ")");
    if (a->w_dtype != MK_BF16 && a->w_dtype != MK_FP8_E4M3 && a->w_dtype != MK_F16)
        return fail(MK_ERR_ARG, "gemm: weights must be bf16, fp8-e4m3 or f16 (then A is f16 too)");
    if (a->c_dtype != MK_F32 && a->c_dtype != MK_BF16 && a->c_dtype != MK_F16 && a->epilogue != MK_EPI_HEADS)
        return fail(MK_ERR_ARG, "gemm: C must be f32, bf16 or f16");
    if (a->lda % 8 || (reinterpret_cast<uintptr_t>(a->a) & 15) || (reinterpret_cast<uintptr_t>(a->w) & 15))
        return fail(MK_ERR_ARG, "gemm: A and W must be 16-byte aligned with lda a multiple of 8");
    if (a->lda >= (1u << 23) || a->K >= (1u << 23))
        return fail(MK_ERR_ARG, "gemm: lda and K must be below 2^23 (32-bit byte offsets within a tile)");
    if (a->epilogue > MK_EPI_PAIR_SUM)
        return fail(MK_ERR_ARG, "gemm: unknown epilogue");
    const bool glu = a->epilogue == MK_EPI_SWIGLU || a->epilogue == MK_EPI_GEGLU || a->epilogue == MK_EPI_PAIR_SUM;
    if (glu && (a->N % 128 || (a->N / 2) % 4))
        return fail(MK_ERR_ARG, "gemm: a gated linear unit needs N = 2 F a multiple of 128");
    const bool gated = a->epilogue == MK_EPI_GATE_ADD || a->epilogue == MK_EPI_GATE_TANH;
    if (gated && !a->gate)
        return fail(MK_ERR_ARG, "gemm: gated epilogue without a gate");
    if (a->w_dtype == MK_FP8_E4M3 && !a->wscale)
        return fail(MK_ERR_ARG, "gemm: fp8 weights need per-channel scales");
    p = GemmP{};
    p.a = static_cast<const uint16_t*>(a->a);
    p.w = a->w;
    p.wscale = a->wscale;
    p.bias = a->bias;
    p.c = a->c;
    p.gate = a->gate;
    p.gate_alt = a->gate_alt;
    p.split = a->split;
    p.seg_rows = a->seg_rows ? a->seg_rows : 0xffffffffu;
    p.M = a->M;
    p.N = a->N;
    p.K = a->K;
    p.lda = a->lda;
    p.ldc = a->ldc;
    p.sa = a->stride_a;
    p.sc = a->stride_c;
    p.epi = a->epilogue;
    p.c_bf16 = a->c_dtype == MK_BF16 || a->c_dtype == MK_F16;
    p.c_f16 = a->c_dtype == MK_F16;
    p.batch = a->batch;
    p.glu_f = glu ? a->N / 2 : 0;
    if (a->epilogue == MK_EPI_HEADS) {
        // q|k|v columns (N = 3 heads d), or q alone (k and vt NULL: N = heads d); d = 128 on 256-channel tiles
        // (per-head RMSNorm and RoPE optional), d = 64 on 128-channel tiles (no norm, no RoPE)
        const mk_heads_args* h = a->heads;
        // q|k|v, q alone (k, vt NULL), or, for 64-dim heads, k|v alone (q NULL: a cross attention's context)
        const bool qonly = h && h->q && !h->k && !h->vt, kvonly = h && !h->q && h->k && h->vt;
        const uint32_t parts = qonly ? 1 : kvonly ? 2 : 3, d = h ? h->head_dim : 0;
        bool ok = h && (h->q || kvonly) && (qonly || (h->k && h->vt)) && (d == 128 || d == 64) && h->heads &&
                  (!kvonly || d == 64) && uint64_t(a->N) == uint64_t(parts) * h->heads * d && h->k_pad % 16 == 0 &&
                  (qonly || uint64_t(h->row0) + a->M <= h->k_pad) &&
                  (kvonly || uint64_t(h->q_row0) + a->M <= h->q_pad) &&
                  (h->dtype == 0 || h->dtype == MK_BF16 || h->dtype == MK_F16);
        if (d == 128)
            ok = ok && a->N % 256 == 0 && h->rope_mode <= 2 && (!h->rope_mode || h->rope);
        else
            ok = ok && a->N % 128 == 0 && h->rope_mode == 0 && !h->norm_q && !h->norm_k;
        if (!ok)
            return fail(MK_ERR_ARG, "gemm heads epilogue: needs q, k, vt (N = 3 x heads x head_dim), q alone (1 x) "
                                    "or, for head_dim 64, k and vt alone (2 x), head_dim 128 with N a multiple of "
                                    "256 or head_dim 64 with N a multiple of 128 and no norm or RoPE, k_pad a "
                                    "multiple of 16, row0 + M within the padded rows, and dtype bf16 or f16");
        p.hp = HeadsP{static_cast<uint16_t*>(h->q), static_cast<uint16_t*>(h->k), static_cast<uint16_t*>(h->vt),
                      h->heads, h->q_pad, h->k_pad, h->row0, h->q_row0, h->rope_mode, a->N / parts, h->norm_q,
                      h->norm_k, h->rope, h->eps, h->k_scale == 0.0f ? 1.0f : h->k_scale, h->dtype == MK_F16 ? 1u : 0u,
                      h->rope_stride, d};
    }
    return MK_OK;
}

} // namespace gemm_detail

mk_status gemm_take_error(const void* stream, bool all)
{
    using namespace gemm_detail;
    std::lock_guard<std::mutex> lock(g_sk_mutex);
    for (SkDevice& D : g_sk)
        MK_TRY(sk_check(D, static_cast<hipStream_t>(const_cast<void*>(stream)), all));
    return MK_OK;
}

// The tile shape of a launch, by its estimated duration: waves of tiles (rounded up) x k steps x the duration of one
// k step of the tile relative to a 256 x 256 one, measured on MI355X (kt = 20-80, the SDXL and step shapes): 256 x 128
// 0.66, 256 x 64 0.62, 128 x 128 0.67 for a pair of tiles (two workgroups share a CU: 64 KB of LDS each), so a wave of
// 128 x 128 tiles is 2 per CU and an odd last tile costs half a pair; ties keep the larger tile. Convolutions also
// have 256 x 192 tiles (8 waves, 0.78), for their 192- and 384-channel layers, and 128 x 96 tiles (4 waves on
// 16 x 16 x 32, two workgroups a CU) for output channels that are an odd multiple of 96. The heads epilogue
// takes 256 x 256 tiles for 128-dim heads and 128-channel tiles for 64-dim heads; fp8 weights 256-token tiles, and so
// do half-weight convolutions.
// 256 x 256 tiles use stream-K when whole waves leave at least 5% of the last wave's workgroups idle and
// a tile is long (K of 6144 or more; measured, the partials' exchange costs about 24 k steps of a tile, more than the
// balance saves on shorter tiles): the whole waves go round robin, the rest is split by k steps (at least 4 a
// workgroup).
GemmPlan gemm_plan(const mk_gemm_args* a, uint32_t n, uint32_t cus, bool conv)
{
    const uint64_t kt = a[0].K / gemm_detail::BK;
    const uint32_t N = a[0].N;
    const bool heads = a[0].epilogue == MK_EPI_HEADS;
    const bool narrow_ok = a[0].epilogue != MK_EPI_GELU_TANH && a[0].epilogue != MK_EPI_SILU &&
                           a[0].epilogue != MK_EPI_SWIGLU && a[0].epilogue != MK_EPI_GEGLU &&
                           a[0].epilogue != MK_EPI_PAIR_SUM; // 64-wide tiles
    // 128-token tiles: bf16 or half weights (convolutions: bf16 only, as their plans were measured)
    const bool short_ok = !heads && (conv ? a[0].w_dtype == MK_BF16 : a[0].w_dtype != MK_FP8_E4M3);
    auto tiles_of = [&](int bm, int bn) {
        uint64_t t = 0;
        for (uint32_t i = 0; i < n; ++i)
            t += uint64_t((a[i].M + bm - 1) / bm) * a[i].batch * (N / bn);
        return t;
    };
    GemmPlan best{};
    best.cost = -1.0;
    auto consider = [&](int bm, int bn, double c) {
        if (N % bn)
            return;
        GemmPlan pl{};
        pl.bm = bm;
        pl.bn = bn;
        pl.tiles = tiles_of(bm, bn);
        const uint64_t rounds = (pl.tiles + cus - 1) / cus;
        pl.cost = (bm == 128 ? 0.5 * double(rounds) : double(rounds)) * double(kt) * c;
        if (bm == 256 && bn == 256) {
            const uint64_t waves = pl.tiles / cus, idle = rounds * cus - pl.tiles;
            pl.dp = waves * cus;
            pl.sk = waves >= 1 && idle * 20 >= rounds * cus && kt >= 96 && (pl.tiles - pl.dp) * kt >= uint64_t(4) * cus;
            if (pl.sk)
                pl.cost = (double(pl.tiles) / cus + 24.0 / double(kt)) * double(kt);
        }
        if (best.cost < 0 || pl.cost < best.cost)
            best = pl;
    };
    if (heads && a[0].heads && a[0].heads->head_dim == 64) {
        // the 64-dim heads epilogue on 256-token tiles: 0.8 (measured on the SDXL shapes, 2048-8192 tokens x 1280 or
        // 640 channels: 256 x 128 tiles took 10-25% longer than pairs of 128 x 128 at the 0.66 estimate's ties)
        consider(256, 128, 0.8);
        if (a[0].w_dtype != MK_FP8_E4M3)
            consider(128, 128, 0.67);
        return best;
    }
    consider(256, 256, 1.0);
    if (heads)
        return best;
    consider(256, 128, 0.66);
    if (conv)
        consider(256, 192, 0.78);
    if (conv && N % 64) // 96 output channels (and odd multiples of 96) take 128 x 96 tiles, nothing else
        consider(128, 96, 0.5);
    if (narrow_ok)
        consider(256, 64, 0.62);
    if (short_ok)
        consider(128, 128, 0.67);
    if (best.cost < 0) // N not a multiple of 128 with an activation or GLU: the dispatch rejects it
        consider(256, 64, 0.62);
    return best;
}

double gemm_cost(const mk_gemm_args* a, uint32_t n, uint32_t cus) { return gemm_plan(a, n, cus).cost; }
} // namespace mk

using namespace mk;
using namespace mk::gemm_detail;

extern "C" mk_status mk_gemm_grouped(const mk_gemm_args* a, uint32_t count, void* stream)
{
    if (!a)
        return fail(MK_ERR_ARG, "gemm: null argument");
    if (count == 0 || count > 2)
        return fail(MK_ERR_ARG, "gemm: 1 or 2 problems a launch");
    GemmP p[2];
    uint32_t n = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const mk_status st = prepare(&a[i], p[n]);
        if (st != MK_OK)
            return st;
        if (i > 0 && (a[i].N != a[0].N || a[i].K != a[0].K || a[i].w_dtype != a[0].w_dtype ||
                      epi_kind(a[i].epilogue) != epi_kind(a[0].epilogue)))
            return fail(MK_ERR_ARG, "gemm: grouped problems need equal N, K, weight dtype and epilogue kind");
        if (a[i].M && a[i].batch)
            ++n; // empty problems drop out
    }
    if (n == 0)
        return MK_OK;
    const bool f8 = a[0].w_dtype == MK_FP8_E4M3;
    const int ek = epi_kind(a[0].epilogue);
    int cus = 0, dev = 0;
    MK_HIP(hipGetDevice(&dev));
    MK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // the non-empty problems, for the plan
    mk_gemm_args live[2];
    for (uint32_t i = 0, j = 0; i < count; ++i)
        if (a[i].M && a[i].batch)
            live[j++] = a[i];
    const GemmPlan plan = gemm_plan(live, n, uint32_t(cus > 0 ? cus : 1));
    const int bn = plan.bn;
    if (bn == 64 && (ek == EK_ACT || ek == EK_GLU))
        return fail(MK_ERR_UNSUPPORTED, "gemm: activation and GLU epilogues need N a multiple of 128");
    // the heads epilogue writes one head per wave slice: 128-dim heads on 256-channel tiles, 64-dim on 128-channel
    if (ek == EK_HEADS && !((bn == 256 && p[0].hp.hd == 128) || (bn == 128 && p[0].hp.hd == 64)))
        return fail(MK_ERR_UNSUPPORTED, "gemm: heads epilogue tile width does not match the head dim");
    hipStream_t s = static_cast<hipStream_t>(stream);
    mk_status e;
    // 4-wave 128-channel tiles (128 x 128, or 256 x 128 with bn 128) of epilogue kind E: deep-staged (EK_DEEP) when
    // the launch has at most one tile a CU, so each workgroup runs alone on its CU
    const bool deep = !f8 && plan.tiles <= uint64_t(cus > 0 ? cus : 1);
    auto narrow = [&](auto e_c) -> mk_status {
        constexpr int E = decltype(e_c)::value;
        if (plan.bm == 128)
            return deep ? launch<128, 128, false, E | EK_DEEP, 4>(p, n, plan, s)
                        : launch<128, 128, false, E, 4>(p, n, plan, s);
        return deep ? launch<256, 128, false, E | EK_DEEP, 4>(p, n, plan, s)
                    : launch<256, 128, false, E, 4>(p, n, plan, s);
    };
    if (a[0].w_dtype == MK_F16) {
        // half operands (the VAE's 1 x 1 convolutions and attention products; SDXL's F16 matrices): plain, residual,
        // GLU / pair-sum and heads epilogues
        if (ek == EK_ACT)
            return fail(MK_ERR_UNSUPPORTED, "gemm: f16 operands take the STORE, ADD / GATE, GLU, PAIR_SUM and HEADS "
                                            "epilogues");
        auto f16 = [&](auto ek_c) -> mk_status {
            constexpr int K = decltype(ek_c)::value, E = K | EK_F16;
            if (plan.bm == 128 || bn == 128)
                return narrow(std::integral_constant<int, E>{});
            if (bn == 256)
                return launch<256, 256, false, E, 8>(p, n, plan, s);
            if constexpr (K == EK_GLU || K == EK_HEADS)
                return fail(MK_ERR_UNSUPPORTED, "gemm: GLU, pair-sum and heads epilogues need N a multiple of 128");
            else
                return launch<256, 64, false, E, 4>(p, n, plan, s);
        };
        if (ek == EK_STORE)
            return f16(std::integral_constant<int, EK_STORE>{});
        if (ek == EK_RMW)
            return f16(std::integral_constant<int, EK_RMW>{});
        if (ek == EK_HEADS)
            return f16(std::integral_constant<int, EK_HEADS>{});
        return f16(std::integral_constant<int, EK_GLU>{});
    }
    // 256-wide tiles: 8 waves (two a SIMD, 64 x 128 wave tiles), so one wave's waits (barrier, loads) leave the
    // other's MFMAs running
#define MK_GEMM_EK(BN, EK)                                                                                        \
    e = f8 ? launch<256, BN, true, EK, BN == 256 ? 8 : 4>(p, n, plan, s)                                           \
           : launch<256, BN, false, EK, BN == 256 ? 8 : 4>(p, n, plan, s)
    if (plan.bm == 128 || (bn == 128 && !f8)) {
        // 128-channel tiles with bf16 weights: 128 x 128 (launches of few tiles: two workgroups a CU, or one
        // deep-staged) or 256 x 128 (half weights: above)
        if (ek == EK_STORE)
            e = narrow(std::integral_constant<int, EK_STORE>{});
        else if (ek == EK_HEADS)
            e = narrow(std::integral_constant<int, EK_HEADS>{});
        else if (ek == EK_ACT)
            e = narrow(std::integral_constant<int, EK_ACT>{});
        else if (ek == EK_GLU)
            e = narrow(std::integral_constant<int, EK_GLU>{});
        else
            e = narrow(std::integral_constant<int, EK_RMW>{});
    } else if (ek == EK_HEADS) {
        if (bn == 256)
            MK_GEMM_EK(256, EK_HEADS);
        else
            MK_GEMM_EK(128, EK_HEADS);
    } else if (bn == 256) {
        if (ek == EK_STORE)
            MK_GEMM_EK(256, EK_STORE);
        else if (ek == EK_ACT)
            MK_GEMM_EK(256, EK_ACT);
        else if (ek == EK_GLU)
            MK_GEMM_EK(256, EK_GLU);
        else
            MK_GEMM_EK(256, EK_RMW);
    } else if (bn == 128) {
        if (ek == EK_STORE)
            MK_GEMM_EK(128, EK_STORE);
        else if (ek == EK_ACT)
            MK_GEMM_EK(128, EK_ACT);
        else if (ek == EK_GLU)
            MK_GEMM_EK(128, EK_GLU);
        else
            MK_GEMM_EK(128, EK_RMW);
    } else {
        if (ek == EK_STORE)
            MK_GEMM_EK(64, EK_STORE);
        else
            MK_GEMM_EK(64, EK_RMW);
    }
#undef MK_GEMM_EK
    return e;
}

extern "C" mk_status mk_gemm(const mk_gemm_args* a, void* stream) { return mk_gemm_grouped(a, 1, stream); }

extern "C" mk_status mk_gemm_set_wait_limit(uint32_t polls)
{
    std::lock_guard<std::mutex> lock(g_sk_mutex);
    g_sk_polls = polls;
    return MK_OK;
}

namespace mk {
// 3 x 3 convolution as one GEMM over the padded pixel grid: output row r (grid pixel r of (h + 2) x (w + 2)) and tap
// (dy, dx) read input row r + dy (w + 2) + dx of x, whose w + 3 slack rows before the grid make every shift
// non-negative. K = 9 c runs tap-major: with c a multiple of 64 each 64-wide k step lies inside one tap, so the tap
// is a scalar offset of the k step (koffA); with dense weights (c a multiple of 8, not of 64, K = 9 c rounded up to
// 64, k = tap c + channel, zero past 9 c) each 16-byte chunk takes its own tap's row shift (koffq), so no MFMA work
// goes to channel padding (the VAE's 96-channel level: K 864 -> 896 instead of 1152). The ring's output rows are
// computed like the others and are the caller's to ignore (the norm epilogues write them as zeros).
mk_status conv3x3_run(const mk_conv_args* a, uint32_t lda, bool dense, const ConvNorm* nm, void* stream,
                      const ConvUp* up = nullptr)
{
    const char* who = dense ? "conv3x3_dense" : "conv3x3";
    if (!a || !a->x || !a->w || !a->y)
        return fail(MK_ERR_ARG, std::string(who) + ": null argument");
    if (!a->h || !a->width || !a->c || (a->n % 64 && a->n % 96) || !a->n)
        return fail(MK_ERR_ARG, std::string(who) + ": needs h, w >= 1 and channels out a nonzero multiple of 64 or 96");
    if (dense ? (a->c % 8 || a->c % 64 == 0 || a->c > 512 || lda < a->c || lda % 8)
              : (a->c % 64 || a->c > 4096 || lda != a->c))
        return fail(MK_ERR_ARG, dense ? "conv3x3_dense: channels in a multiple of 8 (not of 64) up to 512, lda >= c a "
                                        "multiple of 8"
                                      : "conv3x3: channels in a nonzero multiple of 64 (<= 4096)");
    if ((a->epilogue != MK_EPI_STORE && a->epilogue != MK_EPI_ADD) ||
        (a->epilogue == MK_EPI_ADD && a->y_dtype != MK_F32) || (a->y_dtype != MK_F32 && a->y_dtype != MK_F16))
        return fail(MK_ERR_ARG, std::string(who) + ": epilogue STORE (fp32 or f16) or ADD (fp32)");
    if (nm && (!nm->g || (a->n != 96 && a->n != 192) ||
               (nm->out ? (a->y_dtype != MK_F32 || nm->ld < a->n || nm->ld % 4)
                        : (a->y_dtype != MK_F16 || a->epilogue != MK_EPI_STORE))))
        return fail(MK_ERR_ARG, std::string(who) + ": the norm epilogues need 96 or 192 output channels and a gain, "
                                                   "and either an f16 store or an fp32 output plus a normed one");
    if (up && (nm || dense || !up->out || a->epilogue != MK_EPI_ADD || a->n % 192 || a->width % 256 || up->ld < a->n ||
               up->ld % 4 || a->h > (1u << 14) || a->width > (1u << 14)))
        return fail(MK_ERR_ARG, std::string(who) + ": the 2x-grid epilogue needs an ADD over 192-channel multiples, "
                                                   "an image width of a multiple of 256 and no norm epilogue");
    const uint64_t pw = uint64_t(a->width) + 2, rows = (uint64_t(a->h) + 2) * pw;
    if (rows >= (1u << 31) || (256 + 2 * pw + 2) * lda * 2 >= (uint64_t(1) << 32) || a->ldy < a->n)
        return fail(MK_ERR_ARG, std::string(who) + ": image too large or ldy < n");
    mk_gemm_args g{};
    g.a = a->x;
    g.w = a->w;
    g.bias = a->bias;
    g.c = a->y;
    g.M = uint32_t(rows);
    g.N = a->n;
    g.K = dense ? (9 * a->c + 63) / 64 * 64 : 9 * a->c;
    g.lda = lda;
    g.ldc = a->ldy;
    g.batch = 1;
    g.w_dtype = MK_F16;
    g.c_dtype = a->y_dtype;
    g.epilogue = a->epilogue;
    GemmP p;
    MK_TRY(prepare(&g, p, true));
    p.c_f16 = 1; // every 16-bit grid a convolution writes (its output, a normed or a 2x grid) is half
    p.conv_pw = uint32_t(pw);
    p.conv_tpt = dense ? a->c / 8 : a->c / 64;
    p.conv_inv = (65536u + p.conv_tpt - 1) / p.conv_tpt;
    int cus = 0, dev = 0;
    MK_HIP(hipGetDevice(&dev));
    MK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // tiles over the pixels when the plan for h w rows has a tile height dividing w, else over the padded rows
    mk_gemm_args gp = g;
    gp.M = a->h * a->width;
    GemmPlan plan = gemm_plan(&gp, 1, uint32_t(cus > 0 ? cus : 1), true);
    if (nm) { // the norm epilogues' tiles span the row: 128 x 96 or 256 x 192
        plan.bm = a->n == 96 ? 128 : 256;
        plan.bn = a->n;
    }
    if (up) { // 256 x 192 tiles over the pixels: a tile's rows lie in one image row
        plan.bm = 256;
        plan.bn = 192;
    }
    if (a->width % plan.bm == 0) {
        p.conv_w = a->width;
        p.conv_pix = gp.M;
    } else if (!nm) {
        plan = gemm_plan(&g, 1, uint32_t(cus > 0 ? cus : 1), true);
    }
    plan.sk = false;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool add = a->epilogue == MK_EPI_ADD;
    constexpr int C = EK_CONV | EK_F16, Q = EK_CONV | EK_CONVQ | EK_F16;
    if (up) {
        p.norm_out = up->out;
        p.norm_ld = up->ld;
        p.up_pw = 2 * a->width + 2;
        p.up_slack = 2 * a->width + 3;
        return launch<256, 192, false, EK_RMWUP | C, 8>(&p, 1, plan, s);
    }
    if (nm) {
        p.norm_g = nm->g;
        p.norm_out = nm->out;
        p.norm_ld = nm->ld;
        p.norm_only = nm->out && nm->skip_y ? 1u : 0u;
        if (a->n == 192) {
            if (nm->out)
                return dense ? launch<256, 192, false, EK_RMWN | Q, 8>(&p, 1, plan, s)
                             : launch<256, 192, false, EK_RMWN | C, 8>(&p, 1, plan, s);
            return dense ? launch<256, 192, false, EK_NORM | Q, 8>(&p, 1, plan, s)
                         : launch<256, 192, false, EK_NORM | C, 8>(&p, 1, plan, s);
        }
        if (nm->out)
            return dense ? launch<128, 96, false, EK_RMWN | Q, 4>(&p, 1, plan, s)
                         : launch<128, 96, false, EK_RMWN | C, 4>(&p, 1, plan, s);
        return dense ? launch<128, 96, false, EK_NORM | Q, 4>(&p, 1, plan, s)
                     : launch<128, 96, false, EK_NORM | C, 4>(&p, 1, plan, s);
    }
    // (the tile shapes a convolution's plan may take, each with the implicit-GEMM flags of its K layout)
    auto go = [&](auto f) -> mk_status {
        if (plan.bn == 96)
            return add ? f(std::integral_constant<int, 0>{}) : f(std::integral_constant<int, 1>{});
        if (plan.bm == 128)
            return add ? f(std::integral_constant<int, 2>{}) : f(std::integral_constant<int, 3>{});
        if (plan.bn == 256)
            return add ? f(std::integral_constant<int, 4>{}) : f(std::integral_constant<int, 5>{});
        if (plan.bn == 192)
            return add ? f(std::integral_constant<int, 6>{}) : f(std::integral_constant<int, 7>{});
        if (plan.bn == 128)
            return add ? f(std::integral_constant<int, 8>{}) : f(std::integral_constant<int, 9>{});
        return add ? f(std::integral_constant<int, 10>{}) : f(std::integral_constant<int, 11>{});
    };
    auto shape = [&](auto sel, auto flags) -> mk_status {
        constexpr int i = decltype(sel)::value, F = decltype(flags)::value;
        constexpr int EK = (i % 2 ? EK_STORE : EK_RMW) | F;
        if constexpr (i / 2 == 0)
            return launch<128, 96, false, EK, 4>(&p, 1, plan, s);
        else if constexpr (i / 2 == 1)
            return launch<128, 128, false, EK, 4>(&p, 1, plan, s);
        else if constexpr (i / 2 == 2)
            return launch<256, 256, false, EK, 8>(&p, 1, plan, s);
        else if constexpr (i / 2 == 3)
            return launch<256, 192, false, EK, 8>(&p, 1, plan, s);
        else if constexpr (i / 2 == 4)
            return launch<256, 128, false, EK, 4>(&p, 1, plan, s);
        else
            return launch<256, 64, false, EK, 4>(&p, 1, plan, s);
    };
    if (dense)
        return go([&](auto sel) { return shape(sel, std::integral_constant<int, Q>{}); });
    return go([&](auto sel) { return shape(sel, std::integral_constant<int, C>{}); });
}

mk_status conv3x3_dense(const mk_conv_args* a, uint32_t lda, void* stream, const ConvNorm* nm)
{
    return conv3x3_run(a, lda, true, nm, stream);
}
} // namespace mk

extern "C" mk_status mk_conv3x3(const mk_conv_args* a, void* stream)
{
    return conv3x3_run(a, a ? a->c : 0, false, nullptr, stream);
}

namespace mk {
mk_status conv3x3_fused(const mk_conv_args* a, const ConvNorm& nm, void* stream)
{
    return conv3x3_run(a, a ? a->c : 0, false, &nm, stream);
}
mk_status conv3x3_up(const mk_conv_args* a, const ConvUp& up, void* stream)
{
    return conv3x3_run(a, a ? a->c : 0, false, nullptr, stream, &up);
}
} // namespace mk
