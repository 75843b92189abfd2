// proj: C = A W^T on gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16), fp32 accumulation, with fused epilogues.
//
// Roles: the weight tile is the MFMA A operand (its M = output channels) and the activation tile the B operand (its
// N = tokens), so each lane's accumulators hold 4 consecutive channels of one token: the residual / gate epilogues
// read-modify-write 16 bytes per lane, and a head's 128 channels sit in one lane pair (per-head RMSNorm is one
// cross-lane add, RoPE pairs are lane-local).
//
// Tiling: BM tokens x BN channels x 64 k per workgroup of 4 waves (2 x 2), each wave BN/2 x BM/2 as (BN/64) x (BM/64)
// MFMA blocks of 32 x 32. Both tiles are K-contiguous and staged in LDS with a 16-byte-chunk XOR swizzle
// (chunk ^ (row & 7)) so the fragment reads of 32 rows at one k offset are bank-conflict free; two LDS buffers, the
// next tile's global loads in flight in registers during the current tile's MFMAs, one barrier per k step.
// Workgroups map to tiles XCD-aware (consecutive tiles on one XCD share its L2) and grouped along M.
#include "common.hpp"

namespace mk {

namespace gemm_detail {

struct HeadsP {
    uint16_t *q, *k, *vt;
    uint32_t heads, q_pad, k_pad, row0, q_row0, rope_mode, dim;
    const float *norm_q, *norm_k, *rope;
    float eps;
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
    uint32_t epi, c_bf16;
    uint32_t tiles_m, tiles_n;
    HeadsP hp;
};

constexpr int BK = 64;

__device__ inline int swz(int row, int kc) { return row * 64 + ((kc ^ (row & 7)) << 3); }

// fp8 e4m3 (16 values in a u32x4) -> two bf16x8 chunks, exact.
__device__ inline void f8x16_to_bf16(const u32x4& v, u32x4& lo, u32x4& hi)
{
    uint32_t o[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t x = v[i];
        const float f0 = e4m3_to_f32(uint8_t(x)), f1 = e4m3_to_f32(uint8_t(x >> 8));
        const float f2 = e4m3_to_f32(uint8_t(x >> 16)), f3 = e4m3_to_f32(uint8_t(x >> 24));
        o[2 * i] = (__builtin_bit_cast(uint32_t, f0) >> 16) | (__builtin_bit_cast(uint32_t, f1) & 0xffff0000u);
        o[2 * i + 1] = (__builtin_bit_cast(uint32_t, f2) >> 16) | (__builtin_bit_cast(uint32_t, f3) & 0xffff0000u);
    }
    lo = u32x4{o[0], o[1], o[2], o[3]};
    hi = u32x4{o[4], o[5], o[6], o[7]};
}

// Epilogue of one 4-channel group of one token: acc -> (scale, bias) -> activation / residual / store.
__device__ inline void epi_store(const GemmP& p, int64_t rowoff, int ch, bool alt, f32x4 v)
{
    if (p.wscale) {
        const f32x4 s = *reinterpret_cast<const f32x4*>(p.wscale + ch);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] *= s[j];
    }
    if (p.bias) {
        const f32x4 b = *reinterpret_cast<const f32x4*>(p.bias + ch);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] += b[j];
    }
    if (p.epi == MK_EPI_GELU_TANH) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = gelu_tanh_f(v[j]);
    } else if (p.epi == MK_EPI_SILU) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            v[j] = silu_f(v[j]);
    }
    if (p.epi == MK_EPI_GATE_ADD || p.epi == MK_EPI_GATE_TANH || p.epi == MK_EPI_ADD) {
        f32x4* x = reinterpret_cast<f32x4*>(static_cast<float*>(p.c) + rowoff + ch);
        f32x4 xv = *x;
        if (p.epi == MK_EPI_ADD) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xv[j] += v[j];
        } else {
            const f32x4 g = *reinterpret_cast<const f32x4*>(p.gate + (alt ? p.gate_alt : 0) + ch);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xv[j] += (p.epi == MK_EPI_GATE_TANH ? tanhf(g[j]) : g[j]) * v[j];
        }
        *x = xv;
    } else if (p.c_bf16) {
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.c) + rowoff + ch) =
            u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else {
        *reinterpret_cast<f32x4*>(static_cast<float*>(p.c) + rowoff + ch) = v;
    }
}

// The q / k / v epilogue from a wave's staged slice: 32 tokens x 128 channels (one head of q, k or v) in LDS, row
// stride ld floats, tokens tok0 .. tok0 + 31 (GEMM rows). q, k: two lanes per token, RMSNorm * w over the head (one
// cross-lane add), RoPE, bf16 rows to [batch][heads][pad][128]; v: each lane two head dims across the 32 tokens, bf16
// to V^T [batch][heads][128][k_pad] rows.
__device__ __attribute__((noinline)) void epi_heads(const GemmP& p, const float* st, int ld, int tok0, int nw0, int lane)
{
    const HeadsP& h = p.hp;
    const int which = nw0 / int(h.dim), head = (nw0 % int(h.dim)) / 128;
    const int64_t bh = int64_t(blockIdx.z) * h.heads + head;
    if (which == 2) {
#pragma unroll
        for (int dd = 0; dd < 2; ++dd) {
            const int d = 2 * lane + dd, ch = nw0 + d;
            const float sc = p.wscale ? p.wscale[ch] : 1.0f, bi = p.bias ? p.bias[ch] : 0.0f;
            uint16_t* dst = h.vt + (bh * 128 + d) * int64_t(h.k_pad) + h.row0 + tok0;
            const bool vec = ((h.row0 + tok0) % 8) == 0 && tok0 + 32 <= int(p.M);
            if (vec) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    uint32_t w[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        w[e] = pack_bf16x2(st[(8 * c + 2 * e) * ld + d] * sc + bi, st[(8 * c + 2 * e + 1) * ld + d] * sc + bi);
                    *reinterpret_cast<u32x4*>(dst + 8 * c) = u32x4{w[0], w[1], w[2], w[3]};
                }
            } else {
                for (int t = 0; t < 32 && tok0 + t < int(p.M); ++t)
                    dst[t] = f2bf_bits(st[t * ld + d] * sc + bi);
            }
        }
        return;
    }
    const float* nw = which == 0 ? h.norm_q : h.norm_k;
    const int rt = lane >> 1, half = lane & 1, t = tok0 + rt;
    const float* row = st + rt * ld;
    // the lane's 64 channels: half*64 .. +64 (rope mode 0 / 2), or half*32 .. +32 and 64 + half*32 .. +32 (mode 1,
    // whose pairs (d, d + 64) then sit in one lane)
    const bool m1 = h.rope_mode == 1;
    auto load4 = [&](int d) {
        f32x4 x = *reinterpret_cast<const f32x4*>(row + d);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (p.wscale)
                x[j] *= p.wscale[nw0 + d + j];
            if (p.bias)
                x[j] += p.bias[nw0 + d + j];
        }
        return x;
    };
    float inv = 1.0f;
    if (nw) {
        float ss = 0.0f;
        for (int i = 0; i < 64; i += 4) {
            const int d = m1 ? (i < 32 ? half * 32 + i : 32 + half * 32 + i) : half * 64 + i;
            const f32x4 x = load4(d);
            ss += x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
        }
        ss += __shfl_xor(ss, 1, 64);
        inv = rsqrtf(ss / 128.0f + h.eps);
    }
    if (t >= int(p.M))
        return;
    auto normed = [&](int d) {
        f32x4 x = load4(d);
        if (nw)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                x[j] *= inv * nw[d + j];
        return x;
    };
    const float* cs = h.rope_mode ? h.rope + (int64_t(h.row0) + t) * 128 : nullptr;
    uint16_t* dst = (which == 0 ? h.q : h.k) +
                    (bh * (which == 0 ? h.q_pad : h.k_pad) + (which == 0 ? h.q_row0 : h.row0) + t) * 128;
    if (m1) {
        for (int i = 0; i < 32; i += 4) {
            const int d = half * 32 + i;
            f32x4 a = normed(d), b = normed(d + 64);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float co = cs[2 * (d + j)], si = cs[2 * (d + j) + 1], x = a[j], y = b[j];
                a[j] = x * co - y * si;
                b[j] = x * si + y * co;
            }
            *reinterpret_cast<u32x2*>(dst + d) = u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
            *reinterpret_cast<u32x2*>(dst + d + 64) = u32x2{pack_bf16x2(b[0], b[1]), pack_bf16x2(b[2], b[3])};
        }
        return;
    }
    for (int i = 0; i < 64; i += 4) {
        const int d = half * 64 + i;
        f32x4 a = normed(d);
        if (cs) {
#pragma unroll
            for (int j = 0; j < 4; j += 2) { // pair (d + j) / 2: (cos, sin) at cs[d + j], cs[d + j + 1]
                const float co = cs[d + j], si = cs[d + j + 1], x = a[j], y = a[j + 1];
                a[j] = x * co - y * si;
                a[j + 1] = x * si + y * co;
            }
        }
        *reinterpret_cast<u32x2*>(dst + d) = u32x2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
    }
}

template <int BM, int BN, bool kF8, bool kHeads>
__global__ __launch_bounds__(256, 1) void gemm_kernel(GemmP p)
{
    constexpr int TB = BM / 64, CB = BN / 64;  // 32-row MFMA blocks per wave along tokens / channels
    constexpr int RA = BM * 8 / 256;           // direct-load rounds for the activation tile (64 chunks per wave)
    constexpr int RW = BN * 8 / 256;           // ... for a bf16 weight tile
    constexpr int LW = BN * 4 / 256;           // 16-byte fp8 weight chunks per thread (register staged)
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * (BN + BM) * 64];
    uint16_t(*sW)[BN * 64] = reinterpret_cast<uint16_t(*)[BN * 64]>(smem);
    uint16_t(*sA)[BM * 64] = reinterpret_cast<uint16_t(*)[BM * 64]>(smem + 2 * BN * 64);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave & 1, wm = wave >> 1;

    // Tile of this workgroup: XCD-aware (round-robin dispatch puts workgroup i on XCD i % 8; give each XCD a
    // contiguous run of tiles), then grouped 8 m-tiles at a time so a run shares weight columns.
    const uint32_t total = p.tiles_m * p.tiles_n;
    uint32_t pid = blockIdx.x;
    if (total % 8 == 0)
        pid = (pid % 8) * (total / 8) + pid / 8;
    const uint32_t GM = 8, in_group = GM * p.tiles_n;
    const uint32_t first_m = (pid / in_group) * GM;
    const uint32_t gsize = min(p.tiles_m - first_m, GM);
    const uint32_t tm = first_m + (pid % in_group) % gsize, tn = (pid % in_group) / gsize;
    const int m0 = int(tm) * BM, n0 = int(tn) * BN;

    const uint16_t* A = p.a + int64_t(blockIdx.z) * p.sa;
    const int KT = int(p.K) / BK;

    // Direct loads: wave w's round i fills LDS chunks P = (i * 4 + w) * 64 + lane of the tile; chunk P holds
    // row P / 8 and logical k-chunk (P % 8) ^ (row & 7), so the lane loads that one.
    const uint16_t* ga[RA];
#pragma unroll
    for (int i = 0; i < RA; ++i) {
        const int P = (i * 4 + wave) * 64 + lane, row = P >> 3, kc = (P & 7) ^ (row & 7);
        ga[i] = A + int64_t(min(m0 + row, int(p.M) - 1)) * p.lda + kc * 8;
    }
    const uint16_t* gw[kF8 ? 1 : RW];
    const uint8_t* gw8[kF8 ? LW : 1];
    if constexpr (!kF8) {
#pragma unroll
        for (int i = 0; i < RW; ++i) {
            const int P = (i * 4 + wave) * 64 + lane, row = P >> 3, kc = (P & 7) ^ (row & 7);
            gw[i] = static_cast<const uint16_t*>(p.w) + int64_t(n0 + row) * p.K + kc * 8;
        }
    } else {
#pragma unroll
        for (int i = 0; i < LW; ++i) {
            const int c = tid + 256 * i, row = c >> 2, kc = c & 3;
            gw8[i] = static_cast<const uint8_t*>(p.w) + int64_t(n0 + row) * p.K + kc * 16;
        }
    }
    u32x4 rw[kF8 ? LW : 1];
    auto issue = [&](int kt, int buf) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < RA; ++i)
            load_lds16(ga[i] + k0, (lds_void*)&sA[buf][(i * 4 + wave) * 64 * 8]);
        if constexpr (!kF8) {
#pragma unroll
            for (int i = 0; i < RW; ++i)
                load_lds16(gw[i] + k0, (lds_void*)&sW[buf][(i * 4 + wave) * 64 * 8]);
        } else {
#pragma unroll
            for (int i = 0; i < LW; ++i)
                rw[i] = *reinterpret_cast<const u32x4*>(gw8[i] + k0);
        }
    };
    auto commit_f8 = [&](int buf) {
        if constexpr (kF8) {
#pragma unroll
            for (int i = 0; i < LW; ++i) {
                const int c = tid + 256 * i, row = c >> 2, kc = c & 3;
                u32x4 lo, hi;
                f8x16_to_bf16(rw[i], lo, hi);
                *reinterpret_cast<u32x4*>(&sW[buf][swz(row, 2 * kc)]) = lo;
                *reinterpret_cast<u32x4*>(&sW[buf][swz(row, 2 * kc + 1)]) = hi;
            }
        }
    };

    f32x16 acc[CB][TB];
#pragma unroll
    for (int i = 0; i < CB; ++i)
#pragma unroll
        for (int j = 0; j < TB; ++j)
            acc[i][j] = f32x16{};

    issue(0, 0);
    commit_f8(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int r32 = lane & 31, hk = lane >> 5;
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT)
            issue(kt + 1, buf ^ 1);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            bf16x8 wf[CB], af[TB];
            const int kc = ks * 2 + hk;
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                wf[cb] = *reinterpret_cast<const bf16x8*>(&sW[buf][swz(wn * (BN / 2) + cb * 32 + r32, kc)]);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
                af[tb] = *reinterpret_cast<const bf16x8*>(&sA[buf][swz(wm * (BM / 2) + tb * 32 + r32, kc)]);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
#pragma unroll
                for (int tb = 0; tb < TB; ++tb)
                    acc[cb][tb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[cb], af[tb], acc[cb][tb], 0, 0, 0);
        }
        if (kt + 1 < KT)
            commit_f8(buf ^ 1);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }

    // ---- epilogue through LDS: per 32-token block, each wave stages its 32 x WC slice (fp32, padded rows), then
    // reads it back row-contiguous: two lanes per token, WC/2 channels each ----
    constexpr int WC = BN / 2, LDW = WC + 4, CW = WC / 2;
    static_assert(4 * 32 * LDW * 4 <= 2 * (BN + BM) * 64 * 2, "staging does not fit");
    float* st = reinterpret_cast<float*>(smem) + wave * 32 * LDW;
    const int rt = lane >> 1, half = lane & 1;
    const int64_t zc = int64_t(blockIdx.z) * p.sc;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<f32x4*>(st + r32 * LDW + cb * 32 + 8 * i + 4 * hk) =
                    f32x4{acc[cb][tb][4 * i], acc[cb][tb][4 * i + 1], acc[cb][tb][4 * i + 2], acc[cb][tb][4 * i + 3]};
        __syncthreads();
        const int tok0 = m0 + wm * (BM / 2) + tb * 32;
        if constexpr (kHeads) {
            epi_heads(p, st, LDW, tok0, n0 + wn * WC, lane);
        } else {
            const int t = tok0 + rt;
            if (t < int(p.M)) {
                const int64_t rowoff = zc + int64_t(t) * p.ldc;
                const bool alt = (uint32_t(t) % p.seg_rows) < p.split;
                const int ch0 = n0 + wn * WC + half * CW;
                for (int j = 0; j < CW; j += 4)
                    epi_store(p, rowoff, ch0 + j, alt, *reinterpret_cast<const f32x4*>(st + rt * LDW + half * CW + j));
            }
        }
        __syncthreads();
    }
}

template <int BM, int BN, bool kF8, bool kHeads = false>
hipError_t launch(const GemmP& p, uint32_t batch, hipStream_t s)
{
    GemmP q = p;
    q.tiles_m = cdiv(p.M, BM);
    q.tiles_n = p.N / BN;
    gemm_kernel<BM, BN, kF8, kHeads><<<dim3(q.tiles_m * q.tiles_n, 1, batch), 256, 0, s>>>(q);
    return hipGetLastError();
}

} // namespace gemm_detail
} // namespace mk

using namespace mk;
using namespace mk::gemm_detail;

extern "C" mk_status mk_gemm(const mk_gemm_args* a, void* stream)
{
    if (!a || !a->a || !a->w || (!a->c && a->epilogue != MK_EPI_HEADS))
        return fail(MK_ERR_ARG, "gemm: null argument");
    if (a->K % 64 || a->N % 64 || a->K == 0 || a->N == 0)
        return fail(MK_ERR_ARG, "gemm: K and N must be nonzero multiples of 64 (K " + std::to_string(a->K) + ", N " +
                                    std::to_string(a->N) + ")");
    if (a->w_dtype != MK_BF16 && a->w_dtype != MK_FP8_E4M3)
        return fail(MK_ERR_ARG, "gemm: weights must be bf16 or fp8-e4m3");
    if (a->lda % 8 || (reinterpret_cast<uintptr_t>(a->a) & 15) || (reinterpret_cast<uintptr_t>(a->w) & 15))
        return fail(MK_ERR_ARG, "gemm: A and W must be 16-byte aligned with lda a multiple of 8");
    if (a->epilogue > MK_EPI_HEADS)
        return fail(MK_ERR_ARG, "gemm: unknown epilogue");
    const bool gated = a->epilogue == MK_EPI_GATE_ADD || a->epilogue == MK_EPI_GATE_TANH;
    if (gated && !a->gate)
        return fail(MK_ERR_ARG, "gemm: gated epilogue without a gate");
    if (a->M == 0 || a->batch == 0)
        return MK_OK;
    GemmP p{};
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
    p.c_bf16 = a->c_dtype == MK_BF16;
    if (a->w_dtype == MK_FP8_E4M3 && !a->wscale)
        return fail(MK_ERR_ARG, "gemm: fp8 weights need per-channel scales");
    const bool f8 = a->w_dtype == MK_FP8_E4M3;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (a->epilogue == MK_EPI_HEADS) {
        const mk_heads_args* h = a->heads;
        if (!h || !h->q || !h->k || !h->vt || h->head_dim != 128 || a->N % 256 || (a->N / 3) % 128 ||
            a->N / 3 != h->heads * 128 || h->rope_mode > 2 || (h->rope_mode && !h->rope) ||
            uint64_t(h->row0) + a->M > h->k_pad || uint64_t(h->q_row0) + a->M > h->q_pad)
            return fail(MK_ERR_ARG, "gemm heads epilogue: needs q, k, vt, head_dim 128, N = 3 * heads * 128 a multiple "
                                    "of 256, and row0 + M within the padded rows");
        p.hp = HeadsP{static_cast<uint16_t*>(h->q), static_cast<uint16_t*>(h->k), static_cast<uint16_t*>(h->vt),
                      h->heads, h->q_pad, h->k_pad, h->row0, h->q_row0, h->rope_mode, a->N / 3, h->norm_q, h->norm_k, h->rope,
                      h->eps};
        e = f8 ? launch<256, 256, true, true>(p, a->batch, s) : launch<256, 256, false, true>(p, a->batch, s);
    } else if (a->N % 256 == 0 && uint64_t(cdiv(a->M, 256)) * (a->N / 256) * a->batch >= 512) {
        e = f8 ? launch<256, 256, true>(p, a->batch, s) : launch<256, 256, false>(p, a->batch, s);
    } else if (a->N % 128 == 0) {
        e = f8 ? launch<256, 128, true>(p, a->batch, s) : launch<256, 128, false>(p, a->batch, s);
    } else {
        e = f8 ? launch<256, 64, true>(p, a->batch, s) : launch<256, 64, false>(p, a->batch, s);
    }
    if (e != hipSuccess)
        return hip_check(e, "gemm launch");
    return MK_OK;
}
