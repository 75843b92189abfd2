// attention: joint softmax(Q K^T scale) V on gfx950 bf16 MFMA (v_mfma_f32_32x32x16_bf16), online softmax in fp32.
//
// Each wave owns 64 queries (two 32-query sub-tiles) and computes S^T = K Q^T: the MFMA's A operand is a K tile
// (rows = keys), its B operand the wave's Q held in registers for the whole pass (cols = queries). A lane then holds
// 16 scores of one query per 32-key block, so the row max is lane-local plus one swap with lane ^ 32, and the
// probabilities convert in registers to the B operand of O^T = V^T P^T: the A operand is read from a V^T tile (rows =
// head dims, keys contiguous). The P^T slots permute keys (slot 8h + 4ii + j <-> key 16s + 8ii + 4h + j); the V^T
// fragment reads use the same permutation, so the dot products are unchanged.
//
// A workgroup of 4 waves (256 queries) shares each 64-key K and V^T tile, staged in LDS by direct global->LDS loads
// (double-buffered, the next tile in flight during the current tile's MFMAs) with XOR swizzles chosen so every
// fragment read is bank-conflict free: K [key][d] chunk c at c ^ (key & 15), V^T [d][key] chunk c at
// c ^ ((d >> 1) & 7).
#include "common.hpp"

namespace mk {

namespace {

struct AttnP {
    const uint16_t *q, *k, *vt;
    uint16_t* out;
    uint32_t heads, n_q, q_pad, n_k, k_pad, q_pos0, block;
    int64_t ldo, so;
    float c; // scale * log2(e)
};

constexpr int kQW = 64;  // queries per wave
constexpr int kKT = 64;  // keys per tile

template <int D>
__global__ __launch_bounds__(256, 1) void attn_kernel(AttnP p)
{
    constexpr int DS = D / 16;        // 16-wide d steps of Q K^T
    constexpr int DT = D / 32;        // 32-row d blocks of O^T
    constexpr int KC = D / 8;         // 16-byte chunks per K row
    constexpr int RK = kKT * KC / 256; // direct-load rounds for a K tile (64 chunks per wave per round)
    constexpr int RV = D * 8 / 256;    // ... for a V^T tile (D rows of 64 keys = 8 chunks)
    __shared__ __attribute__((aligned(16))) uint16_t sK[2][kKT * D];
    __shared__ __attribute__((aligned(16))) uint16_t sV[2][D * kKT];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r32 = lane & 31, hk = lane >> 5;
    const uint32_t head = blockIdx.y, bi = blockIdx.z;
    const int64_t bh = int64_t(bi) * p.heads + head;
    const uint16_t* Q = p.q + bh * p.q_pad * D;
    const uint16_t* K = p.k + bh * p.k_pad * D;
    const uint16_t* VT = p.vt + bh * int64_t(D) * p.k_pad;
    const int q0 = int(blockIdx.x) * 4 * kQW + wave * kQW;

    // Q fragments (B operand of S^T): query q0 + qt*32 + r32, d = ds*16 + hk*8 .. +8.
    bf16x8 qf[2][DS];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = min(q0 + qt * 32 + r32, int(p.n_q) - 1);
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
            qf[qt][ds] = *reinterpret_cast<const bf16x8*>(Q + int64_t(qi) * D + ds * 16 + hk * 8);
    }

    // Direct-load sources: wave w, round i fills chunks P = (i*4 + w)*64 + lane.
    const uint16_t* gk[RK];
#pragma unroll
    for (int i = 0; i < RK; ++i) {
        const int P = (i * 4 + wave) * 64 + lane, key = P / KC, c = (P % KC) ^ (key & (KC - 1));
        gk[i] = K + int64_t(key) * D + c * 8;
    }
    const uint16_t* gv[RV];
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        const int P = (i * 4 + wave) * 64 + lane, d = P >> 3, c = (P & 7) ^ ((d >> 1) & 7);
        gv[i] = VT + int64_t(d) * p.k_pad + c * 8;
    }
    auto issue = [&](int t, int buf) {
        const int k0 = t * kKT;
#pragma unroll
        for (int i = 0; i < RK; ++i)
            load_lds16(gk[i] + int64_t(k0) * D, (lds_void*)&sK[buf][(i * 4 + wave) * 512]);
#pragma unroll
        for (int i = 0; i < RV; ++i)
            load_lds16(gv[i] + k0, (lds_void*)&sV[buf][(i * 4 + wave) * 512]);
    };

    f32x16 oacc[2][DT];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
            oacc[qt][dt] = f32x16{};
    float m[2] = {-1e30f, -1e30f}, l[2] = {0.0f, 0.0f};
    const int qpos[2] = {int(p.q_pos0) + q0 + r32, int(p.q_pos0) + q0 + 32 + r32};

    const int ntiles = int((p.n_k + kKT - 1) / kKT);
    issue(0, 0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1, k0 = t * kKT;
        if (t + 1 < ntiles)
            issue(t + 1, buf ^ 1);
        // ---- S^T = K Q^T: sacc[qt][kt], value r <-> key k0 + kt*32 + 8(r/4) + 4hk + r%4 ----
        f32x16 sacc[2][2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
                sacc[qt][kt] = f32x16{};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            bf16x8 kf[2];
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const int key = kt * 32 + r32, c = (ds * 2 + hk) ^ (key & (KC - 1));
                kf[kt] = *reinterpret_cast<const bf16x8*>(&sK[buf][key * D + c * 8]);
            }
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
                    sacc[qt][kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kt], qf[qt][ds], sacc[qt][kt], 0, 0, 0);
        }
        // ---- mask: padding keys, and the causal prefix (rows before `block` see keys up to themselves) ----
        const bool pad = k0 + kKT > int(p.n_k);
        const bool causal = uint32_t(int(p.q_pos0) + q0) < p.block && k0 + kKT - 1 > int(p.q_pos0) + q0;
        if (pad || causal) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = k0 + kt * 32 + 8 * (r / 4) + 4 * hk + (r % 4);
                        const bool hide =
                            key >= int(p.n_k) || (uint32_t(qpos[qt]) < p.block && key > qpos[qt]);
                        if (hide)
                            sacc[qt][kt][r] = -__builtin_inff();
                    }
        }
        // ---- online softmax (scaled by c into the log2 domain) ----
        bf16x8 pb[2][4];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            float mx = -1e30f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    mx = fmaxf(mx, sacc[qt][kt][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float mn = fmaxf(m[qt], mx * p.c);
            const float alpha = exp2f(m[qt] - mn);
            m[qt] = mn;
            float s = 0.0f;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float e = exp2f(fmaf(sacc[qt][kt][r], p.c, -mn));
                    sacc[qt][kt][r] = e;
                    s += e;
                }
            l[qt] = l[qt] * alpha + s;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    oacc[qt][dt][r] *= alpha;
            // P^T fragments: step s (16 keys) = accumulators sacc[s/2][8(s%2) .. +8]
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const f32x16& a = sacc[qt][st / 2];
                const int o = 8 * (st % 2);
                u32x4 w{pack_bf16x2(a[o], a[o + 1]), pack_bf16x2(a[o + 2], a[o + 3]), pack_bf16x2(a[o + 4], a[o + 5]),
                        pack_bf16x2(a[o + 6], a[o + 7])};
                pb[qt][st] = __builtin_bit_cast(bf16x8, w);
            }
        }
        // ---- O^T += V^T P^T: A = V^T rows d = dt*32 + r32, keys 16s + 4hk + 0..3 and 16s + 8 + 4hk + 0..3 ----
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int d = dt * 32 + r32, sw = (d >> 1) & 7;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const u32x2 lo = *reinterpret_cast<const u32x2*>(&sV[buf][d * kKT + (((2 * st) ^ sw) << 3) + 4 * hk]);
                const u32x2 hi =
                    *reinterpret_cast<const u32x2*>(&sV[buf][d * kKT + (((2 * st + 1) ^ sw) << 3) + 4 * hk]);
                const bf16x8 vf = __builtin_bit_cast(bf16x8, u32x4{lo[0], lo[1], hi[0], hi[1]});
#pragma unroll
                for (int qt = 0; qt < 2; ++qt)
                    oacc[qt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pb[qt][st], oacc[qt][dt], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }

    // ---- normalise and write: lane holds query q0 + qt*32 + r32, dims dt*32 + 8i + 4hk + j ----
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const float lt = l[qt] + __shfl_xor(l[qt], 32, 64);
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        const int qi = q0 + qt * 32 + r32;
        if (qi >= int(p.n_q))
            continue;
        uint16_t* o = p.out + int64_t(bi) * p.so + int64_t(qi) * p.ldo + int64_t(head) * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const f32x16& a = oacc[qt][dt];
                *reinterpret_cast<u32x2*>(o + dt * 32 + 8 * i + 4 * hk) =
                    u32x2{pack_bf16x2(a[4 * i] * inv, a[4 * i + 1] * inv),
                          pack_bf16x2(a[4 * i + 2] * inv, a[4 * i + 3] * inv)};
            }
    }
}

} // namespace
} // namespace mk

using namespace mk;

extern "C" mk_status mk_attention(const void* q, const void* k, const void* vt, void* out, uint32_t batch,
                                  uint32_t heads, uint32_t d, uint32_t n_q, uint32_t q_pad, uint32_t n_k,
                                  uint32_t k_pad, int64_t ldo, int64_t stride_o, uint32_t q_pos0, uint32_t block,
                                  float scale, void* stream)
{
    if (!q || !k || !vt || !out)
        return fail(MK_ERR_ARG, "attention: null pointer");
    if (d != 64 && d != 128)
        return fail(MK_ERR_ARG, "attention: head dim must be 64 or 128");
    if (n_q == 0 || n_k == 0 || n_q > q_pad || k_pad % kKT || n_k > k_pad)
        return fail(MK_ERR_ARG, "attention: need 0 < n_q <= q_pad, 0 < n_k <= k_pad, k_pad a multiple of 64");
    if (ldo % 4 || (reinterpret_cast<uintptr_t>(out) & 7))
        return fail(MK_ERR_ARG, "attention: output rows must be 8-byte aligned");
    AttnP p{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(vt),
            static_cast<uint16_t*>(out), heads, n_q, q_pad, n_k, k_pad, q_pos0, block, ldo, stride_o,
            scale * 1.4426950408889634f};
    const dim3 grid(cdiv(n_q, 4 * kQW), heads, batch);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (d == 128)
        attn_kernel<128><<<grid, 256, 0, s>>>(p);
    else
        attn_kernel<64><<<grid, 256, 0, s>>>(p);
    MK_LAUNCH_CHECK("attention");
    return MK_OK;
}
