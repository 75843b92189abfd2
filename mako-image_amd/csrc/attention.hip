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
// into a ring of three buffers, with XOR swizzles chosen so every fragment read is bank-conflict free: K [key][d]
// chunk c at c ^ (key & 15), V^T [d][key] chunk c at c ^ ((d >> 1) & 7). V^T holds its keys in the vt_col order, so a
// lane's 8 P V keys are one 16-byte read. Within a wave the next tile's S^T MFMAs
// are issued alongside the current tile's softmax, so the matrix cores and the VALUs work at the same time.
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
constexpr int kNB = 3;   // K / V^T tile buffers (a ring: load t + 2 while t + 1 is read and t's V is in use)
// Lazy rescaling: the running max the exponentials use moves only when a row max exceeds it by more than 2^8, so
// P <= 256 (exact enough in bf16, far from fp32 overflow) and the output is rescaled on few tiles.
constexpr float kLazy = 8.0f;

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

__device__ inline uint32_t cvt_bf16x2(float a, float b)
{
    const bf16x2 v = {(__bf16)a, (__bf16)b}; // v_cvt_pk_bf16_f32: round to nearest even
    return __builtin_bit_cast(uint32_t, v);
}

template <int D>
__global__ __launch_bounds__(256, 1) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_kernel(AttnP p)
{
    constexpr int DS = D / 16;         // 16-wide d steps of K Q^T
    constexpr int DT = D / 32;         // 32-row d blocks of O^T
    constexpr int KC = D / 8;          // 16-byte chunks per K row
    constexpr int RK = kKT * KC / 256; // direct-load rounds for a K tile (64 chunks per wave per round)
    constexpr int RV = D * 8 / 256;    // ... for a V^T tile (D rows of 64 keys = 8 chunks)
    __shared__ __attribute__((aligned(16))) uint16_t sK[kNB][kKT * D];
    __shared__ __attribute__((aligned(16))) uint16_t sV[kNB][D * kKT];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r32 = lane & 31, hk = lane >> 5;
    // K rows are D/8 16-byte chunks; a fragment read serves 16 consecutive keys at one chunk a cycle (64 banks):
    // 256-byte rows (D = 128) need 16 distinct chunks (key & 15), 128-byte rows (D = 64) take the two bank halves
    // from the row parity and 8 distinct chunks from (key >> 1) & 7.
    auto kswz = [](int key, int c) { return KC == 16 ? c ^ (key & 15) : c ^ ((key >> 1) & 7); };
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
        const int P = (i * 4 + wave) * 64 + lane, key = P / KC, c = kswz(key, P % KC);
        gk[i] = K + int64_t(key) * D + c * 8;
    }
    const uint16_t* gv[RV];
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        const int P = (i * 4 + wave) * 64 + lane, d = P >> 3, c = (P & 7) ^ ((d >> 1) & 7);
        gv[i] = VT + int64_t(d) * p.k_pad + c * 8;
    }
    const int ntiles = int((p.n_k + kKT - 1) / kKT);
    auto issue = [&](int t) {
        // past the end: the last tile again, into the free slot (keeps the loop free of branches)
        const int buf = t % kNB, k0 = min(t, ntiles - 1) * kKT;
#pragma unroll
        for (int i = 0; i < RK; ++i)
            load_lds16(gk[i] + int64_t(k0) * D, (lds_void*)&sK[buf][(i * 4 + wave) * 512]);
#pragma unroll
        for (int i = 0; i < RV; ++i)
            load_lds16(gv[i] + k0, (lds_void*)&sV[buf][(i * 4 + wave) * 512]);
    };

    // S^T = K Q^T for the 32 keys kt*32 .. of a tile: sacc[qt], value r <-> key k0 + kt*32 + 8(r/4) + 4hk + r%4
    auto qk = [&](int buf, int kt, f32x16 (&sacc)[2]) {
        sacc[0] = f32x16{};
        sacc[1] = f32x16{};
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
            const int key = kt * 32 + r32, c = kswz(key, ds * 2 + hk);
            const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sK[buf][key * D + c * 8]);
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
                sacc[qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[qt][ds], sacc[qt], 0, 0, 0);
        }
    };

    f32x16 oacc[2][DT];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
            oacc[qt][dt] = f32x16{};
    float m[2] = {-1e30f, -1e30f}, l[2] = {0.0f, 0.0f};
    const int qpos[2] = {int(p.q_pos0) + q0 + r32, int(p.q_pos0) + q0 + 32 + r32};
    // rows before `block` see keys up to themselves: a mask is needed on keys past the wave's first such row
    const bool wave_causal = uint32_t(int(p.q_pos0) + q0) < p.block;

    // softmax of 32 keys' scores (from k0) -> P^T fragments pb[qt][0..1]; rescales O when the running max moves
    auto softmax = [&](f32x16 (&sacc)[2], int k0, u32x4 (&pb)[2][2]) {
        if (k0 + 32 > int(p.n_k) || (wave_causal && k0 + 31 > int(p.q_pos0) + q0)) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = k0 + 8 * (r / 4) + 4 * hk + (r % 4);
                    if (key >= int(p.n_k) || (uint32_t(qpos[qt]) < p.block && key > qpos[qt]))
                        sacc[qt][r] = -__builtin_inff();
                }
        }
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            float mx = -1e30f;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                mx = fmaxf(mx, sacc[qt][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * p.c;
            if (__any(mx > m[qt] + kLazy)) {
                const float mn = fmaxf(m[qt], mx);
                const float alpha = __builtin_amdgcn_exp2f(m[qt] - mn);
                m[qt] = mn;
                l[qt] *= alpha;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        oacc[qt][dt][r] *= alpha;
            }
            float s = 0.0f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float e = __builtin_amdgcn_exp2f(fmaf(sacc[qt][r], p.c, -m[qt]));
                sacc[qt][r] = e;
                s += e;
            }
            l[qt] += s;
            // P^T fragment of 16-key step st: accumulators 8 st .. 8 st + 7
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const int o = 8 * st;
                const f32x16& a = sacc[qt];
                pb[qt][st] = u32x4{cvt_bf16x2(a[o], a[o + 1]), cvt_bf16x2(a[o + 2], a[o + 3]),
                                   cvt_bf16x2(a[o + 4], a[o + 5]), cvt_bf16x2(a[o + 6], a[o + 7])};
            }
        }
    };

    // O^T += V^T P^T over 32 keys kt*32 ..: A = V^T rows d = dt*32 + r32
    auto pv = [&](int buf, int kt, const u32x4 (&pb)[2][2]) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int d = dt * 32 + r32, sw = (d >> 1) & 7;
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                // keys 16 s2 + 4hk + 0..3 and 16 s2 + 8 + 4hk + 0..3 are V^T columns 16 s2 + 8hk .. +8 (vt_col)
                const int s2 = 2 * kt + st;
                const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&sV[buf][d * kKT + (((2 * s2 + hk) ^ sw) << 3)]);
#pragma unroll
                for (int qt = 0; qt < 2; ++qt)
                    oacc[qt][dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, __builtin_bit_cast(bf16x8, pb[qt][st]),
                                                                          oacc[qt][dt], 0, 0, 0);
            }
        }
    };

    // Pipeline over 32-key halves of 64-key tiles held in a ring of three LDS buffers: while the VALUs run one half's
    // softmax, the matrix cores compute the next half's S^T; tile t + 1 is resident and tile t + 2 loading during
    // tile t.
    issue(0);
    issue(1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    f32x16 s_a[2], s_b[2];
    qk(0, 0, s_a);
    for (int t = 0; t < ntiles; ++t) {
        if (t > 0) {
            __builtin_amdgcn_s_waitcnt(0); // tile t + 1 resident; every wave done with tile t - 1's buffer
            __syncthreads();
        }
        issue(t + 2);
        const int buf = t % kNB;
        u32x4 pb[2][2];
        qk(buf, 1, s_b);
        softmax(s_a, t * kKT, pb);
        pv(buf, 0, pb);
        qk((t + 1) % kNB, 0, s_a); // past the last tile this reads a resident buffer and is discarded
        softmax(s_b, t * kKT + 32, pb);
        pv(buf, 1, pb);
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
                    u32x2{cvt_bf16x2(a[4 * i] * inv, a[4 * i + 1] * inv), cvt_bf16x2(a[4 * i + 2] * inv, a[4 * i + 3] * inv)};
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
