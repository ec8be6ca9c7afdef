// k_lmhead.hip -- the model's LM head with the sampler's first statistic in
// its epilogue.
//
// Reference: mini_engine/model/qwen2.py:176-183, F.linear(h[last_idx],
// self.lm_head): logits[r, v] = sum_k h[r, k] * lm_head[v, k], with the tied
// embedding lm_head = model.embed_tokens.weight (qwen2.py:92-96), fp32
// (mini_engine/engine.py:29).  Here:
//
//   logits[r, v] = sum_k hidden[r, k] * weight[v, k]          fp32 on MFMA
//   best[r]      = max over v of (gkey(logits[r, v]) << 32) | ~v
//
// gkey is the sampler's greedy key (NaN highest, -0 as +0), so best[r] names
// the first index of the row's maximum, the token sampling.py:47-48 returns
// for a greedy row; the sampler (mxs_sample_head) takes it from there and
// does not read such a row's logits again.  Each workgroup reduces its
// columns' maxima per row and adds them with one 64-bit atomic max per row.
//
// Two kernels:
//   k_lmhead_narrow  B <= 16 (decode batches): bound by the weight stream
//                    (151,936 x 896 x 4 B = 545 MB for the reference model);
//                    weights go straight from HBM into MFMA operands.
//   k_lmhead         larger batches: each workgroup owns LH_NT = 128
//                    vocabulary columns and up to 256 rows, so the weights
//                    stream once per 256 rows.  Per stage of LH_KC = 32
//                    features the weight tile (128 x 32) and the hidden tile
//                    (rows x 32) are staged in LDS (rows padded to 33 floats:
//                    conflict-free column reads), the next stage's tiles are
//                    loaded into registers while the current one is
//                    multiplied, and each wave accumulates a 32-column slice
//                    for every block of 32 rows (32x32x2 MFMA, 16 floats per
//                    lane per block).
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mxs_device.h"
#include "sampler_params.h"

namespace mxs {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int LH_NT = 128;              // vocabulary columns per workgroup: 4 waves x 32
constexpr int LH_KC = 32;               // features per stage
constexpr int LH_MBMAX = 8;             // row blocks of 32 per workgroup: at most 256 rows
constexpr int LH_THREADS = 256;
constexpr int LH_PAD = LH_KC + 1;
static_assert(4 * LH_MBMAX * 32 * 8 <= LH_NT * LH_PAD * 4, "the row maxima fit in the weight tile");

// the sampler's greedy key of a logit: NaN is the maximum, -0 equals +0
__device__ __forceinline__ uint32_t gkey(float x) { return (x != x) ? 0xFFFFFFFFu : vkey(x); }

template <int MB>
struct LhTiles {
    f32x4 w[4];     // weight rows (t >> 3) + 32 j, features 4 (t & 7) .. + 3
    f32x4 h[MB];    // hidden rows (t >> 3) + 32 i, same features
};

// One stage's tiles from global memory into registers: rows past the
// matrix read its last row (their results are dropped), features past D
// read as zeros.  Rows of both matrices are 16-byte aligned (checked by the
// caller), so the 16-byte vector holding feature k < D lies in the same
// aligned block as that feature: whole vectors are read, with no branch
// (a branch around a load makes the compiler wait for the loads before
// it), and the lanes past D are replaced by zeros.  A vector wholly past D
// reads the row's first vector instead.
template <int MB>
__device__ __forceinline__ void lh_load(LhTiles<MB>& t, const float* __restrict__ H, int nr, int r0, long long ldh,
                                        const float* __restrict__ W, int V, long long ldw, int n0, int k0, int D)
{
    const int tid = threadIdx.x;
    const int k = k0 + (tid & 7) * 4;
    const int ka = k < D ? k : 0;
    auto rd = [&](const float* row) -> f32x4 { return *(const f32x4*)(row + ka); };
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int v = n0 + (tid >> 3) + 32 * j;
        v = v < V ? v : V - 1;
        t.w[j] = rd(W + (size_t)v * (size_t)ldw);
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        const int row = (tid >> 3) + 32 * i;
        const int rr = row < nr ? row : nr - 1;
        t.h[i] = rd(H + (size_t)(r0 + rr) * (size_t)ldh);
    }
    if (k + 3 >= D) {   // (the last stage's tail only; after the loads were issued)
        const bool x = k < D, y = k + 1 < D, z = k + 2 < D;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            t.w[j].x = x ? t.w[j].x : 0.0f; t.w[j].y = y ? t.w[j].y : 0.0f;
            t.w[j].z = z ? t.w[j].z : 0.0f; t.w[j].w = 0.0f;
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
            t.h[i].x = x ? t.h[i].x : 0.0f; t.h[i].y = y ? t.h[i].y : 0.0f;
            t.h[i].z = z ? t.h[i].z : 0.0f; t.h[i].w = 0.0f;
        }
    }
}

template <int MB>
__device__ __forceinline__ void lh_store(const LhTiles<MB>& t, float* ws, float* hs)
{
    const int tid = threadIdx.x;
    const int c = (tid & 7) * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float* d = ws + ((tid >> 3) + 32 * j) * LH_PAD + c;
        d[0] = t.w[j].x; d[1] = t.w[j].y; d[2] = t.w[j].z; d[3] = t.w[j].w;
    }
#pragma unroll
    for (int i = 0; i < MB; ++i) {
        float* d = hs + ((tid >> 3) + 32 * i) * LH_PAD + c;
        d[0] = t.h[i].x; d[1] = t.h[i].y; d[2] = t.h[i].z; d[3] = t.h[i].w;
    }
}

// MB: row blocks of 32 this instance holds (the launch takes the smallest
// that covers its rows, so that small batches keep few registers live)
template <int MB>
__global__ __launch_bounds__(LH_THREADS) void k_lmhead(const float* __restrict__ H, int B, int D, long long ldh,
                                                       const float* __restrict__ W, int V, long long ldw,
                                                       float* __restrict__ C, long long ldc, u64* __restrict__ best)
{
    __shared__ __align__(16) float ws[LH_NT * LH_PAD];   // (also the row maxima: 4 x MB x 32 u64 <= its size)
    __shared__ __align__(16) float hs[MB * 32 * LH_PAD];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int n0 = blockIdx.x * LH_NT;
    const int r0 = blockIdx.y * (MB * 32);
    const int nr = B - r0 < MB * 32 ? B - r0 : MB * 32;
    f32x16 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[mb][j] = 0.0f;

    LhTiles<MB> t;
    lh_load(t, H, nr, r0, ldh, W, V, ldw, n0, 0, D);
    // MFMA 32x32x2 operands: lane l supplies A[l % 32][l / 32] (a row of the
    // block, feature kk + l / 32) and B[l / 32][l % 32] (a column of the slice)
    const int arow = lane & 31, akk = lane >> 5;
    // (every block of the instance is multiplied, also blocks past the
    // batch, which hold copies of its last row: no branch keeps the LDS
    // reads from running ahead of the products)
    for (int k0 = 0; k0 < D; k0 += LH_KC) {
        __syncthreads();   // (the previous stage's reads of ws and hs are done)
        lh_store(t, ws, hs);
        __syncthreads();
        if (k0 + LH_KC < D) lh_load(t, H, nr, r0, ldh, W, V, ldw, n0, k0 + LH_KC, D);
#pragma unroll
        for (int kk = 0; kk < LH_KC; kk += 2) {
            const float b = ws[(32 * w + arow) * LH_PAD + kk + akk];
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const float a = hs[(32 * mb + arow) * LH_PAD + kk + akk];
                acc[mb] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[mb], 0, 0, 0);
            }
        }
    }

    // epilogue: lane l, accumulator register j of block mb holds row
    // 32 mb + 8 (j / 4) + 4 (l / 32) + j % 4 and column l % 32 of the slice.
    // Each row's maximum over the workgroup's 128 columns is reduced in LDS
    // (the waves' slices) before one atomic per row and workgroup, which is
    // skipped when best[m] already holds a larger key (best only grows, so
    // any value read bounds the final one from below).
    __syncthreads();   // (ws is reused for the waves' row maxima)
    u64* rowmax = (u64*)ws;   // [4][MB * 32]
    const int n = n0 + 32 * w + arow;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int mi = 32 * mb + 8 * (j >> 2) + 4 * akk + (j & 3);   // row within the workgroup
            const int m = r0 + mi;
            const float x = acc[mb][j];
            const bool in = m < B && n < V;
            if (in) C[(size_t)m * (size_t)ldc + (size_t)n] = x;
            u64 key = in ? (((u64)gkey(x) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)n)) : 0ull;
#pragma unroll
            for (int s = 1; s < 32; s <<= 1) {   // the 32 lanes of this half hold the same row
                const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)key, s, 64);
                const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(key >> 32), s, 64);
                const u64 o = ((u64)hi << 32) | lo;
                key = o > key ? o : key;
            }
            if (arow == 0) rowmax[w * (MB * 32) + mi] = key;
        }
    }
    __syncthreads();
    for (int mi = tid; mi < nr; mi += LH_THREADS) {
        u64 key = rowmax[mi];
#pragma unroll
        for (int v = 1; v < 4; ++v) {
            const u64 o = rowmax[v * (MB * 32) + mi];
            key = o > key ? o : key;
        }
        const u64 cur = __hip_atomic_load(&best[r0 + mi], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (key > cur) atomicMax(&best[r0 + mi], key);
    }
}

// ------------------------------------------------------------ small batches
//
// Up to 32 rows the product is bound by the weight stream (545 MB for the
// reference model's head), and staging weight tiles through LDS behind
// barriers leaves too few bytes in flight.  Here each wave owns 16 NT
// vocabulary rows (NT tiles of 16) over all D features and streams them
// straight into registers, NP chunks ahead, with no LDS and no barrier
// until the epilogue.  A chunk is 16 NV features of each row: lane l holds
// row l % 16 of a tile and the NV 16-byte vectors at features
// 16 NV c + 4 NV q .. + 4 NV - 1 (q = l / 16), so the four lanes of a row
// read 16 NV contiguous floats of it.  The 16x16x4 MFMA contracts, at step
// e of the chunk, the features 16 NV c + 4 NV q + e of the four quarters q:
// each lane's own vector elements are its operands, and the hidden rows
// (clamped into the batch, from the caches: every wave reads the same
// ones, once per chunk for all NT tiles) are read the same way.  D is a
// multiple of 16 NV NP (the launcher checks), so no chunk is partial and
// the pipeline's rounds divide them.
template <int MQ, int NV, int NP, int NT>   // MQ: 16-row batch blocks (B <= 16 MQ)
__global__ __launch_bounds__(LH_THREADS) void k_lmhead_narrow(const float* __restrict__ H, int B, int D, long long ldh,
                                                              const float* __restrict__ W, int V, long long ldw,
                                                              float* __restrict__ C, long long ldc,
                                                              u64* __restrict__ best)
{
    constexpr int CF = 16 * NV;   // features per chunk
    __shared__ u64 rowmax[4][MQ * 16];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int q = lane >> 4, j = lane & 15;
    const int nb = (blockIdx.x * 4 + w) * (16 * NT);   // the wave's first vocabulary row
    const float* wr[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
        wr[t] = W + (size_t)(nb + 16 * t + j < V ? nb + 16 * t + j : V - 1) * (size_t)ldw + 4 * NV * q;
    const float* hr[MQ];
#pragma unroll
    for (int i = 0; i < MQ; ++i)
        hr[i] = H + (size_t)(16 * i + j < B ? 16 * i + j : B - 1) * (size_t)ldh + 4 * NV * q;
    const int nch = D / CF;

    f32x4 acc[NT][MQ];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < MQ; ++i) acc[t][i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 bw[NP][NT][NV], bh[NP][MQ][NV];
    // chunk c's vectors into slot p.  The chunks past the last (issued by
    // the pipeline's last round, never used) read the cached hidden rows
    // instead of more weights.  (No branch: a branch around a load makes
    // the compiler wait for every load in flight at the join.)
    auto issue = [&](int p, int c) {
        const bool live = c < nch;
        const int k = live ? CF * c : 0;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float* a = (live ? wr[t] : hr[0]) + k;
#pragma unroll
            for (int v = 0; v < NV; ++v) bw[p][t][v] = *(const f32x4*)(a + 4 * v);
        }
#pragma unroll
        for (int i = 0; i < MQ; ++i)
#pragma unroll
            for (int v = 0; v < NV; ++v) bh[p][i][v] = *(const f32x4*)(hr[i] + k + 4 * v);
    };
#pragma unroll
    for (int p = 0; p < NP; ++p) issue(p, p);
    __builtin_amdgcn_sched_barrier(0);
    for (int c0 = 0; c0 < nch; c0 += NP) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
#pragma unroll
            for (int v = 0; v < NV; ++v)
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int i = 0; i < MQ; ++i)
#pragma unroll
                        for (int t = 0; t < NT; ++t)
                            acc[t][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(bh[p][i][v][e], bw[p][t][v][e],
                                                                              acc[t][i], 0, 0, 0);
            issue(p, c0 + p + NP);
            __builtin_amdgcn_sched_barrier(0);   // (the loads stay NP chunks ahead of their use)
        }
    }

    // epilogue: lane l, register r of block i holds batch row 16 i + 4 (l / 16)
    // + r and vocabulary row l % 16 of the tile
#pragma unroll
    for (int i = 0; i < MQ; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int mi = 16 * i + 4 * q + r;
            u64 key = 0;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int n = nb + 16 * t + j;
                const float x = acc[t][i][r];
                const bool in = mi < B && n < V;
                if (in) C[(size_t)mi * (size_t)ldc + (size_t)n] = x;
                const u64 kt = in ? (((u64)gkey(x) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)n)) : 0ull;
                key = kt > key ? kt : key;
            }
#pragma unroll
            for (int s = 1; s < 16; s <<= 1) {   // the 16 lanes of this quarter hold the same row
                const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)key, s, 64);
                const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(key >> 32), s, 64);
                const u64 o = ((u64)hi << 32) | lo;
                key = o > key ? o : key;
            }
            if (j == 0) rowmax[w][mi] = key;
        }
    }
    __syncthreads();
    for (int mi = tid; mi < B && mi < MQ * 16; mi += LH_THREADS) {
        u64 key = rowmax[0][mi];
#pragma unroll
        for (int v = 1; v < 4; ++v) key = rowmax[v][mi] > key ? rowmax[v][mi] : key;
        const u64 cur = __hip_atomic_load(&best[mi], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (key > cur) atomicMax(&best[mi], key);
    }
}

__global__ void k_fill_u64(u64* p, int n)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0ull;
}

}  // namespace

hipError_t launch_lm_head(const float* H, int B, int D, long long ldh, const float* W, int V, long long ldw,
                          float* C, long long ldc, u64* best, hipStream_t s)
{
    hipLaunchKernelGGL(k_fill_u64, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, s, best, B);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const unsigned nx = (unsigned)((V + LH_NT - 1) / LH_NT);
    // up to 16 rows (and D a multiple of 64) the weight stream's kernel; above,
    // the LDS-tiled one with the fewest 32-row blocks that cover the batch
    constexpr int NV = 2, NP = 2, NT = 2;
    if (B <= 16 && D % (16 * NV * NP) == 0)
        hipLaunchKernelGGL((k_lmhead_narrow<1, NV, NP, NT>), dim3((unsigned)((V + 64 * NT - 1) / (64 * NT))),
                           dim3(LH_THREADS), 0, s, H, B, D, ldh, W, V, ldw, C, ldc, best);
    else if (B <= 32) hipLaunchKernelGGL(k_lmhead<1>, dim3(nx, 1), dim3(LH_THREADS), 0, s, H, B, D, ldh, W, V, ldw, C, ldc, best);
    else if (B <= 64) hipLaunchKernelGGL(k_lmhead<2>, dim3(nx, 1), dim3(LH_THREADS), 0, s, H, B, D, ldh, W, V, ldw, C, ldc, best);
    else if (B <= 128) hipLaunchKernelGGL(k_lmhead<4>, dim3(nx, 1), dim3(LH_THREADS), 0, s, H, B, D, ldh, W, V, ldw, C, ldc, best);
    else hipLaunchKernelGGL(k_lmhead<LH_MBMAX>, dim3(nx, (unsigned)((B + LH_MBMAX * 32 - 1) / (LH_MBMAX * 32))),
                            dim3(LH_THREADS), 0, s, H, B, D, ldh, W, V, ldw, C, ldc, best);
    return hipGetLastError();
}

}  // namespace mxs
