// mxs_sampler.hip -- gfx950 sampler chain behind the C ABI of include/mxs_sampler.h.
//
// Reference chain: mini_engine/sampling.py:30-69, one [vocab] row per call.
// Here one call samples a whole [B, V] batch with two launches:
//
// k_chunks  grid B x NC, workgroup (r, c) owns chunk c of row r (<= 16384
//           logits).  It streams the chunk from HBM once in 128-bit loads into
//           LDS (fp16 upcast to fp32 there), applies the repetition penalty in
//           place for the history ids inside the chunk (an LDS bitmap marks
//           each id once), then per row mode:
//             greedy  chunk argmax as a packed (key, ~index)
//             top-k   MSD radix select on order-preserving keys for the
//                     chunk's k-th largest, widened over the rounding of x / T,
//                     and the survivors written to the chunk's candidate slot
//             other   chunk maximum only
//           Results go to fixed per-(row, chunk) slots: no atomics, no
//           cross-workgroup waits, nothing to clear between calls.
// k_rows    grid B, one workgroup per row, after k_chunks (the kernel boundary
//           makes the slots visible).  Exact top-k over the candidates, bitonic
//           sort in LDS, integer softmax masses, exact top-p cut, inverse-CDF
//           draw.  Rows with top-k off or above KMAX (or whose candidates
//           overflow) are resolved by multi-pass histogram refinement over the
//           row in global memory.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stddef.h>
#include <stdint.h>

#include "mxs_device.h"
#include "mxs_sampler.h"

using namespace mxs;

namespace {

struct ChunkOut {          // one slot per (row, chunk), 16 bytes
    u64 best;              // greedy: max (key << 32 | ~index); sampling rows: max selection key << 32
    uint32_t count;        // candidates written to the chunk's slot
    uint32_t flags;
};
static_assert(sizeof(ChunkOut) == 16, "ChunkOut layout");

enum : uint32_t { FLAG_BAD_HISTORY = 1u, FLAG_OVERFLOW = 2u };
enum RowMode { MODE_GREEDY = 0, MODE_TOPK = 1, MODE_LARGE = 2, MODE_INVALID = 3 };

struct Params {
    const void* logits;
    int B, V;
    long long ld;
    int CS, NC;
    const float* T;
    const int32_t* K;
    const float* P;
    const float* PEN;
    const int32_t* hoff;
    const int32_t* hids;
    const float* U;
    int64_t* out_tok;
    int32_t* out_status;
    float* out_probs;
    ChunkOut* parts;       // [B * NC]
    uint32_t* cand_sk;     // [B * NC * CHUNK_CAP] selection keys
    uint32_t* cand_idx;    // [B * NC * CHUNK_CAP] token ids
};

struct Geometry {
    int NC, CS;
};

Geometry geometry(int B, int V)
{
    const int target_wgs = 2048;
    auto cdiv = [](long long a, long long b) { return (int)((a + b - 1) / b); };
    int nc_min = cdiv(V, CS_MAX);
    int nc_max = cdiv(V, CS_MIN);
    if (nc_max > NC_MAX) nc_max = NC_MAX;
    int want = cdiv(target_wgs, B > 0 ? B : 1);
    int NC = want < nc_max ? want : nc_max;
    if (NC < nc_min) NC = nc_min;
    if (NC < 1) NC = 1;
    int CS = cdiv(cdiv(V, NC), 8) * 8;
    NC = cdiv(V, CS);
    return Geometry{NC, CS};
}

__device__ __forceinline__ RowMode classify(float T, int k, int V)
{
    if (T == 0.0f) return MODE_GREEDY;
    if (T != T) return MODE_INVALID;
    if (k >= 1 && k <= KMAX && k < V) return MODE_TOPK;
    return MODE_LARGE;
}

template <typename TIn> struct VecIO;
template <> struct VecIO<float> {
    static constexpr int W = 4;
    typedef float4 vec_t;
    __device__ static void put(float* dst, const vec_t& v) { *(float4*)dst = v; }
    __device__ static float one(const float* p, int i) { return p[i]; }
};
template <> struct VecIO<__half> {
    static constexpr int W = 8;
    typedef uint4 vec_t;
    __device__ static float h2f(uint32_t bits16)
    {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
    }
    __device__ static void put(float* dst, const vec_t& v)
    {
        float4 a, b;
        a.x = h2f(v.x & 0xFFFFu); a.y = h2f(v.x >> 16);
        a.z = h2f(v.y & 0xFFFFu); a.w = h2f(v.y >> 16);
        b.x = h2f(v.z & 0xFFFFu); b.y = h2f(v.z >> 16);
        b.z = h2f(v.w & 0xFFFFu); b.w = h2f(v.w >> 16);
        *(float4*)dst = a;
        *(float4*)(dst + 4) = b;
    }
    __device__ static float one(const __half* p, int i)
    {
        return h2f(__builtin_bit_cast(uint16_t, p[i]));
    }
};

__device__ __forceinline__ float penalize(float v, float pen) { return v > 0.0f ? v / pen : v * pen; }

// The smallest selection key s whose tempered value fl32(x(s) / T) is
// >= fl32(x(th) / T).  Division by T is monotone, so the predicate is
// monotone in s; values a few ulps below x(th) can round onto the same
// tempered value and then tie with it.
__device__ uint32_t widen_threshold(uint32_t th, float T, bool neg)
{
    __shared__ uint32_t s_res;
    if (wave_id() == 0) {
        const int lane = lane_id();
        const float kth = sel_inv(th, neg) / T;
        auto pred = [&](uint32_t s) -> bool { return s >= SK_MIN && (sel_inv(s, neg) / T) >= kth; };
        bool ok = th >= (uint32_t)lane && pred(th - (uint32_t)lane);
        u64 mask = __ballot(ok);
        uint32_t res;
        if (~mask != 0ull) {
            int j = __builtin_ctzll(~mask);        // first failing lane; lanes 0..j-1 hold
            res = th - (uint32_t)(j - 1);
        } else {
            uint32_t lo = SK_MIN, hi = th - 63u;   // pred(hi) holds
            if (pred(lo)) {
                res = lo;
            } else {
                while (hi - lo > 1u) {
                    uint32_t mid = lo + (hi - lo) / 2u;
                    if (pred(mid)) hi = mid; else lo = mid;
                }
                res = hi;
            }
        }
        if (lane == 0) s_res = res;
    }
    __syncthreads();
    uint32_t r = s_res;
    __syncthreads();
    return r;
}

// ================================================================ k_chunks

template <typename TIn>
__global__ __launch_bounds__(NT, 2) void k_chunks(Params p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    float* xs = (float*)(smem + K1_XS);
    uint32_t* hist = (uint32_t*)(smem + K1_HIST);
    uint32_t* bm = (uint32_t*)(smem + K1_BM);
    __shared__ uint32_t s_wcnt;

    const int tid = threadIdx.x;
    const int r = blockIdx.x / p.NC;
    const int c = blockIdx.x - r * p.NC;
    const int V = p.V;
    const float T = p.T[r];
    const int k = p.K[r];
    const float pen = p.PEN[r];
    const RowMode mode = classify(T, k, V);
    const bool neg = T < 0.0f;
    const int e0 = c * p.CS;
    const int e1 = (e0 + p.CS < V) ? e0 + p.CS : V;
    const int n = e1 - e0;
    const TIn* rowp = (const TIn*)p.logits + (size_t)r * (size_t)p.ld;
    const int h0 = p.hoff ? p.hoff[r] : 0;
    const int h1 = p.hoff ? p.hoff[r + 1] : 0;
    const bool pen_on = (pen != 1.0f) && (h1 > h0);
    const size_t slot = (size_t)blockIdx.x;

    if (p.out_probs) {
        float* o = p.out_probs + (size_t)r * (size_t)V;
        for (int i = e0 + tid; i < e1; i += NT) o[i] = 0.0f;
    }

    // ---- stream the chunk into LDS; penalty bitmap from the history
    typedef VecIO<TIn> IO;
    constexpr int VW = IO::W;
    constexpr int MAXV = CS_MAX / (NT * VW);
    if (pen_on)
        for (int w = tid; w < CS_MAX / 32; w += NT) bm[w] = 0;
    __syncthreads();
    // 128-bit loads when the chunk start is 16-byte aligned (every chunk of a
    // row whose start is: CS is a multiple of 8 elements), scalar otherwise.
    const bool vec_ok = (((uintptr_t)(rowp + e0)) & 15u) == 0;
    const int nvec = vec_ok ? n / VW : 0;
    typename IO::vec_t regs[MAXV];
    const typename IO::vec_t* src = (const typename IO::vec_t*)(rowp + e0);
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        int v = tid + j * NT;
        regs[j] = typename IO::vec_t{};
        if (v < nvec) regs[j] = src[v];
    }
    uint32_t flags = 0;
    if (pen_on) {
        bool bad = false;
        for (int h = h0 + tid; h < h1; h += NT) {
            int id = p.hids[h];
            if (id < 0 || id >= V) { bad = true; continue; }
            if (id >= e0 && id < e1) {
                int o = id - e0;
                atomicOr(&bm[o >> 5], 1u << (o & 31));
            }
        }
        if (block_sum<uint32_t>(bad ? 1u : 0u)) flags |= FLAG_BAD_HISTORY;
    }
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        int v = tid + j * NT;
        if (v < nvec) IO::put(xs + v * VW, regs[j]);
    }
    for (int i = nvec * VW + tid; i < n; i += NT) xs[i] = IO::one(rowp, e0 + i);
    __syncthreads();
    if (pen_on) {   // sampling.py:38-45, each id once
        for (int w = tid; w < (n + 31) / 32; w += NT) {
            uint32_t bits = bm[w];
            while (bits) {
                int b = __builtin_ctz(bits);
                bits &= bits - 1u;
                int o = w * 32 + b;
                xs[o] = penalize(xs[o], pen);
            }
        }
        __syncthreads();
    }

    // ---- per-mode chunk work
    u64 best = 0;
    uint32_t count = 0;
    if (mode == MODE_GREEDY) {   // sampling.py:47-48
        u64 b = 0;
        for (int i = tid; i < n; i += NT) {
            float x = xs[i];
            uint32_t g = (x != x) ? 0xFFFFFFFFu : vkey(x);
            u64 v = ((u64)g << 32) | (u64)(0xFFFFFFFFu - (uint32_t)(e0 + i));
            b = v > b ? v : b;
        }
        best = block_max<u64>(b);
    } else if (mode == MODE_TOPK || mode == MODE_LARGE) {
        uint32_t mx = 0;
        for (int i = tid; i < n; i += NT) {
            uint32_t s = selkey(xs[i], neg);
            mx = s > mx ? s : mx;
        }
        best = (u64)block_max<uint32_t>(mx) << 32;

        if (mode == MODE_TOPK) {   // sampling.py:52-54, a superset of the chunk's share
            uint32_t theta = 0;
            if (n > k) {
                auto key = [&](int i) -> uint32_t { return selkey(xs[i], neg); };
                uint32_t th = block_select_desc(n, (uint32_t)k, key, hist, 32u);
                if (th < SK_MIN) th = SK_MIN;
                theta = widen_threshold(th, T, neg);
            }
            uint32_t mine = 0;
            for (int i = tid; i < n; i += NT) mine += selkey(xs[i], neg) >= theta ? 1u : 0u;
            const uint32_t total = block_sum<uint32_t>(mine);
            if (total > (uint32_t)CHUNK_CAP) {
                flags |= FLAG_OVERFLOW;
            } else {
                count = total;
                if (tid == 0) s_wcnt = 0;
                __syncthreads();
                uint32_t* dsk = p.cand_sk + slot * CHUNK_CAP;
                uint32_t* didx = p.cand_idx + slot * CHUNK_CAP;
                for (int i0 = 0; i0 < n; i0 += NT) {
                    int i = i0 + tid;
                    uint32_t s = 0;
                    bool keep = false;
                    if (i < n) {
                        s = selkey(xs[i], neg);
                        keep = s >= theta;
                    }
                    u64 mask = __ballot(keep);
                    if (mask) {
                        int first = __builtin_ctzll(mask);
                        uint32_t wb = 0;
                        if (lane_id() == first) wb = atomicAdd(&s_wcnt, (uint32_t)__builtin_popcountll(mask));
                        wb = __shfl(wb, first, 64);
                        if (keep) {
                            uint32_t o = wb + lanes_below(mask);
                            dsk[o] = s;
                            didx[o] = (uint32_t)(e0 + i);
                        }
                    }
                }
            }
        }
    }
    if (tid == 0) p.parts[slot] = ChunkOut{best, count, flags};
}

// ================================================================ k_rows

struct Found {
    uint32_t vk;
    uint32_t idx;
    u64 E;     // exclusive prefix mass in sorted order
    u64 w;     // the element's mass
};

// Multi-pass resolution of one row over its logits in global memory: used
// when top-k is off or above KMAX, and when candidates overflow (massive ties).
// Penalized values come from a full-row LDS bitmap of the history.
template <typename TIn>
struct LargeRow {
    const TIn* row;
    int V;
    float T;
    bool neg;
    float pen;
    bool pen_on;
    const uint32_t* rbm;   // V bits
    uint32_t thk;          // kept by top-k: selection key >= thk
    float m;               // max tempered logit
    u64* MH;               // 2048 masses (overlaps keys)
    uint32_t* CH;          // 2048 counts
    u64* keys;             // LCAP sort keys

    __device__ float x_at(int i) const
    {
        float x = VecIO<TIn>::one(row, i);
        if (pen_on && ((rbm[i >> 5] >> (i & 31)) & 1u)) x = penalize(x, pen);
        return x;
    }

    // Level lev histogram of masses and counts over kept elements whose value
    // key matches `prefix` on the digits above lev.  Returns the mass total.
    __device__ u64 mass_hist(int lev, uint32_t prefix)
    {
        const int sh = lev == 0 ? 21 : (lev == 1 ? 10 : 0);
        const int nb = lev == 2 ? 1024 : 2048;
        const int hsh = lev == 0 ? 32 : (lev == 1 ? 21 : 10);
        for (int b = threadIdx.x; b < 2048; b += NT) { MH[b] = 0; CH[b] = 0; }
        __syncthreads();
        u64 tot = 0;
        for (int i = threadIdx.x; i < V; i += NT) {
            float x = x_at(i);
            if (selkey(x, neg) < thk) continue;
            float l = x / T;
            uint32_t vk = vkey(l);
            if (lev > 0 && (vk >> hsh) != prefix) continue;
            u64 w = mass_of(l - m);
            uint32_t d = (vk >> sh) & (uint32_t)(nb - 1);
            atomicAdd(&MH[d], w);
            atomicAdd(&CH[d], 1u);
            tot += w;
        }
        return block_sum<u64>(tot);
    }

    // q-th smallest index (0-based) among the `count` kept elements whose value key is vk.
    __device__ uint32_t select_index(uint32_t vk, uint32_t q, uint32_t count)
    {
        uint32_t* H = CH;   // digits of the index: [17:9] then [8:0] (V <= 2^18)
        uint32_t hi_bin = 0;
        for (int lev = 0; lev < 2; ++lev) {
            for (int b = threadIdx.x; b < 512; b += NT) H[b] = 0;
            __syncthreads();
            for (int i = threadIdx.x; i < V; i += NT) {
                if (lev == 1 && ((uint32_t)i >> 9) != hi_bin) continue;
                float x = x_at(i);
                if (selkey(x, neg) < thk) continue;
                if (vkey(x / T) != vk) continue;
                atomicAdd(&H[lev == 0 ? ((uint32_t)i >> 9) : ((uint32_t)i & 511u)], 1u);
            }
            __syncthreads();
            // the q-th smallest is the (count - q)-th largest
            BinHit hit = find_desc<uint32_t>(H, 512, (u64)(count - 1u - q));
            uint32_t in_bin = H[hit.bin];
            uint32_t below = count - (uint32_t)hit.above - in_bin;
            __syncthreads();
            if (lev == 1) return (hi_bin << 9) | (uint32_t)hit.bin;
            hi_bin = (uint32_t)hit.bin;
            count = in_bin;
            q -= below;
        }
        return 0;
    }

    // The element at mass position t (t < total kept mass) of the sorted order
    // (value descending, index ascending).  If mh0_ready the level-0
    // histogram is already in MH/CH.
    __device__ Found find(u64 t, bool mh0_ready)
    {
        __shared__ Found s_found;
        __shared__ uint32_t s_cnt;
        u64 A_base = 0;
        uint32_t prefix = 0;
        for (int lev = 0; lev < 3; ++lev) {
            if (!(lev == 0 && mh0_ready)) mass_hist(lev, prefix);
            const int nb = lev == 2 ? 1024 : 2048;
            const int sh = lev == 0 ? 21 : (lev == 1 ? 10 : 0);
            const int width = lev == 2 ? 10 : 11;
            BinHit hit = find_desc<u64>(MH, nb, t - A_base);
            const u64 A_b = A_base + hit.above;
            const uint32_t cnt = CH[hit.bin];
            const u64 mass_b = MH[hit.bin];
            const uint32_t key_prefix = (prefix << width) | (uint32_t)hit.bin;
            __syncthreads();
            if (cnt <= (uint32_t)LCAP) {
                if (threadIdx.x == 0) s_cnt = 0;
                __syncthreads();
                for (int i = threadIdx.x; i < V; i += NT) {
                    float x = x_at(i);
                    if (selkey(x, neg) < thk) continue;
                    uint32_t vk = vkey(x / T);
                    if ((vk >> sh) != key_prefix) continue;
                    uint32_t o = atomicAdd(&s_cnt, 1u);
                    if (o < (uint32_t)LCAP) keys[o] = ((u64)vk << 32) | (u64)(0xFFFFFFFFu - (uint32_t)i);
                }
                __syncthreads();
                const int n = (int)cnt;
                const int P = pow2_ceil(n);
                for (int j = n + threadIdx.x; j < P; j += NT) keys[j] = 0;
                __syncthreads();
                bitonic_sort_desc(keys, P);
                constexpr int PER = LCAP / NT;
                const int j0 = threadIdx.x * PER;
                u64 wv[PER], run = 0;
#pragma unroll
                for (int q = 0; q < PER; ++q) {
                    int j = j0 + q;
                    u64 w = 0;
                    if (j < n) w = mass_of(okey_inv((uint32_t)(keys[j] >> 32)) - m);
                    wv[q] = w;
                    run += w;
                }
                u64 tot;
                u64 E = A_b + (block_incl_scan<u64>(run, &tot) - run);
#pragma unroll
                for (int q = 0; q < PER; ++q) {
                    int j = j0 + q;
                    if (j < n && E <= t && t < E + wv[q])
                        s_found = Found{(uint32_t)(keys[j] >> 32), 0xFFFFFFFFu - (uint32_t)keys[j], E, wv[q]};
                    E += wv[q];
                }
                __syncthreads();
                Found f = s_found;
                __syncthreads();
                return f;
            }
            if (lev < 2) {
                A_base = A_b;
                prefix = key_prefix;
                continue;
            }
            // one value shared by more than LCAP elements: equal masses, index order
            const u64 w = mass_b / cnt;
            const u64 q = (t - A_b) / w;
            uint32_t idx = select_index(key_prefix, (uint32_t)q, cnt);
            return Found{key_prefix, idx, A_b + q * w, w};
        }
        return Found{0, 0, 0, 0};
    }
};

template <typename TIn>
__device__ void finish_large(const Params& p, int r, float T, int k, float top_p, float pen,
                             bool pen_on, u64 best, float u, int64_t& tok, int32_t& st)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const int V = p.V;
    LargeRow<TIn> L;
    L.row = (const TIn*)p.logits + (size_t)r * (size_t)p.ld;
    L.V = V;
    L.T = T;
    L.neg = T < 0.0f;
    L.pen = pen;
    L.pen_on = pen_on;
    uint32_t* rbm = (uint32_t*)(smem + K2_A);
    L.rbm = rbm;
    L.MH = (u64*)(smem + K2_B);
    L.keys = (u64*)(smem + K2_B);
    L.CH = (uint32_t*)(smem + K2_HIST);

    if (pen_on) {
        const int words = (V + 31) >> 5;
        for (int w = threadIdx.x; w < words; w += NT) rbm[w] = 0;
        __syncthreads();
        for (int h = p.hoff[r] + threadIdx.x; h < p.hoff[r + 1]; h += NT) {
            int id = p.hids[h];     // range-checked by k_chunks
            atomicOr(&rbm[id >> 5], 1u << (id & 31));
        }
        __syncthreads();
    }

    const float m = sel_inv((uint32_t)(best >> 32), L.neg) / T;
    if (!isfinite(m)) { st = MXS_ROW_NONFINITE; tok = -1; return; }
    L.m = m;

    // sampling.py:52-54: exact k-th largest over the row
    L.thk = 0;
    if (k > 0 && k < V) {
        auto key = [&](int i) -> uint32_t { return selkey(L.x_at(i), L.neg); };
        uint32_t skk = block_select_desc(V, (uint32_t)k, key, L.CH, 0u);
        if (skk < SK_MIN) skk = SK_MIN;
        L.thk = widen_threshold(skk, T, L.neg);
    }

    // sampling.py:56-66 and 69
    const u64 W = L.mass_hist(0, 0);
    bool have_bound = false;
    uint32_t vk_b = 0, idx_b = 0;
    u64 Wk = W;
    bool mh0 = true;
    if (top_p < 1.0f) {
        if (!(top_p > 0.0f)) { st = MXS_ROW_EMPTY_NUCLEUS; tok = -1; return; }
        Found b = L.find(ceil_mul(top_p, W) - 1, true);
        have_bound = true;
        vk_b = b.vk;
        idx_b = b.idx;
        Wk = b.E + b.w;
        mh0 = false;
    }
    Found d = L.find(floor_mul(clamp_uniform(u), Wk), mh0);
    tok = (int64_t)d.idx;
    st = MXS_ROW_OK;

    // sampling.py:68
    if (p.out_probs) {
        float* out = p.out_probs + (size_t)r * (size_t)V;
        for (int i = threadIdx.x; i < V; i += NT) {
            float x = L.x_at(i);
            if (selkey(x, L.neg) < L.thk) continue;
            float l = x / T;
            uint32_t vk = vkey(l);
            if (have_bound && !(vk > vk_b || (vk == vk_b && (uint32_t)i <= idx_b))) continue;
            out[i] = (float)((double)mass_of(l - m) / (double)Wk);
        }
    }
}

// Top-k rows.  The chunks' candidates hold every element whose tempered
// value reaches the row's k-th largest.  Returns false when the survivors do
// not fit the LDS sort; the caller then takes the multi-pass path.
__device__ bool finish_topk(const Params& p, int r, float T, int k, float top_p, float u,
                            const uint32_t* counts, const uint32_t* off, int N,
                            int64_t& tok, int32_t& st)
{
    extern __shared__ __align__(16) unsigned char smem[];
    uint32_t* ck = (uint32_t*)(smem + K2_A);          // CAND_LDS candidate keys
    u64* keys = (u64*)(smem + K2_B);                  // SORT_CAP sort keys
    u64* cum = (u64*)(smem + K2_B + 8 * SORT_CAP);    // SORT_CAP prefix masses
    uint32_t* hist = (uint32_t*)(smem + K2_HIST);
    __shared__ uint32_t s_n;
    const int NC = p.NC, V = p.V;
    const bool neg = T < 0.0f;
    const uint32_t kk = (uint32_t)(k < V ? k : V);
    const size_t slot0 = (size_t)r * NC;
    const bool in_lds = N <= CAND_LDS;

    if (in_lds) {
        for (int c = 0; c < NC; ++c) {
            const uint32_t* src = p.cand_sk + (slot0 + c) * CHUNK_CAP;
            for (int j = threadIdx.x; j < (int)counts[c]; j += NT) ck[off[c] + j] = src[j];
        }
        __syncthreads();
    }
    auto visit = [&](auto&& f) {
        if (in_lds) {
            for (int i = threadIdx.x; i < N; i += NT) f(ck[i]);
        } else {
            for (int c = 0; c < NC; ++c) {
                const uint32_t* src = p.cand_sk + (slot0 + c) * CHUNK_CAP;
                for (int j = threadIdx.x; j < (int)counts[c]; j += NT) f(src[j]);
            }
        }
    };

    // sampling.py:52-54: the k-th largest, then everything that rounds onto it
    uint32_t sk_k = block_select_desc_v(kk, visit, hist, 0u);
    if (sk_k < SK_MIN) sk_k = SK_MIN;
    const uint32_t theta = widen_threshold(sk_k, T, neg);
    uint32_t mine = 0;
    visit([&](uint32_t s) { mine += s >= theta ? 1u : 0u; });
    const int n1 = (int)block_sum<uint32_t>(mine);
    if (n1 > SORT_CAP) return false;

    if (threadIdx.x == 0) s_n = 0;
    __syncthreads();
    for (int c = 0; c < NC; ++c) {
        const int cnt = (int)counts[c];
        const uint32_t* gsk = p.cand_sk + (slot0 + c) * CHUNK_CAP;
        const uint32_t* gidx = p.cand_idx + (slot0 + c) * CHUNK_CAP;
        for (int j0 = 0; j0 < cnt; j0 += NT) {
            const int j = j0 + threadIdx.x;
            uint32_t s = 0;
            bool keep = false;
            if (j < cnt) {
                s = in_lds ? ck[off[c] + j] : gsk[j];
                keep = s >= theta;
            }
            u64 mask = __ballot(keep);
            if (mask) {
                int first = __builtin_ctzll(mask);
                uint32_t base = 0;
                if (lane_id() == first) base = atomicAdd(&s_n, (uint32_t)__builtin_popcountll(mask));
                base = __shfl(base, first, 64);
                if (keep) {
                    const uint32_t idx = gidx[j];
                    const uint32_t vk = vkey(sel_inv(s, neg) / T);
                    keys[base + lanes_below(mask)] = ((u64)vk << 32) | (u64)(0xFFFFFFFFu - idx);
                }
            }
        }
    }
    __syncthreads();
    const int P = pow2_ceil(n1);
    for (int j = n1 + threadIdx.x; j < P; j += NT) keys[j] = 0;
    __syncthreads();
    bitonic_sort_desc(keys, P);

    // sampling.py:57-59: masses in sorted order and their inclusive prefix sums
    const float m = okey_inv((uint32_t)(keys[0] >> 32));
    if (!isfinite(m)) { st = MXS_ROW_NONFINITE; tok = -1; return true; }
    constexpr int PER = SORT_CAP / NT;
    const int j0 = threadIdx.x * PER;
    u64 wv[PER], run = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        int j = j0 + q;
        u64 w = 0;
        if (j < n1) w = mass_of(okey_inv((uint32_t)(keys[j] >> 32)) - m);
        wv[q] = w;
        run += w;
    }
    u64 W;
    u64 acc = block_incl_scan<u64>(run, &W) - run;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        acc += wv[q];
        cum[j0 + q] = acc;
    }
    __syncthreads();

    // sampling.py:56, 62-63: keep j while the mass before it is < top_p * W
    int nstar = n1;
    if (top_p < 1.0f) {
        if (!(top_p > 0.0f)) { st = MXS_ROW_EMPTY_NUCLEUS; tok = -1; return true; }
        const u64 Tm = ceil_mul(top_p, W);
        uint32_t cnt = 0;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            int j = j0 + q;
            if (j < n1 && cum[j] - wv[q] < Tm) ++cnt;
        }
        nstar = (int)block_sum<uint32_t>(cnt);
    }
    const u64 Wk = cum[nstar - 1];

    // sampling.py:69: the first j with C_j > floor(u * Wk)
    const u64 D = floor_mul(clamp_uniform(u), Wk);
    uint32_t below = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        int j = j0 + q;
        if (j < nstar && cum[j] <= D) ++below;
    }
    const int jd = (int)block_sum<uint32_t>(below);
    tok = (int64_t)(0xFFFFFFFFu - (uint32_t)keys[jd]);
    st = MXS_ROW_OK;

    // sampling.py:68
    if (p.out_probs) {
        float* out = p.out_probs + (size_t)r * (size_t)V;
        for (int j = threadIdx.x; j < nstar; j += NT) {
            u64 w = cum[j] - (j ? cum[j - 1] : 0ull);
            out[0xFFFFFFFFu - (uint32_t)keys[j]] = (float)((double)w / (double)Wk);
        }
    }
    return true;
}

template <typename TIn>
__global__ __launch_bounds__(NT, 1) void k_rows(Params p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    uint32_t* off = (uint32_t*)(smem + K2_OFF);
    __shared__ uint32_t s_counts[NC_MAX];
    const int tid = threadIdx.x;
    const int r = blockIdx.x;
    const int NC = p.NC, V = p.V;
    const float T = p.T[r];
    const int k = p.K[r];
    const float pen = p.PEN[r];
    const RowMode mode = classify(T, k, V);
    const int h0 = p.hoff ? p.hoff[r] : 0;
    const int h1 = p.hoff ? p.hoff[r + 1] : 0;
    const bool pen_on = (pen != 1.0f) && (h1 > h0);

    u64 best = 0;
    uint32_t fl = 0;
    for (int c = tid; c < NC; c += NT) {
        ChunkOut o = p.parts[(size_t)r * NC + c];
        best = o.best > best ? o.best : best;
        fl |= o.flags;
        s_counts[c] = o.count;
    }
    best = block_max<u64>(best);
    const uint32_t flags = block_max<uint32_t>(fl & FLAG_BAD_HISTORY) |
                           block_max<uint32_t>(fl & FLAG_OVERFLOW);
    if (tid == 0) {
        uint32_t a = 0;
        for (int c = 0; c < NC; ++c) { off[c] = a; a += s_counts[c]; }
        off[NC] = a;
    }
    __syncthreads();
    const int N = (int)off[NC];
    const float top_p = p.P[r];
    const float u = p.U ? p.U[r] : 0.0f;
    int64_t tok = -1;
    int32_t st = MXS_ROW_OK;

    if (flags & FLAG_BAD_HISTORY) {
        st = MXS_ROW_BAD_HISTORY;
    } else if (mode == MODE_INVALID) {
        st = MXS_ROW_BAD_PARAM;
    } else if (mode == MODE_GREEDY) {
        tok = (int64_t)(0xFFFFFFFFu - (uint32_t)best);
        if (p.out_probs && tid == 0) p.out_probs[(size_t)r * (size_t)V + (size_t)tok] = 1.0f;
    } else {
        bool done = false;
        if (mode == MODE_TOPK && !(flags & FLAG_OVERFLOW))
            done = finish_topk(p, r, T, k, top_p, u, s_counts, off, N, tok, st);
        if (!done) {
            __syncthreads();
            finish_large<TIn>(p, r, T, k, top_p, pen, pen_on, best, u, tok, st);
        }
    }
    if (tid == 0) {
        p.out_tok[r] = st == MXS_ROW_OK ? tok : -1;
        if (p.out_status) p.out_status[r] = st;
    }
}

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Layout {
    size_t parts, cand_sk, cand_idx, total;
};

Layout layout(int B, int V)
{
    Geometry g = geometry(B, V);
    const size_t slots = (size_t)B * (size_t)g.NC;
    Layout L;
    L.parts = 0;
    L.cand_sk = align256(slots * sizeof(ChunkOut));
    L.cand_idx = L.cand_sk + align256(slots * CHUNK_CAP * sizeof(uint32_t));
    L.total = L.cand_idx + align256(slots * CHUNK_CAP * sizeof(uint32_t));
    return L;
}

template <typename TIn>
hipError_t launch(const Params& p, hipStream_t s)
{
    static const hipError_t a1 = hipFuncSetAttribute((const void*)k_chunks<TIn>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, K1_LDS_BYTES);
    static const hipError_t a2 = hipFuncSetAttribute((const void*)k_rows<TIn>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, K2_LDS_BYTES);
    (void)a1;
    (void)a2;
    hipLaunchKernelGGL(k_chunks<TIn>, dim3((unsigned)((long long)p.B * p.NC)), dim3(NT), K1_LDS_BYTES, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_rows<TIn>, dim3((unsigned)p.B), dim3(NT), K2_LDS_BYTES, s, p);
    return hipGetLastError();
}

}  // namespace

extern "C" {

const char* mxs_version(void) { return "mxs-sampler 0.2.0 gfx950"; }

const char* mxs_status_string(int status)
{
    switch (status) {
    case MXS_OK: return "ok";
    case MXS_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MXS_ERR_ALIGNMENT: return "logits not element-aligned or workspace not 256-byte aligned";
    case MXS_ERR_WORKSPACE_TOO_SMALL: return "workspace too small";
    case MXS_ERR_VOCAB_TOO_LARGE: return "vocabulary larger than MXS_MAX_VOCAB";
    case MXS_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
    }
}

size_t mxs_workspace_bytes(int B, int V)
{
    if (B <= 0 || V <= 0 || V > MXS_MAX_VOCAB) return 0;
    return layout(B, V).total;
}

int mxs_sample(const void* logits, int dtype, int B, int V, int64_t ld,
               const float* temperature, const int32_t* top_k,
               const float* top_p, const float* penalty,
               const int32_t* hist_offsets, const int32_t* hist_ids,
               const float* uniforms,
               int64_t* out_tokens, int32_t* out_status, float* out_probs,
               void* workspace, size_t workspace_bytes, mxs_stream_t stream)
{
    if (B < 0 || V <= 0) return MXS_ERR_INVALID_ARGUMENT;
    if (V > MXS_MAX_VOCAB) return MXS_ERR_VOCAB_TOO_LARGE;
    if (dtype != MXS_DTYPE_F32 && dtype != MXS_DTYPE_F16) return MXS_ERR_INVALID_ARGUMENT;
    if (B == 0) return MXS_OK;
    if (!logits || !temperature || !top_k || !top_p || !penalty || !out_tokens || !workspace)
        return MXS_ERR_INVALID_ARGUMENT;
    if (hist_offsets && !hist_ids) return MXS_ERR_INVALID_ARGUMENT;
    if (ld < V) return MXS_ERR_INVALID_ARGUMENT;
    const uintptr_t esize = dtype == MXS_DTYPE_F32 ? 4u : 2u;
    if (((uintptr_t)logits & (esize - 1u)) || ((uintptr_t)workspace & 255u)) return MXS_ERR_ALIGNMENT;
    const Layout L = layout(B, V);
    if (workspace_bytes < L.total) return MXS_ERR_WORKSPACE_TOO_SMALL;

    const Geometry g = geometry(B, V);
    Params p;
    p.logits = logits;
    p.B = B;
    p.V = V;
    p.ld = ld;
    p.CS = g.CS;
    p.NC = g.NC;
    p.T = temperature;
    p.K = top_k;
    p.P = top_p;
    p.PEN = penalty;
    p.hoff = hist_offsets;
    p.hids = hist_ids;
    p.U = uniforms;
    p.out_tok = out_tokens;
    p.out_status = out_status;
    p.out_probs = out_probs;
    char* ws = (char*)workspace;
    p.parts = (ChunkOut*)(ws + L.parts);
    p.cand_sk = (uint32_t*)(ws + L.cand_sk);
    p.cand_idx = (uint32_t*)(ws + L.cand_idx);

    hipStream_t s = (hipStream_t)stream;
    hipError_t e = dtype == MXS_DTYPE_F32 ? launch<float>(p, s) : launch<__half>(p, s);
    return e == hipSuccess ? MXS_OK : MXS_ERR_HIP;
}

}  // extern "C"
