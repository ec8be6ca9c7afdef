// sampler_kernels.h -- the gfx950 sampler chain's device code.
//
// Reference chain: mini_engine/sampling.py:30-69, one [vocab] row per call.
// Here one call samples a whole [B, V] batch with one launch of k_fused: one
// workgroup per row (152 KB of dynamic LDS, so one row per CU), which streams
// the row from HBM once and finishes it on chip:
//   greedy     a packed (key, index) maximum;
//   top-k      candidates above a sampled, then verified, lower bound on the
//              k-th largest key, kept in LDS; exact k-th, top-p cut and draw
//              from a counting sort of the candidates by mass bins;
//   top-k off  a mass pass over the row, then the cut's and the draw's bins
//              gathered and ranked;
// with general paths (compaction and exact select, finish_large) for what
// the fast ones decline: failed bounds, full buffers, heavy ties.
//
// Included by the k_*.hip files, each of which instantiates one kernel set;
// everything here has internal linkage.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "mxs_device.h"
#include "mxs_sampler.h"
#include "sampler_params.h"

namespace mxs {
namespace {

enum RowMode { MODE_GREEDY = 0, MODE_TOPK = 1, MODE_LARGE = 2, MODE_INVALID = 3 };


__device__ __forceinline__ RowMode classify(float T, int k, int V)
{
    if (T == 0.0f) return MODE_GREEDY;
    if (T != T) return MODE_INVALID;
    if (k >= 1 && k <= KMAX && k < V) return MODE_TOPK;
    return MODE_LARGE;
}

// Row r's history range [h0, h1) in p.hids from its two raw words (CSR
// offsets hoff[r], hoff[r + 1], or a range hbegin[r], hend[r]).  The ids are
// read only when the penalty applies (pen != 1, sampling.py:38); then a
// range outside [0, nhids), or CSR offsets that decrease, make the row an
// error (bad = true) and its history empty, so nothing outside hids is read.
__device__ __forceinline__ void history_range(const Params& p, int w0, int w1, float pen, int& h0, int& h1, bool& bad)
{
    h0 = 0;
    h1 = 0;
    bad = false;
    if (!p.hoff || pen == 1.0f) return;
    const bool ranged = p.hend != nullptr;
    if (ranged && w1 <= w0) return;   // an empty range
    if (w0 < 0 || (long long)w1 > p.nhids || w1 < w0) { bad = true; return; }
    h0 = w0;
    h1 = w1;
}

// 16-byte vectors of a row (clang vector types, which load from any
// address space) and the conversion of their elements to float.
template <typename TIn> struct VecIO;
template <> struct VecIO<float> {
    static constexpr int W = 4;
    typedef float vec_t __attribute__((ext_vector_type(4)));
    __device__ static void unpack(const vec_t& v, float* d) { d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w; }
    __device__ static float one(const float* p, int i) { return p[i]; }
};
template <> struct VecIO<__half> {
    static constexpr int W = 8;
    typedef uint32_t vec_t __attribute__((ext_vector_type(4)));
    __device__ static float h2f(uint32_t bits16)
    {
        return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
    }
    __device__ static void unpack(const vec_t& v, float* d)
    {
        d[0] = h2f(v.x & 0xFFFFu); d[1] = h2f(v.x >> 16);
        d[2] = h2f(v.y & 0xFFFFu); d[3] = h2f(v.y >> 16);
        d[4] = h2f(v.z & 0xFFFFu); d[5] = h2f(v.z >> 16);
        d[6] = h2f(v.w & 0xFFFFu); d[7] = h2f(v.w >> 16);
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
__device__ __forceinline__ uint32_t widen_threshold(uint32_t th, float T, bool neg)
{
    // every wave computes it (the same result), so no barrier is needed
    const int lane = lane_id();
    const float kth = sel_inv(th, neg) / T;
    auto pred = [&](uint32_t s) -> bool { return s >= SK_MIN && (sel_inv(s, neg) / T) >= kth; };
    const bool ok = th >= (uint32_t)lane && pred(th - (uint32_t)lane);
    const u64 mask = __ballot(ok);
    if (~mask != 0ull) {
        const int j = __builtin_ctzll(~mask);        // first failing lane; lanes 0..j-1 hold
        return th - (uint32_t)(j - 1);
    }
    uint32_t lo = SK_MIN, hi = th - 63u;   // pred(hi) holds
    if (pred(lo)) return lo;
    while (hi - lo > 1u) {
        const uint32_t mid = lo + (hi - lo) / 2u;
        if (pred(mid)) hi = mid; else lo = mid;
    }
    return hi;
}

struct Reduced {
    uint32_t max, min, any;
};

// One barrier round: max of a, min of b, OR of c over the workgroup.
__device__ __forceinline__ Reduced block_reduce(uint32_t a, uint32_t b, uint32_t c)
{
    __shared__ uint32_t s[3][NWAVES];
    a = wave_max_u32(a);
    b = wave_min_u32(b);
    c = wave_or_u32(c);
    __syncthreads();
    if (lane_id() == 0) { s[0][wave_id()] = a; s[1][wave_id()] = b; s[2][wave_id()] = c; }
    __syncthreads();
    Reduced r{s[0][0], s[1][0], s[2][0]};
#pragma unroll
    for (int i = 1; i < NWAVES; ++i) {
        r.max = s[0][i] > r.max ? s[0][i] : r.max;
        r.min = s[1][i] < r.min ? s[1][i] : r.min;
        r.any |= s[2][i];
    }
    return r;
}

// ================================================================ finishing a row

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

// LDS regions the multi-pass path works in.
struct LargeLds {
    uint32_t* rbm;   // V bits: history bitmap of the row
    u64* MH;         // 2048 masses
    u64* keys;       // LCAP sort keys (may overlap MH)
    uint32_t* CH;    // 2048 counts
};

// lds.rbm holds the row's history bitmap when pen_on.
// skmax: the row's largest selection key, over penalized values when
// max_penalized (else over raw values, and it is taken again here).
// thk_known: the top-k threshold thk is already exact (else it is selected).
template <typename TIn>
__device__ __forceinline__ void finish_large(const Params& p, int r, float T, int k, float top_p, float pen,
                             bool pen_on, uint32_t skmax, bool max_penalized,
                             bool thk_known, uint32_t thk, float u, const LargeLds& lds,
                             int64_t& tok, int32_t& st)
{
    const int V = p.V;
    LargeRow<TIn> L;
    L.row = (const TIn*)p.logits + (size_t)r * (size_t)p.ld;
    L.V = V;
    L.T = T;
    L.neg = T < 0.0f;
    L.pen = pen;
    L.pen_on = pen_on;
    uint32_t* rbm = lds.rbm;
    L.rbm = rbm;
    L.MH = lds.MH;
    L.keys = lds.keys;
    L.CH = lds.CH;

    if (pen_on && !max_penalized) {
        uint32_t mx = 0;
        for (int i = threadIdx.x; i < V; i += NT) {
            const uint32_t sk = selkey(L.x_at(i), L.neg);
            mx = sk > mx ? sk : mx;
        }
        skmax = block_max<uint32_t>(mx);
    }
    const float m = sel_inv(skmax, L.neg) / T;
    if (!isfinite(m)) { st = MXS_ROW_NONFINITE; tok = -1; return; }
    L.m = m;

    // sampling.py:52-54: exact k-th largest over the row
    L.thk = thk_known ? thk : 0;
    if (!thk_known && k > 0 && k < V) {
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

// The value a selection key stands for, ordered like the key: x, or -x
// when T < 0.
__device__ __forceinline__ float sel_val(uint32_t s, bool neg)
{
    const float x = sel_inv(s, neg);
    return neg ? -x : x;
}

// The r-th largest (0-based) of the cnt <= 64 keys for which in_bin holds.
template <class Visit, class InBin>
__device__ __forceinline__ uint32_t rank_in_bin(Visit visit, InBin in_bin, uint32_t cnt, uint32_t r)
{
    __shared__ uint32_t g_keys[64];
    __shared__ uint32_t g_n, g_res;
    if (threadIdx.x == 0) { g_n = 0; g_res = 0; }
    __syncthreads();
    visit([&](uint32_t k) {
        if (in_bin(k)) {
            const uint32_t slot = atomicAdd(&g_n, 1u);
            if (slot < 64u) g_keys[slot] = k;
        }
    });
    __syncthreads();
    if (wave_id() == 0) {
        const uint32_t lane = (uint32_t)lane_id();
        const uint32_t n = g_n < cnt ? g_n : cnt;
        const uint32_t mine = lane < n ? g_keys[lane] : 0u;
        uint32_t gt = 0, ge = 0;
        for (uint32_t t = 0; t < n; ++t) {   // broadcast reads of the gathered keys
            const uint32_t other = g_keys[t];
            gt += other > mine ? 1u : 0u;
            ge += other >= mine ? 1u : 0u;
        }
        const u64 mask = __ballot(lane < n && gt <= r && r < ge);
        if (mask && lane == (uint32_t)__builtin_ctzll(mask)) g_res = mine;
    }
    __syncthreads();
    const uint32_t res = g_res;
    __syncthreads();
    return res;
}

// Exact kk-th largest (1-based) selection key.  Each level histograms the
// keys of the current range into 2048 bins that are linear in the value the
// keys stand for (key-space bins when the range is not finite); the bin
// holding the answer is a contiguous key range because the bin function is
// monotone.  A bin of at most 64 keys is finished by ranking, otherwise it
// becomes the next range; lo and hi fall into different bins, so every level
// narrows the range.
// Keys outside [lo, hi] are ignored; at least kk keys must lie inside.
template <class Visit>
__device__ __forceinline__ uint32_t select_exact_in(uint32_t kk, Visit visit, uint32_t* hist, bool neg,
                                                    uint32_t lo, uint32_t hi)
{
    for (int lev = 0; lev < 64 && lo != hi; ++lev) {
        const float ylo = sel_val(lo, neg), yhi = sel_val(hi, neg);
        const float scale = 2047.0f / (yhi - ylo);
        const bool lin = __builtin_isfinite(ylo) && __builtin_isfinite(yhi) && yhi > ylo && scale > 0.0f &&
                         __builtin_isfinite(scale);
        const uint32_t span = hi - lo;
        const int sh = span >= 2048u ? (32 - __builtin_clz(span)) - 11 : 0;
        auto bin_of = [&](uint32_t k) -> uint32_t {
            if (lin) {
                const float f = (sel_val(k, neg) - ylo) * scale;
                return f < 2047.0f ? (uint32_t)f : 2047u;
            }
            return (k - lo) >> sh;
        };
        for (int b = threadIdx.x; b < 2048; b += NT) hist[b] = 0;
        __syncthreads();
        visit([&](uint32_t k) {
            if (k >= lo && k <= hi) atomicAdd(&hist[bin_of(k)], 1u);
        });
        __syncthreads();
        const BinHit hit = find_desc<uint32_t>(hist, 2048, (u64)(kk - 1u));
        const uint32_t cnt = hist[hit.bin];
        kk -= (uint32_t)hit.above;
        __syncthreads();
        if (!lin && sh == 0) return lo + (uint32_t)hit.bin;
        if (cnt <= 64u) {
            const uint32_t b = (uint32_t)hit.bin;
            return rank_in_bin(visit, [&](uint32_t k) { return k >= lo && k <= hi && bin_of(k) == b; },
                               cnt, kk - 1u);
        }
        uint32_t bmx = 0, bmn = 0xFFFFFFFFu;
        visit([&](uint32_t k) {
            if (k >= lo && k <= hi && bin_of(k) == (uint32_t)hit.bin) {
                bmx = k > bmx ? k : bmx;
                bmn = k < bmn ? k : bmn;
            }
        });
        const Reduced br = block_reduce(bmx, bmn, 0u);
        lo = br.min;
        hi = br.max;
    }
    return lo;
}


// Fallback of finish_kept for heavy ties: bitonic sort of the kept set, then
// the prefix sums in sorted order.
__device__ __forceinline__ bool finish_sorted(const Params& p, int r, u64* keys, u64* cum, int n1, float top_p, float u,
                              int64_t& tok, int32_t& st)
{
    __syncthreads();
    const int P = pow2_ceil(n1);
    for (int j = n1 + threadIdx.x; j < P; j += NT) keys[j] = 0;
    __syncthreads();
    bitonic_sort_desc(keys, P);
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
    if (p.out_probs) {
        float* out = p.out_probs + (size_t)r * (size_t)p.V;
        for (int j = threadIdx.x; j < nstar; j += NT) {
            u64 w = cum[j] - (j ? cum[j - 1] : 0ull);
            out[0xFFFFFFFFu - (uint32_t)keys[j]] = (float)((double)w / (double)Wk);
        }
    }
    return true;
}

struct Picked {
    u64 key;   // (value key << 32) | ~index
    u64 E;     // mass before it in sorted order
    u64 w;     // its mass
    int ok;    // 0: the bin held more than 64 elements
};

// Kept-by-top-k tokens in LDS (keys[0..n) as (value key << 32 | ~index), any
// order) -> top-p cut, draw and post-filter probabilities (sampling.py:56-69).
// Masses go into a histogram over value bins; the bin holding a given mass
// position is finished by ranking its elements in one wave.  A bin of more
// than 64 elements (heavy ties) falls back to a bitonic sort of the set.
__device__ __forceinline__ bool finish_kept(const Params& p, int r, u64* keys, u64* wm, int n, float top_p, float u,
                            u64* MH, uint32_t* CH, int64_t& tok, int32_t& st)
{
    __shared__ u64 g_key[64], g_w[64];
    __shared__ uint32_t g_n;
    __shared__ Picked g_pick;

    uint32_t vmax = 0, vmin = 0xFFFFFFFFu;
    for (int j = threadIdx.x; j < n; j += NT) {
        const uint32_t vk = (uint32_t)(keys[j] >> 32);
        vmax = vk > vmax ? vk : vmax;
        vmin = vk < vmin ? vk : vmin;
    }
    const Reduced rd = block_reduce(vmax, vmin, 0u);
    const float m = okey_inv(rd.max);
    if (!isfinite(m)) { st = MXS_ROW_NONFINITE; tok = -1; return true; }
    // Bins linear in d = l - m over [dmin, 0] (d = -inf in bin 0): monotone
    // in the sorted order, and spread evenly where float keys are not.
    float dmin = okey_inv(rd.min) - m;
    if (!(dmin > -INFINITY)) {   // -inf logits are kept: the smallest finite d
        uint32_t fmn = 0xFFFFFFFFu;
        for (int j = threadIdx.x; j < n; j += NT) {
            const uint32_t vk = (uint32_t)(keys[j] >> 32);
            if (vk > SK_MIN) fmn = vk < fmn ? vk : fmn;
        }
        const uint32_t f = block_reduce(0u, fmn, 0u).min;
        dmin = f == 0xFFFFFFFFu ? 0.0f : okey_inv(f) - m;
    }
    float scale = dmin < 0.0f ? 2047.0f / -dmin : 0.0f;
    if (!__builtin_isfinite(scale)) scale = 0.0f;
    auto bin_of = [&](uint32_t vk) -> uint32_t {
        const float d = okey_inv(vk) - m;
        if (!(d > -INFINITY)) return 0u;
        const float f = (d - dmin) * scale;
        return f < 2047.0f ? (uint32_t)f : 2047u;
    };
    for (int b = threadIdx.x; b < 2048; b += NT) { MH[b] = 0; CH[b] = 0; }
    __syncthreads();
    u64 part = 0;
    for (int j = threadIdx.x; j < n; j += NT) {
        const uint32_t vk = (uint32_t)(keys[j] >> 32);
        const u64 w = mass_of(okey_inv(vk) - m);
        wm[j] = w;
        part += w;
        const uint32_t bin = bin_of(vk);
        atomicAdd(&MH[bin], w);
        atomicAdd(&CH[bin], 1u);
    }
    const u64 W = block_sum<u64>(part);

    // the element at mass position t of the sorted order (value desc, index asc)
    auto pick = [&](u64 t) -> Picked {
        const BinHit hit = find_desc<u64>(MH, 2048, t);
        const uint32_t cnt = CH[hit.bin];
        if (threadIdx.x == 0) { g_n = 0; g_pick = Picked{0, 0, 0, cnt <= 64u ? 1 : 0}; }
        __syncthreads();
        if (cnt <= 64u) {
            for (int j = threadIdx.x; j < n; j += NT) {
                if (bin_of((uint32_t)(keys[j] >> 32)) == (uint32_t)hit.bin) {
                    const uint32_t slot = atomicAdd(&g_n, 1u);
                    if (slot < 64u) { g_key[slot] = keys[j]; g_w[slot] = wm[j]; }
                }
            }
            __syncthreads();
            if (wave_id() == 0) {
                const uint32_t lane = (uint32_t)lane_id();
                const uint32_t c = g_n < 64u ? g_n : 64u;
                const u64 mk = lane < c ? g_key[lane] : 0ull;
                const u64 mw = lane < c ? g_w[lane] : 0ull;
                u64 before = 0;
                for (uint32_t q = 0; q < c; ++q)   // broadcast reads of the gathered bin
                    before += g_key[q] > mk ? g_w[q] : 0ull;
                const u64 E = hit.above + before;
                if (lane < c && E <= t && t < E + mw) g_pick = Picked{mk, E, mw, 1};
            }
        }
        __syncthreads();
        const Picked res = g_pick;
        __syncthreads();
        return res;
    };

    bool bounded = false;
    u64 bound = 0, Wk = W;
    if (top_p < 1.0f) {   // sampling.py:56-63
        if (!(top_p > 0.0f)) { st = MXS_ROW_EMPTY_NUCLEUS; tok = -1; return true; }
        const Picked b = pick(ceil_mul(top_p, W) - 1);
        if (!b.ok) return finish_sorted(p, r, keys, wm, n, top_p, u, tok, st);
        bounded = true;
        bound = b.key;
        Wk = b.E + b.w;
    }
    const Picked d = pick(floor_mul(clamp_uniform(u), Wk));   // sampling.py:69
    if (!d.ok) return finish_sorted(p, r, keys, wm, n, top_p, u, tok, st);
    tok = (int64_t)(0xFFFFFFFFu - (uint32_t)d.key);
    st = MXS_ROW_OK;

    if (p.out_probs) {   // sampling.py:68
        float* out = p.out_probs + (size_t)r * (size_t)p.V;
        for (int j = threadIdx.x; j < n; j += NT)
            if (!bounded || keys[j] >= bound)
                out[0xFFFFFFFFu - (uint32_t)keys[j]] = (float)((double)wm[j] / (double)Wk);
    }
    return true;
}

// ---------------------------------------------------------------- top-k from the stream's segments
//
// The common top-k case, finished from the stream's per-wave buffer segments
// as they are (no compaction).  The buffer holds every element whose
// tempered value l reaches l_est = l(est), and the k-th largest l is at least
// l_est.  One pass histograms the counts and masses of those elements over
// 2048 bins linear in d = l - m on [l_est - m, 0] (monotone in the sorted
// order).  Then one wave finds the bin of the k-th largest, of the top-p cut
// and of the draw; each of these is resolved by gathering that bin's elements
// (at most 64) and ranking them within the wave.  The other waves only help
// to gather.

__device__ __forceinline__ u64 readlane64(u64 v, int l)
{
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((u64)hi << 32) | lo;
}

// Inclusive sums over the wave's lanes: from lane 0 up (prefix), from lane 63
// down (suffix); the wave's total.
__device__ __forceinline__ u64 wave_prefix_incl(u64 v) { return wave_prefix_u64(v); }
__device__ __forceinline__ u64 wave_sum64(u64 v) { return readlane64(wave_prefix_u64(v), 63); }
__device__ __forceinline__ u64 wave_suffix_incl(u64 v)
{
    const u64 pre = wave_prefix_u64(v);
    return readlane64(pre, 63) - pre + v;
}

struct WHit {
    int bin;
    u64 above;   // sum of the bins above `bin`
};

// Called by one whole wave, lane L holding s = the sum of h[32L, 32L + 32):
// the bin b of h[0, 2048) with above(b) <= t < above(b) + h[b], where
// above(b) is the sum of the bins above b.  Requires t < the total.
template <typename T>
__device__ __forceinline__ WHit wave_find_desc(const T* h, u64 s, u64 t);

// The same, with incl = wave_suffix_incl(s) computed once by the caller.
template <typename T>
__device__ __forceinline__ WHit wave_find_desc_pre(const T* h, u64 s, u64 incl, u64 t)
{
    const int lane = lane_id();
    const u64 msk = __ballot(incl - s <= t && t < incl);
    const int L = msk ? __builtin_ctzll(msk) : 0;
    const u64 a = readlane64(incl - s, L);
    // lane L's 32 bins, highest first, one per lane
    const u64 v = lane < 32 ? (u64)h[32 * L + 31 - lane] : 0ull;
    const u64 pi = wave_prefix_incl(v);
    const u64 m2 = __ballot(lane < 32 && a + pi - v <= t && t < a + pi);
    const int j = m2 ? __builtin_ctzll(m2) : 0;
    return WHit{32 * L + 31 - j, a + readlane64(pi - v, j)};
}
template <typename T>
__device__ __forceinline__ WHit wave_find_desc(const T* h, u64 s, u64 t)
{
    return wave_find_desc_pre<T>(h, s, wave_suffix_incl(s), t);
}

// Called by one whole wave: the sum of h over the bins above b.
template <typename T>
__device__ __forceinline__ u64 wave_sum_above(const T* h, u64 s, int b)
{
    const int lane = lane_id();
    const int L = b >> 5, i = b & 31;
    u64 v = lane > L ? s : 0ull;
    if (lane < 32 && lane > i) v += (u64)h[32 * L + lane];
    return wave_sum64(v);
}

// S[g] = the sum of H[32 g, 32 g + 32) for the 64 groups of a 2048-bin
// histogram, by the whole workgroup: 4 bins per thread, then sums over each
// 8-lane group by DPP; ends with a barrier.
template <typename T>
__device__ __forceinline__ void group_sums(const T* H, T* S)
{
    const int tid = threadIdx.x;
    T v = H[4 * tid] + H[4 * tid + 1] + H[4 * tid + 2] + H[4 * tid + 3];
    v += dpp_step(v, (T)0, 0);   // lanes i-1, i-2, i-4 within the row:
    v += dpp_step(v, (T)0, 1);   // lane 8g + 7 then holds lanes 8g .. 8g + 7
    v += dpp_step(v, (T)0, 2);
    if ((tid & 7) == 7) S[tid >> 3] = v;
    __syncthreads();
}

// One element of a gathered bin per lane: its key, mass, the number of the
// bin's keys above it and their mass.
struct Ranked {
    u64 key, w, E;
    uint32_t gt;
    bool valid;
};
// Input, from the kernel's pass over the segments: every buffered element
// with l >= l_est carries its bin + 1 in bits 18 and up of its id word
// (V <= 2^18), the others 0 there; CH holds the counts per bin (2048 bins
// linear in d = l - m on [l_est - m, 0], monotone in the sorted order).
//
// CH turns into the offsets of the bins in descending order (a counting
// sort), which also names the bin kb of the k-th largest, and a second pass
// places the elements of the bins >= kb (they include the top-k
// set) there in the kept list KL, bin by bin, with their masses, which also
// go into MH / MS.  After that pass CH[b] is the end of bin b in KL and
// CH[b + 1] its start.  Wave 0 resolves the k-th, the top-p cut and the draw,
// each from the bin that holds it, read directly from KL.  Returns false,
// having written nothing but KL and CH, when a needed bin holds more than 64
// elements or KL would exceed KL_CAP: the caller then takes the general path.
constexpr int TAG_SHIFT = 18;
constexpr uint32_t ID_MASK = (1u << TAG_SHIFT) - 1u;
static_assert(MXS_MAX_VOCAB <= (1 << TAG_SHIFT), "ids and bin tags share a word");
constexpr int KL_CAP = 2048;
static_assert(KL_CAP * 16 <= KF_MH - KF_BM, "the kept list fits where the history bitmap was");

__device__ __forceinline__ bool finish_segs(const Params& p, int r, const uint32_t* ck, const uint32_t* ci,
                                            const uint32_t* seg, float T, bool neg, uint32_t kk, float m,
                                            float top_p, float u, u64* MH, uint32_t* CH, u64* MS, u64* KL,
                                            int64_t& tok, int32_t& st)
{
    __shared__ int g_fail;
    __shared__ u64 g_tok, g_wk, g_cut;
    __shared__ uint32_t g_vkk;
    __shared__ int g_st, g_bounded;
    const int wv = wave_id(), lane = lane_id();
    const int tid = threadIdx.x;
    const uint32_t cw = seg[wv];
    const uint32_t* wck = ck + wv * FSEG;
    const uint32_t* wci = ci + wv * FSEG;

    // CH -> exclusive offsets in descending bin order (this thread's 4 bins
    // are 2047 - 4 tid down to 2044 - 4 tid); the thread whose bins hold
    // position k - 1 names the k-th's bin
    __shared__ int g_kb;
    __shared__ uint32_t g_kabove, g_kn;
    {
        uint32_t c[4], sum = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) { c[i] = CH[2047 - 4 * tid - i]; sum += c[i]; }
        uint32_t total;
        uint32_t off = block_incl_scan<uint32_t>(sum, &total) - sum;   // (its barriers end the reads above)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = 2047 - 4 * tid - i;
            if (off <= kk - 1u && kk - 1u < off + c[i]) { g_kb = b; g_kabove = off; g_kn = c[i]; }
            CH[b] = off;
            off += c[i];
        }
    }
    __syncthreads();
    // (at least k elements are binned: the bound held)
    const int kb = g_kb;
    const uint32_t nabove = g_kabove, nkb = g_kn;
    if (__builtin_expect(nabove + nkb > (uint32_t)KL_CAP || nkb > 64u, 0)) return false;
    // the bins from kb up: masses, and their places in KL
    const uint32_t tkb = (uint32_t)kb + 1u;
    // four entries per lane at a time: loads, then arithmetic, then the
    // atomics, then the placements, each issued together
    for (uint32_t j0 = (uint32_t)lane; j0 < cw; j0 += 256) {
        uint32_t word[4], skv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t j = j0 + 64u * q < cw ? j0 + 64u * q : j0;
            word[q] = wci[j];
            skv[q] = wck[j];
        }
        bool in[4];
        float lq[4];
        u64 wq[4];
        uint32_t at[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            in[q] = j0 + 64u * q < cw && (word[q] >> TAG_SHIFT) >= tkb;
            lq[q] = sel_inv(skv[q], neg) / T;
            wq[q] = in[q] ? mass_of(lq[q] - m) : 0ull;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (in[q]) {
                const uint32_t b = (word[q] >> TAG_SHIFT) - 1u;
                atomicAdd(&MH[b], wq[q]);
                at[q] = atomicAdd(&CH[b], 1u);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (in[q]) {
                KL[2 * at[q]] = ((u64)vkey(lq[q]) << 32) | (u64)(0xFFFFFFFFu - (word[q] & ID_MASK));
                KL[2 * at[q] + 1] = wq[q];
            }
        }
    }
    __syncthreads();
    group_sums<u64>(MH, MS);
    const uint32_t nk = CH[kb];   // (the end of kb: the size of KL)
    if (wv == 0) {
        bool fail = false;
        const u64 ms = MS[lane];
        const u64 msuf = wave_suffix_incl(ms);   // (for every search below)
        const u64 Ak = wave_sum_above<u64>(MH, ms, kb);
        // bin b's elements, one per lane, ranked
        auto load_bin = [&](int b) -> Ranked {
            const uint32_t e = CH[b], s0 = b == 2047 ? 0u : CH[b + 1];
            const uint32_t n = e - s0;
            if (n > 64u) fail = true;
            Ranked q{0ull, 0ull, 0ull, 0u, (uint32_t)lane < n};
            if (q.valid) { q.key = KL[2 * (s0 + lane)]; q.w = KL[2 * (s0 + lane) + 1]; }
            // ranks by broadcast reads of the bin's keys, four at a time
            // (entries past the bin read as zero keys, which are below all)
            for (uint32_t i = 0; i < n; i += 4) {
                u64 o[4], ow[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const bool in = i + c < n;
                    o[c] = in ? KL[2 * (s0 + i + c)] : 0ull;
                    ow[c] = in ? KL[2 * (s0 + i + c) + 1] : 0ull;
                }
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const bool above = o[c] > q.key;
                    q.gt += above ? 1u : 0u;
                    q.E += above ? ow[c] : 0ull;
                }
            }
            return q;
        };
        // sampling.py:52-54: the k-th largest of its bin; its value ties stay
        Ranked q = load_bin(kb);
        int qb = kb;
        const uint32_t rk = (kk - 1u) - nabove;
        const u64 mk = __ballot(q.valid && q.gt == rk);
        if (!mk) fail = true;
        const uint32_t vkk = (uint32_t)(readlane64(q.key, mk ? __builtin_ctzll(mk) : 0) >> 32);
        const bool kept = q.valid && (uint32_t)(q.key >> 32) >= vkk;
        const u64 W = Ak + wave_sum64(kept ? q.w : 0ull);
        // the element at mass position x < W: its key, the mass before it, its mass
        auto pick_at = [&](u64 x, u64& key, u64& E, u64& w) {
            int b = kb;
            u64 A = Ak;
            if (x < Ak) {
                const WHit h = wave_find_desc_pre<u64>(MH, ms, msuf, x);
                b = h.bin;
                A = h.above;
            }
            if (b != qb) { q = load_bin(b); qb = b; }
            const bool elig = b == kb ? (q.valid && (uint32_t)(q.key >> 32) >= vkk) : q.valid;
            const u64 hm = __ballot(elig && A + q.E <= x && x < A + q.E + q.w);
            if (!hm) { fail = true; return; }
            const int l0 = __builtin_ctzll(hm);
            key = readlane64(q.key, l0);
            E = A + readlane64(q.E, l0);
            w = readlane64(q.w, l0);
        };
        int32_t rst = MXS_ROW_OK;
        u64 Wk = W, cutkey = 0, dkey = 0;
        bool bounded = false;
        if (top_p < 1.0f && !(top_p > 0.0f)) {
            rst = MXS_ROW_EMPTY_NUCLEUS;
        } else {
            u64 E, w;
            if (top_p < 1.0f) {   // sampling.py:56-63
                bounded = true;
                pick_at(ceil_mul(top_p, W) - 1, cutkey, E, w);
                Wk = E + w;
            }
            pick_at(floor_mul(clamp_uniform(u), Wk), dkey, E, w);   // sampling.py:69
        }
        if (lane == 0) {
            g_fail = fail ? 1 : 0;
            g_tok = dkey;
            g_wk = Wk;
            g_cut = cutkey;
            g_vkk = vkk;
            g_st = rst;
            g_bounded = bounded ? 1 : 0;
        }
    }
    __syncthreads();
    if (__builtin_expect(g_fail != 0, 0)) return false;
    st = g_st;
    if (st != MXS_ROW_OK) { tok = -1; return true; }
    tok = (int64_t)(0xFFFFFFFFu - (uint32_t)g_tok);
    if (p.out_probs) {   // sampling.py:68
        const u64 wkk = g_wk, cut = g_cut;
        const uint32_t vk_k = g_vkk;
        const bool bnd = g_bounded != 0;
        float* out = p.out_probs + (size_t)r * (size_t)p.V;
        for (uint32_t i = (uint32_t)tid; i < nk; i += NT) {
            const u64 key = KL[2 * i];
            if (bnd ? key >= cut : (uint32_t)(key >> 32) >= vk_k)
                out[0xFFFFFFFFu - (uint32_t)key] = (float)((double)KL[2 * i + 1] / (double)wkk);
        }
    }
    return true;
}

// ================================================================ k_fused
//
// One workgroup per row, the whole chain in one launch.  The row streams from
// HBM once, in 128-bit loads with two tiles of FTILE logits in flight per
// workgroup; the penalty is applied from an LDS bitmap of the row's history
// (inline, or to the buffered candidates afterwards).
//   greedy  a packed (key, index) maximum;
//   top-k   every element whose selection key reaches a lower bound theta on
//           the row's k-th largest key (from a sample, checked afterwards)
//           is appended to its wave's LDS segment; the segments are then
//           binned by mass and counting-sorted (finish_segs).  When the
//           bound fails or a segment fills, the row streams again into one
//           shared buffer whose bound rises by compaction whenever it nears
//           capacity;
//   other   the row's extreme keys, then the top-p-only path.

// Streams the row in tiles of FTILE logits, FTILE / NT = 16 per thread:
// elem(i, e, x) for slot i in [0, 16) of this thread's share of the tile,
// element index e and its penalized value x; then tile_end(id), called by all
// threads (it may synchronize), where id(i) is the element index of slot i in
// that tile; it returns true to stop the stream.  Slots past the row's end
// are skipped; in every wave the lanes that skip a slot are its highest
// ones, so a ballot taken in elem is complete in lane 0.
//
// A row that starts on a 16-byte boundary is read in 128-bit loads, one tile
// per register buffer, two buffers alternating so that the next tile is in
// flight while this one is processed.  The loads are unconditional (vectors
// past the row's end read its last vector again, tiles past the end its last
// tile): a branch around loads makes the compiler wait for all of them.
// Constructing a RowStream issues the first two tiles, so a kernel can create
// it before its set-up and overlap the two; run() consumes it once, restart()
// issues the first tiles again.
constexpr int FPT = FTILE / NT;   // logits per thread per tile (16)

__device__ __align__(16) const uint4 g_zero_vec = {0u, 0u, 0u, 0u};

template <typename TIn>
struct RowStream {
    typedef VecIO<TIn> IO;
    static constexpr int VW = IO::W;
    static constexpr int FU = FPT / VW;   // 16-byte loads per thread per tile
    static constexpr int TV = NT * FU;    // vectors per tile
    typedef typename IO::vec_t vec_t;

    const TIn* rowp;
    int V, nvec, ntile;
    vec_t A[FU], Bf[FU];

    // (issue = false: the first tiles are left for restart(); the loads are
    // issued all the same, of a dummy vector, since a branch around them
    // would make the compiler wait for every load in flight)
    __device__ __forceinline__ RowStream(const TIn* rp, int v, bool issue = true) : rowp(rp), V(v)
    {
        nvec = ((((uintptr_t)rp) & 15u) == 0) ? v / VW : 0;
        ntile = (nvec + TV - 1) / TV;
        restart(issue);
    }
    // The stream of another range of logits (the first two tiles issued).
    __device__ __forceinline__ void retarget(const TIn* rp, int v)
    {
        rowp = rp;
        V = v;
        nvec = ((((uintptr_t)rp) & 15u) == 0) ? v / VW : 0;
        ntile = (nvec + TV - 1) / TV;
        restart();
    }
    // The first two tiles.  The tile numbers pass through an empty asm
    // statement, so that the compiler computes these addresses at each use
    // instead of keeping one set alive (in scratch) for all the passes.
    __device__ __forceinline__ void restart(bool live = true)
    {
        int t0 = 0;
        asm volatile("" : "+s"(t0));
        load(A, t0, live);
        load(Bf, t0 + 1, live);
    }
    // (no branch: a row with no whole vector reads a dummy vector instead)
    __device__ __forceinline__ void load(vec_t (&b)[FU], int t, bool live = true)
    {
        typedef const __attribute__((address_space(1))) vec_t* gptr;   // global memory: plain vector loads
        const gptr src = (nvec > 0 && live) ? (gptr)rowp : (gptr)&g_zero_vec;
        const int lastv = (nvec > 0 && live) ? nvec - 1 : 0;
        t = t < ntile ? t : ntile - 1;
        t = t > 0 ? t : 0;
#pragma unroll
        for (int j = 0; j < FU; ++j) {
            const int vi = t * TV + j * NT + (int)threadIdx.x;
            b[j] = src[vi < lastv ? vi : lastv];
        }
    }
    // PART: the last tile, which may end inside the row's vectors.  ALL:
    // every slot is visited, elem(i, e, x, valid), so that no lane leaves the
    // others (a slot past the row's end has valid false and x a duplicate of
    // one of the row's values).
    template <bool PART, bool PEN, bool ALL, class Elem>
    __device__ __forceinline__ void proc(const vec_t (&b)[FU], int t, const uint32_t* bm, float pen, Elem& elem)
    {
        const int tid = threadIdx.x;
        uint32_t hw[FU];   // the history bitmap words of this tile, read together
        if constexpr (PEN) {
#pragma unroll
            for (int j = 0; j < FU; ++j) {
                const int vi = t * TV + j * NT + tid;
                hw[j] = (!PART || vi < nvec) ? bm[(vi * VW) >> 5] : 0u;
            }
        }
#pragma unroll
        for (int j = 0; j < FU; ++j) {
            const int vi = t * TV + j * NT + tid;
            if (!ALL && PART && vi >= nvec) continue;
            float xs[VW];
            IO::unpack(b[j], xs);
            const int e = vi * VW;
            if constexpr (PEN) {
                const uint32_t bits = (hw[j] >> (e & 31)) & ((1u << VW) - 1u);
                if (bits) {
#pragma unroll
                    for (int q = 0; q < VW; ++q)
                        if ((bits >> q) & 1u) xs[q] = penalize(xs[q], pen);
                }
            }
            if constexpr (ALL) {
                const bool valid = !PART || vi < nvec;
#pragma unroll
                for (int q = 0; q < VW; ++q) elem(j * VW + q, e + q, xs[q], valid);
            } else {
#pragma unroll
                for (int q = 0; q < VW; ++q) elem(j * VW + q, e + q, xs[q]);
            }
        }
    }
    // VAL: tile_end(id, val) also gets val(i), the raw (unpenalized) value
    // of slot i, read again from the tile's registers (they stay live until
    // the next load into them).
    template <bool PEN, bool ALL = false, bool VAL = false, class Elem, class TileEnd>
    __device__ __forceinline__ void run(const uint32_t* bm, float pen, Elem&& elem, TileEnd&& tile_end)
    {
        const int tid = threadIdx.x;
        const int nfull = nvec / TV;   // tiles wholly inside the row's vectors
        auto vid = [&](int t) {
            return [=](int i) { return (t * TV + (i / VW) * NT + tid) * VW + i % VW; };
        };
        auto end_of = [&](const vec_t (&b)[FU], int t) -> bool {
            if constexpr (VAL) {
                return tile_end(vid(t), [&](int i) {
                    float xs[VW];
                    IO::unpack(b[i / VW], xs);
                    return xs[i % VW];
                });
            } else {
                return tile_end(vid(t));
            }
        };
        // A holds tile t, Bf tile t + 1
        int t = 0;
        for (; t + 1 < nfull; t += 2) {
            proc<false, PEN, ALL>(A, t, bm, pen, elem);
            if (end_of(A, t)) return;
            load(A, t + 2);
            proc<false, PEN, ALL>(Bf, t + 1, bm, pen, elem);
            if (end_of(Bf, t + 1)) return;
            load(Bf, t + 3);
        }
        if (t < nfull) {
            proc<false, PEN, ALL>(A, t, bm, pen, elem);
            if (end_of(A, t)) return;
            ++t;
#pragma unroll
            for (int j = 0; j < FU; ++j) A[j] = Bf[j];   // (one call site for the last tile)
        }
        if (t < ntile) {
            proc<true, PEN, ALL>(A, t, bm, pen, elem);
            if (end_of(A, t)) return;
        }
        // the rest of the row (all of a row that is not 16-byte aligned), element by element
        for (int e0 = nvec * VW; e0 < V; e0 += FTILE) {
            float xs[FPT];
#pragma unroll
            for (int i = 0; i < FPT; ++i) {
                const int e = e0 + i * NT + tid;
                xs[i] = ALL ? IO::one(rowp, e < V ? e : V - 1) : (e < V ? IO::one(rowp, e) : 0.0f);
            }
#pragma unroll
            for (int i = 0; i < FPT; ++i) {
                const int e = e0 + i * NT + tid;
                if (ALL || e < V) {
                    const int ev = e < V ? e : V - 1;
                    float x = xs[i];
                    if constexpr (PEN) {
                        if ((bm[ev >> 5] >> (ev & 31)) & 1u) x = penalize(x, pen);
                    }
                    if constexpr (ALL) elem(i, e, x, e < V);
                    else elem(i, e, x);
                }
            }
            if constexpr (VAL) {
                if (tile_end([=](int i) { return e0 + i * NT + tid; }, [&](int i) { return xs[i]; })) return;
            } else {
                if (tile_end([=](int i) { return e0 + i * NT + tid; })) return;
            }
        }
    }
    // run() with the inline penalty chosen at run time
    template <class Elem, class TileEnd>
    __device__ __forceinline__ void run_pen(const uint32_t* bm, bool pen_inline, float pen, Elem&& elem,
                                            TileEnd&& tile_end)
    {
        if (pen_inline) run<true>(bm, pen, elem, tile_end);
        else run<false>(bm, pen, elem, tile_end);
    }
    // run_pen() whose tile_end gets each slot's raw value too: tile_end(id, val)
    template <class Elem, class TileEnd>
    __device__ __forceinline__ void run_pen_val(const uint32_t* bm, bool pen_inline, float pen, Elem&& elem,
                                                TileEnd&& tile_end)
    {
        if (pen_inline) run<true, false, true>(bm, pen, elem, tile_end);
        else run<false, false, true>(bm, pen, elem, tile_end);
    }
    // run_pen() visiting every slot: elem(i, e, x, valid)
    template <class Elem, class TileEnd>
    __device__ __forceinline__ void run_pen_all(const uint32_t* bm, bool pen_inline, float pen, Elem&& elem,
                                                TileEnd&& tile_end)
    {
        if (pen_inline) run<true, true>(bm, pen, elem, tile_end);
        else run<false, true>(bm, pen, elem, tile_end);
    }
    // One pass over the raw 16-bit values of an fp16 row: vec(v, e) for each
    // whole vector (elements e .. e + 7, two per 32-bit word), then
    // one(bits16, e) for the elements after the last whole vector.
    template <class Vec, class One>
    __device__ __forceinline__ void run_raw(Vec&& vec, One&& one)
    {
        static_assert(VW == 8, "fp16 rows");
        const int tid = threadIdx.x;
        const int nfull = nvec / TV;
        auto words = [&](const vec_t (&b)[FU], int t, bool part) {
#pragma unroll
            for (int j = 0; j < FU; ++j) {
                const int vi = t * TV + j * NT + tid;
                if (part && vi >= nvec) continue;
                vec(b[j], vi * VW);
            }
        };
        vec_t C[FU], D[FU];   // (four tiles in flight: the passes over fp16 rows wait on latency)
        load(C, 2);
        load(D, 3);
        int t = 0;
        for (; t + 3 < ntile; t += 4) {
            words(A, t, false);
            load(A, t + 4);
            words(Bf, t + 1, false);
            load(Bf, t + 5);
            words(C, t + 2, false);
            load(C, t + 6);
            words(D, t + 3, true);
            load(D, t + 7);
        }
        if (t < ntile) words(A, t, true);
        if (t + 1 < ntile) words(Bf, t + 1, true);
        if (t + 2 < ntile) words(C, t + 2, true);
        for (int e = nvec * VW + tid; e < V; e += NT) one((uint32_t)__builtin_bit_cast(uint16_t, rowp[e]), e);
    }
};

// One pass over a row from its first tile.
template <typename TIn, bool PEN, class Elem, class TileEnd>
__device__ __forceinline__ void stream_row(const TIn* rowp, int V, const uint32_t* bm, float pen,
                                           Elem&& elem, TileEnd&& tile_end)
{
    RowStream<TIn> rs(rowp, V);
    rs.template run<PEN>(bm, pen, elem, tile_end);
}

template <typename TIn, class Elem, class TileEnd>
__device__ __forceinline__ void stream_row_pen(const TIn* rowp, int V, const uint32_t* bm, bool pen_inline, float pen,
                                               Elem&& elem, TileEnd&& tile_end)
{
    RowStream<TIn> rs(rowp, V);
    rs.run_pen(bm, pen_inline, pen, elem, tile_end);
}

// Exclusive prefix over the wave of c (0 <= c < 32) and the wave's total,
// from bit-plane ballots (no cross-lane data movement).
__device__ __forceinline__ uint32_t wave_excl_small(uint32_t c, uint32_t& total)
{
    uint32_t pre = 0, tot = 0;
#pragma unroll
    for (int b = 0; b < 5; ++b) {
        const u64 m = __ballot((c >> b) & 1u);
        pre += lanes_below(m) << b;
        tot += (uint32_t)__builtin_popcountll(m) << b;
    }
    total = tot;
    return pre;
}

// ---------------------------------------------------------------- top-p only
//
// Rows with top-k off (k <= 0 or k >= V) in the fused kernel: the whole row
// takes part in the top-p cut (sampling.py:56-66).  One pass computes every
// element's integer mass and histograms the masses by bins linear in
// d = l - m; the cut and the draw each find their bin by a search over the
// mass histogram, gather that bin's elements (found by comparing selection
// keys with the bin's key interval, so the gathering pass does no division)
// and rank them.

struct SetPick {
    u64 key;   // (vkey << 32) | ~index
    u64 E;     // mass before it within the set, in sorted order
    u64 w;     // its mass
    int ok;
};

// The element at mass position t of the sorted order (value desc, index asc)
// of the n <= LCAP elements keys[0, n) (vkey(l) << 32 | ~index); masses are
// mass_of(l - m).  Sub-bins linear in d over the set's range; a sub-bin of
// more than 64 elements falls back to sorting the set in place.
__device__ __forceinline__ SetPick pick_in_set(u64* keys, int n, u64 t, float m, u64* SMH, uint32_t* SCH)
{
    __shared__ u64 q_key[64], q_w[64];
    __shared__ uint32_t q_n;
    __shared__ SetPick q_pick;
    const int tid = threadIdx.x;
    uint32_t vmax = 0, vmin = 0xFFFFFFFFu;
    for (int j = tid; j < n; j += NT) {
        const uint32_t vk = (uint32_t)(keys[j] >> 32);
        vmax = vk > vmax ? vk : vmax;
        vmin = vk < vmin ? vk : vmin;
    }
    const Reduced rd = block_reduce(vmax, vmin, 0u);
    const float dmin = okey_inv(rd.min) - m, dmax = okey_inv(rd.max) - m;
    float scale = dmax > dmin ? 2047.0f / (dmax - dmin) : 0.0f;
    if (!__builtin_isfinite(scale) || !(dmin > -INFINITY)) scale = 0.0f;
    auto sbin = [&](uint32_t vk) -> uint32_t {
        const float f = ((okey_inv(vk) - m) - dmin) * scale;
        return f > 0.0f ? (f < 2047.0f ? (uint32_t)f : 2047u) : 0u;
    };
    for (int b = tid; b < 2048; b += NT) { SMH[b] = 0; SCH[b] = 0; }
    if (tid == 0) { q_n = 0; q_pick = SetPick{0, 0, 0, 0}; }
    __syncthreads();
    for (int j = tid; j < n; j += NT) {
        const uint32_t vk = (uint32_t)(keys[j] >> 32);
        const uint32_t b = sbin(vk);
        atomicAdd(&SMH[b], mass_of(okey_inv(vk) - m));
        atomicAdd(&SCH[b], 1u);
    }
    __syncthreads();
    const BinHit hit = find_desc<u64>(SMH, 2048, t);
    const uint32_t cnt = SCH[hit.bin];
    if (cnt <= 64u) {
        for (int j = tid; j < n; j += NT) {
            const u64 key = keys[j];
            if (sbin((uint32_t)(key >> 32)) == (uint32_t)hit.bin) {
                const uint32_t slot = atomicAdd(&q_n, 1u);
                if (slot < 64u) { q_key[slot] = key; q_w[slot] = mass_of(okey_inv((uint32_t)(key >> 32)) - m); }
            }
        }
        __syncthreads();
        if (wave_id() == 0) {
            const uint32_t lane = (uint32_t)lane_id();
            const uint32_t c = q_n < 64u ? q_n : 64u;
            const u64 mk = lane < c ? q_key[lane] : 0ull;
            const u64 mw = lane < c ? q_w[lane] : 0ull;
            u64 before = 0;
            for (uint32_t q = 0; q < c; ++q) before += q_key[q] > mk ? q_w[q] : 0ull;
            const u64 E = hit.above + before;
            if (lane < c && E <= t && t < E + mw) q_pick = SetPick{mk, E, mw, 1};
        }
        __syncthreads();
        const SetPick res = q_pick;
        __syncthreads();
        return res;
    }
    // heavy ties: sort the set (descending) and scan its masses
    __syncthreads();
    const int P = pow2_ceil(n);
    for (int j = n + tid; j < P; j += NT) keys[j] = 0;
    __syncthreads();
    bitonic_sort_desc(keys, P);
    constexpr int PER = LCAP / NT;
    const int j0 = tid * PER;
    u64 wv[PER], run = 0;
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int j = j0 + q;
        wv[q] = j < n ? mass_of(okey_inv((uint32_t)(keys[j] >> 32)) - m) : 0ull;
        run += wv[q];
    }
    u64 tot;
    u64 E = block_incl_scan<u64>(run, &tot) - run;
    if (tid == 0) q_pick = SetPick{0, 0, 0, 0};
    __syncthreads();
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int j = j0 + q;
        if (j < n && E <= t && t < E + wv[q]) q_pick = SetPick{keys[j], E, wv[q], 1};
        E += wv[q];
    }
    __syncthreads();
    const SetPick res = q_pick;
    __syncthreads();
    return res;
}

// Smallest s in [lo, hi] with pred(s), for pred monotone (false, then true);
// hi + 1 when pred(hi) is false.  Called by a whole wave, 64 probes per step;
// every step narrows [lo, hi], so it ends within 6 steps per 32 bits.
template <class Pred>
__device__ __forceinline__ uint32_t wave_first_true(uint32_t lo, uint32_t hi, Pred pred)
{
    const uint32_t lane = (uint32_t)lane_id();
    if (!__ballot(lane == 0u && pred(hi))) return hi + 1u;
    while (lo < hi) {
        const u64 span = (u64)(hi - lo);
        const uint32_t pt = lo + (uint32_t)((span * (lane + 1u)) >> 6);   // lane 63 probes hi
        const u64 msk = __ballot(pred(pt));
        const int f = __builtin_ctzll(msk);   // (msk != 0: pred(hi) holds and lane 63 probes hi)
        const uint32_t nhi = (uint32_t)__builtin_amdgcn_readlane((int)pt, f);
        const uint32_t nlo = f > 0 ? (uint32_t)__builtin_amdgcn_readlane((int)pt, f - 1) + 1u : lo;
        lo = nlo;
        hi = nhi;
    }
    return lo;
}

// Top-p cut and draw over a whole row (top-k off).  skmax / skmin: the
// largest and smallest selection keys of the penalized row.  The passes here
// read raw values; the history ids (each once, from the bitmap) are then
// corrected to their penalized values, so no pass branches on the penalty
// per element.  Returns false when a bin holds more than LCAP elements (the
// caller's multi-level path takes over).
template <typename TIn>
__device__ __forceinline__ bool finish_wide(const Params& p, int r, float T, bool neg, float top_p, float u, float pen,
                                            bool pen_on, const uint32_t* bm, const uint32_t* hl, uint32_t nh,
                                            uint32_t skmax, uint32_t skmin, u64* MH, uint32_t* CH, u64* keys_c,
                                            u64* keys_d, u64* SMH, uint32_t* SCH, int64_t& tok, int32_t& st)
{
    __shared__ uint32_t g_iv[4], g_cnt[2];
    const int tid = threadIdx.x;
    const int V = p.V;
    const TIn* rowp = (const TIn*)p.logits + (size_t)r * (size_t)p.ld;
    const float m = sel_inv(skmax, neg) / T;
    if (!isfinite(m)) { st = MXS_ROW_NONFINITE; tok = -1; return true; }
    float dlo = sel_inv(skmin, neg) / T - m;
    if (!(dlo > -104.0f)) dlo = -104.0f;   // masses below are zero
    float scale = dlo < 0.0f ? 2047.0f / -dlo : 0.0f;
    if (!__builtin_isfinite(scale)) scale = 0.0f;
    auto bin_of = [&](float d) -> uint32_t {   // monotone in d
        const float f = (d - dlo) * scale;
        return f > 0.0f ? (f < 2047.0f ? (uint32_t)f : 2047u) : 0u;
    };
    // f(id, raw value) for every history id once: from the list (loads four
    // at a time), or from the bitmap's set bits if the list overflowed
    auto for_history = [&](auto&& f) {
        if (nh <= (uint32_t)HCAP) {
            for (uint32_t i0 = tid; i0 < nh; i0 += 4 * NT) {
                int id[4];
                float xv[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t i = i0 + (uint32_t)(q * NT);
                    id[q] = i < nh ? (int)hl[i] : -1;
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) xv[q] = id[q] >= 0 ? VecIO<TIn>::one(rowp, id[q]) : 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (id[q] >= 0) f(id[q], xv[q]);
            }
        } else {
            const int words = (V + 31) >> 5;
            for (int wd = tid; wd < words; wd += NT) {
                uint32_t bits = bm[wd];
                while (bits) {
                    const int bi = __builtin_ctz(bits);
                    bits &= bits - 1u;
                    f(wd * 32 + bi, VecIO<TIn>::one(rowp, wd * 32 + bi));
                }
            }
        }
    };
    auto is_history = [&](int e) { return ((bm[e >> 5] >> (e & 31)) & 1u) != 0u; };

    // sampling.py:57-59: every element's mass, histogrammed by bin (masses
    // without branches: count_mass(1, d) is mass_of(d) for d <= 0, and the
    // raw value of a history id, which may lie above m, is taken out again
    // with the same function below)
    for (int b = tid; b < 2048; b += NT) MH[b] = 0;
    __syncthreads();
    u64 wsum = 0;
    stream_row<TIn, false>(rowp, V, bm, pen,
        [&](int, int, float x) {
            const float l = x / T;
            const float d = l - m;
            const u64 w = count_mass(1u, d);
            atomicAdd(&MH[bin_of(d)], w);
            wsum += w;
        },
        [&](auto&&) { return false; });
    if (pen_on) {   // the history ids: raw contribution out, penalized one in
        for_history([&](int, float x) {
            const float d0 = x / T - m, d1 = penalize(x, pen) / T - m;
            const u64 w0 = count_mass(1u, d0), w1 = count_mass(1u, d1);
            atomicAdd(&MH[bin_of(d0)], 0ull - w0);
            atomicAdd(&MH[bin_of(d1)], w1);
            wsum += w1 - w0;
        });
    }
    const u64 W = block_sum<u64>(wsum);   // (its barriers publish the histograms)

    // The elements of bins bc and bd (bd < 0: none) into keys_c / keys_d as
    // (vkey(l) << 32 | ~index), found by comparing selection keys with each
    // bin's key interval.  Returns false if a set exceeds LCAP.
    auto gather = [&](int bc, int bd) -> bool {
        if (wave_id() == 0) {
            const uint32_t KHI = 0xFF800000u;   // selection keys of real values: [SK_MIN, KHI]
            auto first_at_least = [&](uint32_t b) -> uint32_t {
                if (b > 2047u) return KHI + 1u;
                return wave_first_true(SK_MIN, KHI, [&](uint32_t sk) { return bin_of(sel_inv(sk, neg) / T - m) >= b; });
            };
            const uint32_t ca = first_at_least((uint32_t)bc), cb = first_at_least((uint32_t)bc + 1u) - 1u;
            uint32_t da = 1u, db = 0u;   // empty
            if (bd >= 0) { da = first_at_least((uint32_t)bd); db = first_at_least((uint32_t)bd + 1u) - 1u; }
            if (lane_id() == 0) { g_iv[0] = ca; g_iv[1] = cb; g_iv[2] = da; g_iv[3] = db; g_cnt[0] = 0; g_cnt[1] = 0; }
        }
        __syncthreads();
        const uint32_t ca = g_iv[0], cb = g_iv[1], da = g_iv[2], db = g_iv[3];
        auto put = [&](uint32_t sk, float x, int e) {
            const u64 key = ((u64)vkey(x / T) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)e);
            if (sk >= ca && sk <= cb) {
                const uint32_t slot = atomicAdd(&g_cnt[0], 1u);
                if (slot < (uint32_t)LCAP) keys_c[slot] = key;
            } else if (sk >= da && sk <= db) {
                const uint32_t slot = atomicAdd(&g_cnt[1], 1u);
                if (slot < (uint32_t)LCAP) keys_d[slot] = key;
            }
        };
        stream_row<TIn, false>(rowp, V, bm, pen,
            [&](int, int e, float x) {
                const uint32_t sk = selkey(x, neg);
                if ((sk >= ca && sk <= cb) || (sk >= da && sk <= db)) {
                    if (!(pen_on && is_history(e))) put(sk, x, e);
                }
            },
            [&](auto&&) { return false; });
        if (pen_on) {
            for_history([&](int e, float x0) {
                const float x = penalize(x0, pen);
                put(selkey(x, neg), x, e);
            });
        }
        __syncthreads();
        const bool ok = g_cnt[0] <= (uint32_t)LCAP && g_cnt[1] <= (uint32_t)LCAP;
        return ok;
    };

    bool bounded = false;
    u64 bound = 0, Wk = W;
    SetPick dp{0, 0, 0, 0};
    if (top_p < 1.0f) {   // sampling.py:56-63
        if (!(top_p > 0.0f)) { st = MXS_ROW_EMPTY_NUCLEUS; tok = -1; return true; }
        const u64 t = ceil_mul(top_p, W) - 1;
        const BinHit hc = find_desc<u64>(MH, 2048, t);
        const u64 A = hc.above;
        // where the draw can land: Wk lies in (A, A + mass of the cut's bin]
        const u64 Dlo = floor_mul(clamp_uniform(u), A), Dhi = floor_mul(clamp_uniform(u), A + MH[hc.bin]);
        int bd = -1;
        if (Dhi < A) {
            const BinHit h1 = find_desc<u64>(MH, 2048, Dlo);
            const BinHit h2 = find_desc<u64>(MH, 2048, Dhi);
            if (h1.bin == h2.bin) bd = h1.bin;
        }
        if (!gather(hc.bin, bd)) return false;
        const int nc = (int)g_cnt[0], nd = (int)g_cnt[1];
        const SetPick c = pick_in_set(keys_c, nc, t - A, m, SMH, SCH);
        if (!c.ok) return false;
        bounded = true;
        bound = c.key;
        Wk = A + c.E + c.w;
        const u64 D = floor_mul(clamp_uniform(u), Wk);   // sampling.py:69
        if (D >= A) {
            dp = pick_in_set(keys_c, nc, D - A, m, SMH, SCH);   // the cut's bin (its kept part lies below Wk)
        } else {
            const BinHit hd = find_desc<u64>(MH, 2048, D);   // a bin above the cut's, wholly kept
            if (hd.bin != bd) {
                if (!gather(hd.bin, -1)) return false;
                dp = pick_in_set(keys_c, (int)g_cnt[0], D - hd.above, m, SMH, SCH);
            } else {
                dp = pick_in_set(keys_d, nd, D - hd.above, m, SMH, SCH);
            }
        }
    } else {
        const u64 D = floor_mul(clamp_uniform(u), W);   // sampling.py:69
        const BinHit hd = find_desc<u64>(MH, 2048, D);
        if (!gather(hd.bin, -1)) return false;
        dp = pick_in_set(keys_c, (int)g_cnt[0], D - hd.above, m, SMH, SCH);
    }
    if (!dp.ok) return false;
    tok = (int64_t)(0xFFFFFFFFu - (uint32_t)dp.key);
    st = MXS_ROW_OK;
    if (p.out_probs) {   // sampling.py:68
        float* out = p.out_probs + (size_t)r * (size_t)V;
        stream_row_pen<TIn>(rowp, V, bm, pen_on, pen,
            [&](int, int e, float x) {
                const float l = x / T;
                const u64 key = ((u64)vkey(l) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)e);
                if (!bounded || key >= bound) out[e] = (float)((double)mass_of(l - m) / (double)Wk);
            },
            [&](auto&&) { return false; });
    }
    return true;
}

// ---------------------------------------------------------------- top-k off, two passes
//
// A row with top-k off takes part in the top-p cut and the draw as a whole
// (sampling.py:56-69).  finish_wide2 reads it twice, with the penalty
// applied from the history bitmap in both passes:
//   pass 1   the row's extremes; every element at or above the sample's
//            largest (penalized) value yhi into an exact list, the top list
//            (per-wave segments, as the top-k stream fills them); every
//            other element counted in one of 2048 bins linear in its value
//            over the sample's range [ylo, yhi) (values below ylo in bin 0);
//   between  the top list's exact masses (total W_top), and for every bin a
//            lower and an upper bound on its mass, from its count and the
//            masses of its value edges; so bounds on the total W, on the
//            positions of the top-p cut and of the draw, and a window of
//            bins for each that must hold it when it is not in the top list;
//   pass 2   the exact mass of every element below yhi, summed in
//            registers (no atomics), the mass of the elements above each
//            window, and the elements of the two windows gathered.
// The cut and the draw are then exact picks from the top list or from their
// window (pick_in_set).  Values y are ordered like the tempered values:
// y = x for T > 0, -x for T < 0, and l = y / |T|.
//
// The top list's threshold is widened over the rounding of y / |T|, so that
// every element tied in l with it is in the list; a tie in l can still
// straddle a bin boundary (bins are at least 1000 ulps wide, so a tie group
// meets at most two bins), so each window is gathered with one more bin on
// either side and the mass above it is counted above that wider range: the
// positions inside the window proper are then exact.
//
// Returns 1 when the row is done (token, or a status); 0 when the general
// path must take over after pass 1, with rd holding the penalized row's
// extreme keys; -1 when the sample's range is degenerate (nothing read
// beyond the sample; the caller streams the row as before).
constexpr int TL_CAP = 2048;             // the top list (u64 keys where the mass histogram was)
constexpr int W2_KC = KF_CK;             // pass 2: the cut's window (LCAP u64)
constexpr int W2_KD = KF_CK + 8 * LCAP;  //         the draw's window (LCAP u64)
constexpr int W2_SMH = KF_CK + 16 * LCAP;   // pick_in_set's masses (2048 u64)
static_assert(W2_SMH + 16384 <= KF_HL, "the windows and pick_in_set's masses fit below the history list");
static_assert(TL_CAP * 8 <= KF_H - KF_MH, "the top list fits where the mass histogram was");
static_assert(WJ_S * WJ_TOPS == TL_CAP && WJ_S * WJ_WINS == LCAP, "a job's lists hold what the owner's do");
constexpr uint32_t W2_SEG_USE = FSEG - 64;   // a wave segment's room (the rest: dummy slots)

// ---- shared rows: the records (sampler_params.h has their layout)
//
// A pass of a shared row is cut into S slices of tps tiles (S <= WJ_S).  The
// owner streams the row from its first tile and claims the slices from the
// front, each one two tiles before it reaches it (so the claim's round trip
// hides behind the stream); helpers claim from the back.  Both claims are
// additions to one word per pass, (back << 16) | front: a claim is granted
// when front + back < S before it, so the first S claims, in the word's
// order, take every slice exactly once (the owner's [0, taken), the
// helpers' [taken, S)) and every later claim is refused.
struct WideJob {
    u64 tag;                          // (epoch << 32) | (WJ_MAGIC << 16) | (S << 8) | phase (1, 2 open; 3 closed)
    uint32_t own;                     // the epoch of the call whose row holds the slot
    uint32_t tps;                     // tiles per slice
    uint32_t q1, q2;                  // the claims of pass 1 and pass 2 (adjacent: one 64-bit read)
    uint32_t done1, done2;            // slices of each pass finished by helpers
    int r, h0, h1, pad0;              // the row, its history
    float T, pen, yhi, ylo, scale, m, yca, ycb, yda, ydb;
    uint32_t neg, pen_on;
    uint32_t gmax, gmin;              // pass 1: the helpers' key extremes
    uint32_t ovf;                     // pass 1: a helper's segment ran full
    uint32_t ver;                     // (job 0's) bumped when a pass opens or a job closes
};
static_assert(sizeof(WideJob) <= WJ_HDR, "a job's header");
static_assert(WJ_S < 256 && WJ_NJOB <= 64, "S fits the tag; one lane per job");
constexpr uint32_t WJ_MAGIC = 0xA5C7u;
constexpr int WJ_SPIN = 1 << 21;      // bounded waits: polls of about 50 ns each

__device__ __forceinline__ WideJob* wj_job(unsigned char* wj, int j) { return (WideJob*)(wj + (size_t)j * WJ_JOB_BYTES); }
// a word of workgroup (or row) r's own, which its unshared passes read (a
// line each; beyond WJ_OWN they share)
__device__ __forceinline__ uint32_t* wj_own_word(const Params& p, int r) { return p.wown + (size_t)(r % WJ_OWN) * 16; }
__device__ __forceinline__ uint32_t* wj_bins(WideJob* J) { return (uint32_t*)((unsigned char*)J + WJ_HDR); }
// slice s's top-list entries and window elements, the slices' counts of
// them ([0]: top list, [1], [2]: windows, WJ_S each), the history bitmap
__device__ __forceinline__ u64* wj_top(WideJob* J, int s) { return (u64*)(wj_bins(J) + 2048) + (size_t)s * WJ_TOPS; }
__device__ __forceinline__ u64* wj_kc(WideJob* J, int s) { return wj_top(J, WJ_S) + (size_t)s * WJ_WINS; }
__device__ __forceinline__ u64* wj_kd(WideJob* J, int s) { return wj_kc(J, WJ_S) + (size_t)s * WJ_WINS; }
__device__ __forceinline__ uint32_t* wj_cnt(WideJob* J, int list) { return (uint32_t*)wj_kd(J, WJ_S) + list * WJ_S; }
__device__ __forceinline__ uint32_t* wj_bm(WideJob* J) { return wj_cnt(J, 3); }
// The records' version (job 0's ver): owners add 1 after a pass opens or a
// job closes, so that idle helpers poll one word and scan the jobs only when
// it moves.
__device__ __forceinline__ void wj_bump(unsigned char* wj)
{
    __builtin_amdgcn_s_waitcnt(0);   // (the tag before the version)
    atomicAdd(&wj_job(wj, 0)->ver, 1u);
}
// slice s's pass-2 sums: wb, ac, ad at [0], [WJ_S], [2 WJ_S]
__device__ __forceinline__ u64* wj_sums(WideJob* J, int s) { return (u64*)(wj_bm(J) + WJ_BMW) + s; }
__device__ __forceinline__ u64 wj_tag(uint32_t epoch, int S, uint32_t phase)
{
    return ((u64)epoch << 32) | ((u64)WJ_MAGIC << 16) | ((u64)S << 8) | phase;
}
// device-scope accesses of the records (they bypass a stale copy in this
// XCD's caches; stores write through, see put_dev)
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* a)
{
    return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 ld_dev64(const u64* a) { return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ float ld_devf(const float* a) { return u2f(ld_dev((const uint32_t*)a)); }
__device__ __forceinline__ void put_dev32(uint32_t* a, uint32_t v)
{
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void put_dev64(u64* a, u64 v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void put_devf(float* a, float v) { put_dev32((uint32_t*)a, f2u(v)); }

// The batch's rows with top-k off among its first NT rows, a bit per row,
// wave w's ballot over rows [64 w, 64 w + 64) at the start of fused_row
// (k_fused): their count, and a row's rank among them.
__shared__ u64 g_wide[NWAVES];
__device__ __forceinline__ uint32_t wide_rows_counted()
{
    uint32_t n = 0;
#pragma unroll
    for (int v = 0; v < NWAVES; ++v) n += (uint32_t)__builtin_popcountll(g_wide[v]);
    return n;
}
__device__ __forceinline__ int wide_rank(int r)
{
    int n = 0;
#pragma unroll
    for (int v = 0; v < NWAVES; ++v) {
        const u64 m = g_wide[v];
        n += v < (r >> 6) ? __builtin_popcountll(m) : 0;
        n += v == (r >> 6) ? __builtin_popcountll(m & ((1ull << (r & 63)) - 1ull)) : 0;
    }
    return n;
}

// The owner's claims from the front (q the pass's word).  A range that is
// all this workgroup's has every slice taken (taken = issued = S) and q a
// word of its own, which it reads after every tile like a claim, so that
// one instance of each pass serves both.  Slice s starts at tile s tps; its claim is issued
// when t = s tps - 1 tiles are done and checked one tile later, before the
// slice's first tile is processed.  after_tile() is true when that slice is
// a helper's: the stream stops there, with slices [0, taken) done.  Thread
// 0 adds to the word after every tile (1 for a claim, else 0: a read), so
// that its result is defined on every path and waited for only where it is
// read.  go: two LDS words, used in turn (one barrier per check).
// A pass with no claims (every instance that shares nothing, and a
// helper's slice): the whole range is this workgroup's.  (Its go words
// are never touched.)
__device__ __forceinline__ uint32_t* hc_go_dummy() { return nullptr; }
struct NoClaims {
    int taken;
    int ntile = 0;
    __device__ __forceinline__ bool after_tile(uint32_t*) { return false; }
};
struct FrontClaims {
    uint32_t* q;
    int S, tps, taken;
    int issued;          // slices [0, issued) claimed or pre-owned (at first, taken)
    int ntile = 0, t = 0;
    uint32_t pend = 0;   // (thread 0) the word before the last addition
    __device__ __forceinline__ bool after_tile(uint32_t* go)
    {
        ++t;
        if (taken < issued && t == taken * tps && t < ntile) {
            uint32_t* g = go + (taken & 1);
            if (threadIdx.x == 0) *g = (pend & 0xFFFFu) + (pend >> 16) < (uint32_t)S ? 1u : 0u;
            __syncthreads();
            if (*g == 0u) return true;
            ++taken;
        }
        const bool claim = issued < S && t == issued * tps - 1;
        // (the address passes through a register, so the compiler does not
        // aggregate the addition over the wave, which would wait for its
        // result at once; a global pointer, since a flat access would also
        // hold the LDS counter)
        typedef __attribute__((address_space(1))) uint32_t gu32;
        gu32* qv = (gu32*)q;
        asm volatile("" : "+v"(qv));
        uint32_t nv = 0u;
        if (threadIdx.x == 0) nv = __hip_atomic_fetch_add(qv, claim ? 1u : 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pend = nv;
        issued += claim ? 1 : 0;
        return false;
    }
};

// ---- the two passes over a range [s0, s0 + n) of the row (a whole row, or
// one slice; s0 a multiple of 32 so that the history bitmap's words align)

// Pass 1: extremes (fmx, fmn), the elements at or above yhi into this
// wave's segment (cw entries; *ovf set when it runs full), every other
// element counted in its bin of CH.  fresh: rs already streams this range
// (the row's first tiles, issued at the kernel's start).  fc: the owner's
// claims of a shared row's slices (a workgroup's own range: all slices
// taken, fc.q a word of its own, see FrontClaims).
template <typename TIn, class FC>
__device__ __forceinline__ void w2_pass1(RowStream<TIn>& rs, const TIn* rowp, int s0, int n, const uint32_t* bm,
                                         bool pen_on, float pen,
                                         bool neg, float yhi, float ylo, float scale, uint32_t* CH,
                                         uint32_t* wck, uint32_t* wci, uint32_t& cw, float& fmx, float& fmn,
                                         uint32_t* ovf, uint32_t* dummy, FC& fc, uint32_t* go,
                                         bool fresh = false)
{
    const int lane = lane_id();
    auto yv = [&](float x) { return neg ? -x : x; };
    auto bin_of = [&](float y) -> uint32_t {   // (a NaN goes to bin 0)
        const float f = (y - ylo) * scale;
        return f >= 1.0f ? (f < 2047.0f ? (uint32_t)f : 2047u) : 0u;
    };
    float tx[FPT];
    uint32_t nhit = 0;
    if (!fresh) rs.retarget(rowp + s0, n);
    fc.ntile = rs.ntile;
    rs.run_pen_all(pen_on ? bm + (s0 >> 5) : bm, pen_on, pen,
        [&](int i, int, float x, bool valid) {
            fmx = __builtin_elementwise_maximum(fmx, x);
            fmn = __builtin_elementwise_minimum(fmn, x);
            const float y = yv(x);
            const bool top = valid && y >= yhi;
            tx[i] = top ? x : __builtin_nanf("");
            nhit += top ? 1u : 0u;
            atomicAdd(valid && !top ? &CH[bin_of(y)] : dummy, 1u);   // (no branch per element)
        },
        [&](auto&& id) -> bool {
            const uint32_t incl = wave_prefix_u32(nhit);
            const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            if (__builtin_expect(cw + tot > W2_SEG_USE, 0)) {
                if (lane == 0) __hip_atomic_store(ovf, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                cw = W2_SEG_USE;   // (the rest of the range still counts toward the extremes)
                nhit = 0;
                return fc.after_tile(go);   // (the claims stay in step with the tiles)
            }
            uint32_t o = cw + incl - nhit;
            const uint32_t dmy = W2_SEG_USE + (uint32_t)lane;
#pragma unroll
            for (int i = 0; i < FPT; ++i) {
                const bool h = tx[i] == tx[i];
                const uint32_t a = h ? o : dmy;
                wck[a] = f2u(tx[i]);
                wci[a] = (uint32_t)(s0 + id(i));
                o += h ? 1u : 0u;
            }
            nhit = 0;
            cw += tot;
            return fc.after_tile(go);
        });
}

// fl32(x / T) from rT = RN64(1 / T): x * rT in binary64 is within 2^-52
// (relative) of x / T, and x / T is never a binary32 rounding boundary (an
// odd 25-bit midpoint times T needs more than 24 significant bits) nor
// nearer to one than 2^-49 (relative) while its quotient is normal, so the
// product rounds to binary32 exactly as the IEEE quotient does.  A
// subnormal quotient may differ by its last bit; pass 2 uses it only in
// d = fl32(l - m), which it leaves unchanged when m = 0 or |m| >= 2^-101
// (the row's maximum; finish_wide2 checks).  Infinities, zeros and NaN
// pass through as in the division.  Two conversions and one binary64
// multiply in place of the division's reciprocal and refinement steps.
__device__ __forceinline__ float div_by_rT(float x, double rT) { return (float)((double)x * rT); }

// Pass 2: the exact masses of the elements below yhi summed (wb), and those
// at or above ycb (ac) and ydb (ad); the elements of the windows [yca, ycb)
// and [yda, ydb) listed in KC and KD (counts in cnt[0], cnt[1]).  fc as
// for pass 1.
template <typename TIn, class FC>
__device__ __forceinline__ void w2_pass2(RowStream<TIn>& rs, const TIn* rowp, int s0, int n, const uint32_t* bm,
                                         bool pen_on, float pen,
                                         bool neg, float T, double rT, float m, float yhi, float yca, float ycb,
                                         float yda,
                                         float ydb, u64& wb, u64& ac, u64& ad, uint32_t* cnt, u64* KC, u64* KD,
                                         FC& fc, uint32_t* go)
{
    auto yv = [&](float x) { return neg ? -x : x; };
    auto has_pen = [&](int e) { return pen_on && ((bm[e >> 5] >> (e & 31)) & 1u); };
    uint32_t mc = 0, md = 0;   // this tile's window elements, a bit per slot
    rs.retarget(rowp + s0, n);
    fc.ntile = rs.ntile;
    rs.run_pen_val(pen_on ? bm + (s0 >> 5) : bm, pen_on, pen,
        [&](int i, int, float x) {
            const float y = yv(x);
            const float l = div_by_rT(x, rT);
            const u64 wgt = y >= yhi ? 0ull : count_mass(1u, l - m);
            wb += wgt;
            ac += y >= ycb ? wgt : 0ull;
            ad += y >= ydb ? wgt : 0ull;
            mc |= (y >= yca && !(y >= ycb) ? 1u : 0u) << i;
            md |= (y >= yda && !(y >= ydb) ? 1u : 0u) << i;
        },
        [&](auto&& id, auto&& val) -> bool {
            if (__ballot((mc | md) != 0u)) {
#pragma unroll
                for (int i = 0; i < FPT; ++i) {
                    if (((mc | md) >> i) & 1u) {
                        const int e = s0 + id(i);
                        float x = val(i);
                        if (has_pen(e)) x = penalize(x, pen);
                        const u64 key = ((u64)vkey(x / T) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)e);
                        if ((mc >> i) & 1u) {
                            const uint32_t s = atomicAdd(&cnt[0], 1u);
                            if (s < (uint32_t)LCAP) KC[s] = key;
                        }
                        if ((md >> i) & 1u) {
                            const uint32_t s = atomicAdd(&cnt[1], 1u);
                            if (s < (uint32_t)LCAP) KD[s] = key;
                        }
                    }
                }
            }
            mc = 0;
            md = 0;
            return fc.after_tile(go);
        });
}

// A helper's claim from the back of a pass (thread 0): the slice, or -1
// when every slice is taken.
__device__ __forceinline__ int wj_claim_back(uint32_t* q, int S)
{
    const uint32_t old = atomicAdd(q, 1u << 16);
    return (old & 0xFFFFu) + (old >> 16) < (uint32_t)S ? S - 1 - (int)(old >> 16) : -1;
}
// Counts this workgroup's slice done, after every wave's results are
// acknowledged (they were written through, or added at device scope).
__device__ __forceinline__ void wj_done(uint32_t* done)
{
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) atomicAdd(done, 1u);
}
// The owner's wait until the helpers finished need slices of a pass
// (thread 0 polls, bounded); then their results are acquired.  False: the
// wait timed out.
__device__ __forceinline__ bool wj_wait(const uint32_t* done, int need)
{
    __shared__ int s_ok;
    if (threadIdx.x == 0) {
        int ok = need <= 0 ? 1 : 0;
        for (int it = 0; it < WJ_SPIN && !ok; ++it) {
            if (ld_dev(done) >= (uint32_t)need) ok = 1;
            else __builtin_amdgcn_s_sleep(2);
        }
        if (ok) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        s_ok = ok;
    }
    __syncthreads();
    const bool ok = s_ok != 0;
    __syncthreads();
    return ok;
}

template <typename TIn, bool SH>
__device__ __forceinline__ int finish_wide2(const Params& p, int r, RowStream<TIn>& rs, float T, bool neg,
                                            float top_p, float u, float pen, bool pen_on, const uint32_t* bm,
                                            const float (&sx)[NSAMP / NT], int se0, int h0, int h1,
                                            unsigned char* smem, uint32_t* CH, Reduced& rd, int64_t& tok, int32_t& st)
{
    constexpr int NS = NSAMP / NT;
    __shared__ uint32_t w2_seg[NWAVES], w2_ovf, w2_cnt[2], w2_dummy, w2_go[2];
    __shared__ uint32_t w2_sc[WJ_S], w2_so[WJ_S], w2_tot;   // helpers' slices: counts, offsets, total
    __shared__ u64 w2_hs[3];                                 // their pass-2 sums
    __shared__ uint32_t w2_r[4][NWAVES];
    __shared__ u64 w2_s[3][NWAVES];
    __shared__ int w2_job;
    const int tid = threadIdx.x, lane = lane_id(), wv = wave_id();
    const int V = p.V;
    const TIn* rowp = (const TIn*)p.logits + (size_t)r * (size_t)p.ld;
    uint32_t* ck = (uint32_t*)(smem + KF_CK);
    uint32_t* ci = (uint32_t*)(smem + KF_CI);
    u64* TL = (u64*)(smem + KF_MH);
    u64* KC = (u64*)(smem + W2_KC);
    u64* KD = (u64*)(smem + W2_KD);
    u64* SMH = (u64*)(smem + W2_SMH);
    auto yv = [&](float x) { return neg ? -x : x; };
    auto has_pen = [&](int e) { return pen_on && ((bm[e >> 5] >> (e & 31)) & 1u); };

    // the sample's range of (penalized) values
    uint32_t kmx = 0, kmn = 0xFFFFFFFFu;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        float x = sx[q];
        if (has_pen(se0 + q)) x = penalize(x, pen);
        const uint32_t ky = okey(yv(x));
        kmx = ky > kmx ? ky : kmx;
        kmn = ky < kmn ? ky : kmn;
    }
    for (int b = tid; b < 2048; b += NT) CH[b] = 0;
    if (tid == 0) { w2_ovf = 0; w2_cnt[0] = 0; w2_cnt[1] = 0; }
    const Reduced sr = block_reduce(kmx, kmn, 0u);   // (its barriers also order the zeroed counts)
    if (!(sr.max > SK_MIN && sr.max < 0xFF800000u && sr.min >= SK_MIN && sr.min < sr.max)) return -1;
    const float yhi = okey_inv(widen_threshold(sr.max, T, neg)), ylo = okey_inv(sr.min);
    const float dy = (yhi - ylo) * 0x1p-11f;
    const float scale = 2048.0f / (yhi - ylo);
    // (bins wider than 1000 ulps of the values at their edges, all finite)
    const float umax = __builtin_fmaxf(__builtin_fabsf(yhi), __builtin_fabsf(ylo)) * 0x1p-23f;
    if (!(yhi > ylo) || !__builtin_isfinite(scale) || !__builtin_isfinite(dy) || !(dy > 1000.0f * umax))
        return -1;

    // The row's job: other workgroups may take slices of both passes, when
    // the batch has rows that do not share (helpers), the row's vectors are
    // whole (slices start at tiles), and no probabilities are written (that
    // third read stays here).  The slot: the row's rank among the batch's
    // rows with top-k off (the first WJ_NJOB of them share); in a batch of
    // more than NT rows, r mod WJ_NJOB, held by the first row of the call
    // to take it (another row goes alone).
    typedef VecIO<TIn> IO;
    const int ntile = (V / IO::W + NT * (FPT / IO::W) - 1) / (NT * (FPT / IO::W));
    const int tps = (ntile + WJ_S - 1) / WJ_S;
    const int S = (ntile + tps - 1) / tps;
    const int f0 = S < (tps == 1 ? 2 : 1) ? S : (tps == 1 ? 2 : 1);   // the owner's slices from the start
    const bool share = p.wj && !p.out_probs && sizeof(TIn) == 4 && (((uintptr_t)rowp) & 15u) == 0 &&
                       V % IO::W == 0 && (p.B > NT || wide_rows_counted() < (uint32_t)p.B);
    if (SH && tid == 0) {
        int j = -1;
        if (share && p.B <= NT) {
            const int rk = wide_rank(r);
            j = rk < WJ_NJOB ? rk : -1;
        } else if (share) {
            WideJob* Jc = wj_job(p.wj, r % WJ_NJOB);
            if (atomicExch(&Jc->own, p.epoch) != p.epoch) j = r % WJ_NJOB;
        }
        w2_job = j;
    }
    int job = -1;   // (constant in the instance that shares nothing)
    if constexpr (SH) {
        __syncthreads();
        job = w2_job;
    }
    WideJob* J = job >= 0 ? wj_job(p.wj, job) : nullptr;
    // the word a pass of this workgroup's own reads after every tile
    uint32_t* own_word = wj_own_word(p, r);
    auto close_job = [&]() {   // no more slices; helpers leave the job
        if (job >= 0) {
            __syncthreads();
            if (tid == 0) {
                put_dev64(&J->tag, wj_tag(p.epoch, S, 3u));
                wj_bump(p.wj);
            }
            job = -1;
        }
    };

    // pass 1
    const int w = wv;
    uint32_t* wck = ck + w * FSEG;
    uint32_t* wci = ci + w * FSEG;
    uint32_t cw = 0;
    float fmx = -INFINITY, fmn = INFINITY;
    if (job >= 0) {   // pass 1 opens: its parameters, then the tag
        uint32_t* gb = wj_bins(J);
        for (int b = tid; b < 2048; b += NT) put_dev32(gb + b, 0u);
        if (tid == 0) {
            put_dev32(&J->tps, (uint32_t)tps);
            put_dev32(&J->q1, (uint32_t)f0); put_dev32(&J->done1, 0u);
            put_dev32((uint32_t*)&J->r, (uint32_t)r);
            put_dev32((uint32_t*)&J->h0, (uint32_t)h0); put_dev32((uint32_t*)&J->h1, (uint32_t)h1);
            put_devf(&J->T, T); put_devf(&J->pen, pen); put_devf(&J->yhi, yhi); put_devf(&J->ylo, ylo);
            put_devf(&J->scale, scale);
            put_dev32(&J->neg, neg ? 1u : 0u); put_dev32(&J->pen_on, pen_on ? 1u : 0u);
            put_dev32(&J->gmax, 0u); put_dev32(&J->gmin, 0xFFFFFFFFu);
            put_dev32(&J->ovf, 0u);
        }
        if (pen_on) {   // the history bitmap, which helpers read instead of the row's history
            uint32_t* gm = wj_bm(J);
            for (int wd = tid; wd < ((V + 31) >> 5); wd += NT) put_dev32(gm + wd, bm[wd]);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (tid == 0) {
            put_dev64(&J->tag, wj_tag(p.epoch, S, 1u));
            wj_bump(p.wj);
        }
    }
    int taken1 = S, taken2 = S;   // the owner's slices of each pass ([taken, S) the helpers')
    if constexpr (!SH) {
        NoClaims fc{S};
        w2_pass1<TIn>(rs, rowp, 0, V, bm, pen_on, pen, neg, yhi, ylo, scale, CH, wck, wci, cw, fmx, fmn, &w2_ovf,
                      &w2_dummy, fc, w2_go, true);
    } else for (bool fresh = true;; fresh = false) {   // (a second round only after a wait that timed out)
        FrontClaims fc = job >= 0 ? FrontClaims{&J->q1, S, tps, f0, f0} : FrontClaims{own_word, S, tps, S, S};
        w2_pass1<TIn>(rs, rowp, 0, V, bm, pen_on, pen, neg, yhi, ylo, scale, CH, wck, wci, cw, fmx, fmn, &w2_ovf,
                      &w2_dummy, fc, w2_go, fresh);
        taken1 = fc.taken;
        if (job < 0 || wj_wait(&J->done1, S - fc.taken)) break;
        // (never expected: then the pass again, here, with the helpers' parts ignored)
        close_job();
        for (int b = tid; b < 2048; b += NT) CH[b] = 0;
        if (tid == 0) w2_ovf = 0;
        __syncthreads();
        cw = 0;
        fmx = -INFINITY;
        fmn = INFINITY;
    }
    uint32_t omax, omin;
    if (fmx != fmx) {   // a NaN (both extremes carry it): keys that say so
        omax = 0xFFFFFFFFu;
        omin = 0u;
    } else {
        omax = neg ? selkey(fmn, true) : selkey(fmx, false);
        omin = neg ? selkey(fmx, true) : selkey(fmn, false);
    }
    {
        const uint32_t a0 = wave_max_u32(omax), a1 = wave_min_u32(omin);
        if (lane == 0) { w2_r[0][w] = a0; w2_r[1][w] = a1; w2_seg[w] = cw; }
    }
    __syncthreads();
    rd = Reduced{0u, 0xFFFFFFFFu, 0u};
    uint32_t ntop = 0, off = 0;
#pragma unroll
    for (int v = 0; v < NWAVES; ++v) {
        rd.max = w2_r[0][v] > rd.max ? w2_r[0][v] : rd.max;
        rd.min = w2_r[1][v] < rd.min ? w2_r[1][v] : rd.min;
        off += v < w ? w2_seg[v] : 0u;
        ntop += w2_seg[v];
    }
    // The helpers' slices [taken, S) of a list (0: top list, 1, 2: windows):
    // their counts and offsets in w2_sc, w2_so, the total in w2_tot (wave
    // 0, a lane per slice); a count above the slice's room is an overflow.
    auto slice_counts = [&](int list, int taken, uint32_t room) -> bool {
        if (w == 0) {
            const uint32_t c = lane < S && lane >= taken ? ld_dev(wj_cnt(J, list) + lane) : 0u;
            const uint32_t incl = wave_prefix_u32(c);
            if (lane < WJ_S) { w2_sc[lane] = c; w2_so[lane] = incl - c; }
            const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            const bool big = __ballot(c > room) != 0;
            if (lane == 0) w2_tot = big ? 0xFFFFFFFFu : tot;
        }
        __syncthreads();
        return w2_tot != 0xFFFFFFFFu;
    };
    // the helpers' part: extremes, bin counts, top-list entries
    uint32_t gtop = 0;
    bool govf = false;
    if (job >= 0) {
        const uint32_t gmx = ld_dev(&J->gmax), gmn = ld_dev(&J->gmin);
        rd.max = gmx > rd.max ? gmx : rd.max;
        rd.min = gmn < rd.min ? gmn : rd.min;
        govf = ld_dev(&J->ovf) != 0u;
        const uint32_t* gb = wj_bins(J);
        for (int b = tid; b < 2048; b += NT) CH[b] += ld_dev(gb + b);
        govf = !slice_counts(0, taken1, (uint32_t)WJ_TOPS) || govf;
        gtop = govf ? 0u : w2_tot;
    }
    // NaN keys lie above the key of +inf and below that of -inf
    const bool has_nan = rd.max > 0xFF800000u || rd.min < 0x007FFFFFu;
    const bool has_inf = rd.max >= 0xFF800000u || rd.min <= 0x007FFFFFu;
    if (has_nan || (has_inf && __builtin_isinf(T))) { close_job(); st = MXS_ROW_NONFINITE; tok = -1; return 1; }
    const float m = sel_inv(rd.max, neg) / T;
    if (!isfinite(m)) { close_job(); st = MXS_ROW_NONFINITE; tok = -1; return 1; }
    if (top_p < 1.0f && !(top_p > 0.0f)) { close_job(); st = MXS_ROW_EMPTY_NUCLEUS; tok = -1; return 1; }
    if (w2_ovf || govf || ntop + gtop > (uint32_t)TL_CAP) { close_job(); return 0; }
    // (pass 2's quotients by rT: exact in d = l - m for these m; see div_by_rT)
    if (m != 0.0f && __builtin_fabsf(m) < 0x1p-101f) { close_job(); return 0; }
    const double rT = 1.0 / (double)T;

    // the top list's keys and exact masses (the helpers' entries after the owner's)
    u64 part = 0;
    for (uint32_t j = (uint32_t)lane; j < cw; j += 64) {
        const float l = u2f(wck[j]) / T;
        TL[off + j] = ((u64)vkey(l) << 32) | (u64)(0xFFFFFFFFu - wci[j]);
        part += mass_of(l - m);
    }
    if (job >= 0) {
        for (int j = taken1 * WJ_TOPS + tid; j < S * WJ_TOPS; j += NT) {
            const int sl = j / WJ_TOPS, i = j % WJ_TOPS;
            if ((uint32_t)i < w2_sc[sl]) {
                const u64 e = ld_dev64(wj_top(J, sl) + i);
                const float l = u2f((uint32_t)(e >> 32)) / T;
                TL[ntop + w2_so[sl] + i] = ((u64)vkey(l) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)e);
                part += mass_of(l - m);
            }
        }
        ntop += gtop;
    }
    const u64 Wtop = block_sum<u64>(part);   // (its barriers publish TL and the counts)

    // bounds on each bin's mass (this thread's bins 2047 - 4 tid - i, in
    // descending order), padded for the polynomial's last-bit wiggles
    const float aT = __builtin_fabsf(T);
    auto mass_at = [&](float y) -> u64 { return mass_of(y / aT - m); };
    u64 mlo[4], mhi[4], slo = 0, shi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int b = 2047 - 4 * tid - i;
        const u64 c = (u64)CH[b];
        const float ye_lo = ylo + ((float)b - 0.01f) * dy;
        float ye_hi = ylo + ((float)b + 1.01f) * dy;
        ye_hi = b == 2047 || ye_hi > yhi ? yhi : ye_hi;
        u64 lo = b == 0 ? 0ull : mass_at(ye_lo);
        u64 hi = mass_at(ye_hi);
        lo = lo > (lo >> 20) + 1 ? lo - (lo >> 20) - 1 : 0ull;
        hi = hi + (hi >> 20) + 1;
        mlo[i] = c * lo;
        mhi[i] = c * hi;
        slo += mlo[i];
        shi += mhi[i];
    }
    u64 Blo, Bhi;
    const u64 prelo0 = block_incl_scan<u64>(slo, &Blo) - slo;   // the mass bounds above this thread's bins
    const u64 prehi0 = block_incl_scan<u64>(shi, &Bhi) - shi;
    const u64 Wlo = Wtop + Blo, Whi = Wtop + Bhi;
    // The bins that can hold a target position pos = q(W) + a (absolute;
    // positions below Wtop are in the top list), q monotone with q(X) <= X,
    // a in [a_lo, a_hi]: [lo, hi], or hi < lo for none.  For bin b with the
    // mass Pre above it, M in it and Suf below it (all in the bulk),
    // pos - (Wtop + Pre) = q(Wtop + Pre + M + Suf) - (Wtop + Pre) + a falls
    // as Pre grows and rises with M + Suf; with independent bounds on the
    // three this is bounded by evaluating q at Wtop + Blo + (Pre_hi - Pre_lo)
    // and at Wtop + Bhi - (Pre_hi - Pre_lo).  (For q near 1, as for a draw
    // deep in the tail, Pre's uncertainty hardly moves the position relative
    // to the bin.)
    auto window = [&](auto qx, long long a_lo, long long a_hi, int& lo, int& hi) {
        int bmax = -1, bmin = 2048;
        u64 pl = prelo0, ph = prehi0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int b = 2047 - 4 * tid - i;
            const u64 dp = ph - pl;
            const long long glo = (long long)qx(Wtop + Blo + dp) - (long long)(Wtop + ph) + a_lo;
            const long long ghi = (long long)qx(Wtop + Bhi - dp) + 1 - (long long)(Wtop + pl) + a_hi;
            if (mhi[i] > 0 && ghi >= 0 && glo < (long long)mhi[i]) {
                bmax = b > bmax ? b : bmax;
                bmin = b < bmin ? b : bmin;
            }
            pl += mlo[i];
            ph += mhi[i];
        }
        const Reduced rw = block_reduce((uint32_t)(bmax + 1), (uint32_t)bmin, 0u);
        hi = (int)rw.max - 1;
        lo = (int)rw.min;
    };
    const bool bounded = top_p < 1.0f;
    const float cu = clamp_uniform(u);
    int c_lo = 2048, c_hi = -1, d_lo = 2048, d_hi = -1;
    if (bounded) {
        // the cut: t = ceil(p W) - 1 in [floor(p W) - 1, floor(p W)]
        window([&](u64 X) { return floor_mul(top_p, X); }, -1, 0, c_lo, c_hi);
        const u64 tlo = ceil_mul(top_p, Wlo) - 1, thi = ceil_mul(top_p, Whi) - 1;
        if (thi >= Wtop) {
            // the draw D = floor(u Wk), Wk = t + 1 + (part of the cut
            // element's mass): at most wmax more than ceil(p W), wmax the
            // largest mass an element of the cut's window (or of the top
            // list, if the cut may lie there) can have
            u64 wmax;
            if (tlo < Wtop) {
                wmax = 1ull << 45;
            } else {
                const int bt = c_hi + 1 < 2047 ? c_hi + 1 : 2047;
                const float yt = bt == 2047 ? yhi : ylo + ((float)bt + 1.01f) * dy;
                const u64 mt = mass_at(yt < yhi ? yt : yhi);
                wmax = mt + (mt >> 20) + 1;
            }
            window([&](u64 X) { return floor_mul(cu, floor_mul(top_p, X)); }, -1, (long long)wmax + 2,
                   d_lo, d_hi);
        }
    } else {
        window([&](u64 X) { return floor_mul(cu, X); }, 0, 0, d_lo, d_hi);   // the draw D = floor(u W)
    }
    // The gathered ranges: one more bin on either side, as value thresholds
    // [ya, yb) (an element is above a window iff y >= yb, in it iff
    // ya <= y < yb; an empty window has ya = yb = yhi).  Pass 2 tests values
    // only: a threshold may fall a rounding away from its bin's edge, which
    // the spare bin on either side absorbs.
    auto edge = [&](int b) -> float { return b <= 0 ? -INFINITY : (b >= 2048 ? yhi : ylo + (float)b * dy); };
    const float yca = c_hi >= c_lo ? edge(c_lo - 1) : yhi, ycb = c_hi >= c_lo ? edge(c_hi + 2) : yhi;
    const float yda = d_hi >= d_lo ? edge(d_lo - 1) : yhi, ydb = d_hi >= d_lo ? edge(d_hi + 2) : yhi;

    // pass 2 (no branch per element: the rare window elements are marked,
    // and written at the tile's end by the waves that have any)
    u64 wb = 0, ac = 0, ad = 0;
    if (job >= 0 && tid == 0) {   // pass 2 opens
        put_dev32(&J->q2, (uint32_t)f0); put_dev32(&J->done2, 0u);
        put_devf(&J->m, m); put_devf(&J->yca, yca); put_devf(&J->ycb, ycb);
        put_devf(&J->yda, yda); put_devf(&J->ydb, ydb);
        __builtin_amdgcn_s_waitcnt(0);
        put_dev64(&J->tag, wj_tag(p.epoch, S, 2u));
        wj_bump(p.wj);
    }
    if constexpr (!SH) {
        NoClaims fc{S};
        w2_pass2<TIn>(rs, rowp, 0, V, bm, pen_on, pen, neg, T, rT, m, yhi, yca, ycb, yda, ydb, wb, ac, ad, w2_cnt, KC, KD,
                      fc, w2_go);
    } else for (;;) {   // (as for pass 1)
        FrontClaims fc = job >= 0 ? FrontClaims{&J->q2, S, tps, f0, f0} : FrontClaims{own_word, S, tps, S, S};
        w2_pass2<TIn>(rs, rowp, 0, V, bm, pen_on, pen, neg, T, rT, m, yhi, yca, ycb, yda, ydb, wb, ac, ad, w2_cnt, KC, KD,
                      fc, w2_go);
        taken2 = fc.taken;
        if (job < 0 || wj_wait(&J->done2, S - fc.taken)) break;
        close_job();
        if (tid == 0) { w2_cnt[0] = 0; w2_cnt[1] = 0; }
        __syncthreads();
        wb = 0; ac = 0; ad = 0;
    }
    {
        const u64 a0 = wave_sum_u64(wb), a1 = wave_sum_u64(ac), a2 = wave_sum_u64(ad);
        if (lane == 0) { w2_s[0][w] = a0; w2_s[1][w] = a1; w2_s[2][w] = a2; }
    }
    __syncthreads();
    u64 WB = 0, AC = 0, AD = 0;
#pragma unroll
    for (int v = 0; v < NWAVES; ++v) { WB += w2_s[0][v]; AC += w2_s[1][v]; AD += w2_s[2][v]; }
    uint32_t nc = w2_cnt[0], nd = w2_cnt[1];
    if (job >= 0) {   // the helpers' sums (a lane per slice) and window elements
        if (w == 0) {
            const bool hs = lane < S && lane >= taken2;
            const u64 sb = hs ? ld_dev64(wj_sums(J, lane)) : 0ull;
            const u64 sc = hs ? ld_dev64(wj_sums(J, lane) + WJ_S) : 0ull;
            const u64 sd = hs ? ld_dev64(wj_sums(J, lane) + 2 * WJ_S) : 0ull;
            const u64 a0 = wave_sum_u64(sb), a1 = wave_sum_u64(sc), a2 = wave_sum_u64(sd);
            if (lane == 0) { w2_hs[0] = a0; w2_hs[1] = a1; w2_hs[2] = a2; }
        }
        __syncthreads();
        WB += w2_hs[0];
        AC += w2_hs[1];
        AD += w2_hs[2];
        // the helpers' window elements after the owner's (a slice's count
        // above its room counts as more than LCAP: the general path)
        for (int list = 1; list <= 2; ++list) {
            uint32_t& n = list == 1 ? nc : nd;
            u64* K = list == 1 ? KC : KD;
            if (!slice_counts(list, taken2, (uint32_t)WJ_WINS)) {
                n = (uint32_t)LCAP + 1u;
                continue;
            }
            if (n + w2_tot <= (uint32_t)LCAP) {
                for (int j = taken2 * WJ_WINS + tid; j < S * WJ_WINS; j += NT) {
                    const int sl = j / WJ_WINS, i = j % WJ_WINS;
                    if ((uint32_t)i < w2_sc[sl])
                        K[n + w2_so[sl] + i] = ld_dev64((list == 1 ? wj_kc(J, sl) : wj_kd(J, sl)) + i);
                }
            }
            n += w2_tot;
            __syncthreads();   // (w2_sc, w2_so are read before the next list's counts)
        }
        close_job();   // (its barrier publishes the lists)
    }
    const u64 W = Wtop + WB;
    if (W < Wlo || W > Whi || nc > (uint32_t)LCAP || nd > (uint32_t)LCAP) return 0;

    // the cut and the draw (sampling.py:56-63, 69)
    u64* SMHp = SMH;
    uint32_t* SCH = CH;
    u64 Wk = W, cutkey = 0;
    if (bounded) {
        const u64 t = ceil_mul(top_p, W) - 1;
        SetPick c;
        if (t < Wtop) {
            c = pick_in_set(TL, (int)ntop, t, m, SMHp, SCH);
            Wk = c.E + c.w;
        } else {
            const u64 x = t - Wtop;
            if (x < AC || !(yca < ycb)) return 0;
            c = pick_in_set(KC, (int)nc, x - AC, m, SMHp, SCH);
            Wk = Wtop + AC + c.E + c.w;
        }
        if (!c.ok) return 0;
        cutkey = c.key;
    }
    const u64 D = floor_mul(cu, Wk);
    SetPick dp;
    if (D < Wtop) {
        dp = pick_in_set(TL, (int)ntop, D, m, SMHp, SCH);
    } else {
        const u64 x = D - Wtop;
        if (x < AD || !(yda < ydb)) return 0;
        dp = pick_in_set(KD, (int)nd, x - AD, m, SMHp, SCH);
    }
    if (!dp.ok) return 0;
    tok = (int64_t)(0xFFFFFFFFu - (uint32_t)dp.key);
    st = MXS_ROW_OK;
    if (p.out_probs) {   // sampling.py:68 (a third read, only when the probabilities are asked for)
        float* out = p.out_probs + (size_t)r * (size_t)V;
        rs.restart();
        rs.run_pen(bm, pen_on, pen,
            [&](int, int e, float x) {
                const float l = x / T;
                const u64 key = ((u64)vkey(l) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)e);
                if (!bounded || key >= cutkey) out[e] = (float)((double)mass_of(l - m) / (double)Wk);
            },
            [&](auto&&) { return false; });
    }
    return 1;
}

// A workgroup that has finished its own row takes slices of the shared
// rows' open passes from the back until none is left and no job is pending;
// while jobs are pending but no slice is open it waits (bounded; only when
// every row's workgroup was resident from the start, p.help).  Nothing is
// polled when the batch has no row with top-k off, or has only such rows
// (then no row shares).  Wave 0 reads every job's tag and claims at once
// (a lane per job), then claims a slice of the chosen pass and reads the
// job's parameters in the same round trip (a lane per word; they were
// written before the tag that opened the pass); a helper stays with its
// pass while it has slices (its next claim rides with the hand-over of the
// last slice).  Its LDS is free: the slice's words of the row's history
// bitmap are read from the job, and each slice's bins, top-list entries and
// window elements are counted here first, then handed over: bins and sums
// by device-scope atomics, entries and their counts into the slice's own
// places (no returning atomic).
template <typename TIn>
__device__ __forceinline__ void help_rows(const Params& p, unsigned char* smem)
{
    if constexpr (sizeof(TIn) != 4) {
        return;
    } else {
        constexpr int NPAR = 17;   // the parameter words: WideJob::r .. pen_on (16), then tps
        static_assert(offsetof(WideJob, pen_on) - offsetof(WideJob, r) == 4 * (NPAR - 2), "parameter words");
        __shared__ int hc_job, hc_phase, hc_slice, hc_S;
        __shared__ uint32_t hc_par[NPAR], hc_ovf, hc_dummy, hc_cnt[2], hc_seg[NWAVES];
        __shared__ u64 hc_s[3][NWAVES];
        if (p.B <= NT) {
            const uint32_t nw = wide_rows_counted();
            if (nw == 0u || nw >= (uint32_t)p.B) return;
        }
        const int tid = threadIdx.x, lane = lane_id(), w = wave_id();
        const int V = p.V;
        uint32_t* bm = (uint32_t*)(smem + KF_BM);
        uint32_t* CH = (uint32_t*)(smem + KF_H);
        uint32_t* ck = (uint32_t*)(smem + KF_CK);
        uint32_t* ci = (uint32_t*)(smem + KF_CI);
        u64* KC = (u64*)(smem + W2_KC);
        u64* KD = (u64*)(smem + W2_KD);
        RowStream<TIn> rs((const TIn*)p.logits, 0, false);
        int j = -1, phase = 0, s = -1, S = 0;   // the slice in hand (s >= 0)
        uint32_t seen = 0;                       // (wave 0) the version at the last scan
        bool rescan = true;                      // (wave 0) scan whatever the version
        u64 last_lm = 0;                         // (wave 0) the jobs pending at the last scan
        for (int idle = 0; idle < WJ_SPIN;) {
            if (s < 0) {
                if (w == 0) {
                    // the records' version: when it has not moved since the last
                    // scan that found nothing to take, wait (or leave) as then
                    uint32_t ver = 0;
                    if (lane == 0) ver = ld_dev(&wj_job(p.wj, 0)->ver);
                    ver = (uint32_t)__builtin_amdgcn_readfirstlane((int)ver);
                    const bool scan = rescan || ver != seen;
                    seen = ver;
                    // lane l: job l's tag and claims
                    u64 tg = 0, qq = 0;
                    if (scan && lane < WJ_NJOB) {
                        WideJob* Jl = wj_job(p.wj, lane);
                        tg = ld_dev64(&Jl->tag);
                        qq = ld_dev64((const u64*)&Jl->q1);
                    }
                    const uint32_t ph = (uint32_t)tg & 0xFFu, Sl = (uint32_t)(tg >> 8) & 0xFFu;
                    const bool live = lane < WJ_NJOB && (uint32_t)(tg >> 32) == p.epoch &&
                                      ((uint32_t)(tg >> 16) & 0xFFFFu) == WJ_MAGIC && (ph == 1u || ph == 2u);
                    const uint32_t q = ph == 1u ? (uint32_t)qq : (uint32_t)(qq >> 32);
                    const bool open = live && (q & 0xFFFFu) + (q >> 16) < Sl;
                    const u64 om = __ballot(open), lm = scan ? __ballot(live) : last_lm;
                    last_lm = lm;
                    rescan = false;
                    int cmd = -2, cph = 0, cs = -1, cS = 0;
                    if (om) {
                        // this workgroup's last job first, else open job number
                        // blockIdx mod (open jobs), so that the helpers spread evenly
                        int pick = (j >= 0 && ((om >> j) & 1u)) ? j : -1;
                        if (pick < 0) {
                            int nth = (int)(blockIdx.x % (unsigned)__builtin_popcountll(om));
                            u64 m = om;
                            for (; nth > 0; --nth) m &= m - 1ull;
                            pick = __builtin_ctzll(m);
                        }
                        cph = __builtin_amdgcn_readlane((int)ph, pick);
                        cS = __builtin_amdgcn_readlane((int)Sl, pick);
                        WideJob* Jp = wj_job(p.wj, pick);
                        // the claim (lane 0) and the parameters (a lane per word) together
                        uint32_t got = 0;
                        if (lane == 0) got = atomicAdd(cph == 1 ? &Jp->q1 : &Jp->q2, 1u << 16);
                        uint32_t pw = 0;
                        if (lane < NPAR)
                            pw = ld_dev(lane < NPAR - 1 ? (const uint32_t*)&Jp->r + lane : &Jp->tps);
                        if (lane < NPAR) hc_par[lane] = pw;
                        cs = (got & 0xFFFFu) + (got >> 16) < (uint32_t)cS ? cS - 1 - (int)(got >> 16) : -1;
                        cmd = pick;   // (a refused claim: scan again at once)
                        rescan = true;
                    } else if (lm && p.help) {
                        cmd = -1;     // jobs pending: wait
                    }
                    if (lane == 0) { hc_job = cmd; hc_phase = cph; hc_slice = cs; hc_S = cS; }
                }
                __syncthreads();
                const int cmd = hc_job;
                s = hc_slice;
                __syncthreads();
                if (cmd == -2) break;
                if (cmd == -1 || s < 0) {
                    if (cmd == -1) __builtin_amdgcn_s_sleep(8);   // (about 200 ns between polls)
                    ++idle;
                    s = -1;
                    continue;
                }
                j = cmd;
                phase = hc_phase;
                S = hc_S;
            }
            idle = 0;
            WideJob* J = wj_job(p.wj, j);
            const int r = (int)hc_par[0], h0 = (int)hc_par[1], h1 = (int)hc_par[2];
            const float T = u2f(hc_par[4]), pen = u2f(hc_par[5]), yhi = u2f(hc_par[6]);
            const bool neg = hc_par[14] != 0u, pen_on = hc_par[15] != 0u;
            const int tps = (int)hc_par[16];
            (void)h0;
            (void)h1;
            if ((unsigned)r >= (unsigned)p.B || tps < 1) {   // (not a record of this call: leave it)
                s = -1;
                j = -1;
                continue;
            }
            const TIn* rowp = (const TIn*)p.logits + (size_t)r * (size_t)p.ld;
            const int L = tps * FTILE;
            const int s0 = s * L < V ? s * L : V;
            const int n = (s0 + L < V ? s0 + L : V) - s0;
            if (pen_on) {   // the slice's words of the row's history bitmap (the owner wrote them)
                const int w0 = s0 >> 5, nw = (n + 31) >> 5;
                const uint32_t* gm = wj_bm(J);
                for (int i = tid; i < nw; i += NT) bm[w0 + i] = ld_dev(gm + w0 + i);
            }
            NoClaims mine{S};
            uint32_t* q;
            uint32_t* done;
            if (phase == 1) {
                const float ylo = u2f(hc_par[7]), scale = u2f(hc_par[8]);
                for (int b = tid; b < 2048; b += NT) CH[b] = 0;
                if (tid == 0) hc_ovf = 0;
                __syncthreads();
                uint32_t cw = 0;
                float fmx = -INFINITY, fmn = INFINITY;
                w2_pass1<TIn>(rs, rowp, s0, n, bm, pen_on, pen, neg, yhi, ylo, scale, CH, ck + w * FSEG,
                              ci + w * FSEG, cw, fmx, fmn, &hc_ovf, &hc_dummy, mine, hc_go_dummy(), false);
                uint32_t omax, omin;
                if (fmx != fmx) {
                    omax = 0xFFFFFFFFu;
                    omin = 0u;
                } else {
                    omax = neg ? selkey(fmn, true) : selkey(fmx, false);
                    omin = neg ? selkey(fmx, true) : selkey(fmn, false);
                }
                if (lane == 0) hc_seg[w] = cw;
                const Reduced rw = block_reduce(omax, omin, 0u);   // (its barriers publish CH, the segments, hc_seg)
                uint32_t* gb = wj_bins(J);
                for (int b = tid; b < 2048; b += NT) {
                    const uint32_t c = CH[b];
                    if (c) atomicAdd(gb + b, c);
                }
                // the slice's top-list entries, the waves' segments in order
                uint32_t base = 0, tot = 0;
#pragma unroll
                for (int v = 0; v < NWAVES; ++v) {
                    base += v < w ? hc_seg[v] : 0u;
                    tot += hc_seg[v];
                }
                u64* gt = wj_top(J, s);
                const uint32_t* wck = ck + w * FSEG;
                const uint32_t* wci = ci + w * FSEG;
                for (uint32_t i = (uint32_t)lane; i < cw; i += 64)
                    if (base + i < (uint32_t)WJ_TOPS) put_dev64(gt + base + i, ((u64)wck[i] << 32) | wci[i]);
                if (tid == 0) {
                    atomicMax(&J->gmax, rw.max);
                    atomicMin(&J->gmin, rw.min);
                    if (hc_ovf) put_dev32(&J->ovf, 1u);
                    put_dev32(wj_cnt(J, 0) + s, tot);   // (above WJ_TOPS: the owner takes the general path)
                }
                q = &J->q1;
                done = &J->done1;
            } else {
                const float m = u2f(hc_par[9]), yca = u2f(hc_par[10]), ycb = u2f(hc_par[11]);
                const float yda = u2f(hc_par[12]), ydb = u2f(hc_par[13]);
                if (tid == 0) { hc_cnt[0] = 0; hc_cnt[1] = 0; }
                __syncthreads();
                u64 wb = 0, ac = 0, ad = 0;
                w2_pass2<TIn>(rs, rowp, s0, n, bm, pen_on, pen, neg, T, 1.0 / (double)T, m, yhi, yca, ycb, yda, ydb, wb, ac, ad, hc_cnt,
                              KC, KD, mine, hc_go_dummy());
                const u64 a0 = wave_sum_u64(wb), a1 = wave_sum_u64(ac), a2 = wave_sum_u64(ad);
                if (lane == 0) { hc_s[0][w] = a0; hc_s[1][w] = a1; hc_s[2][w] = a2; }
                __syncthreads();   // (the lists and the waves' sums are complete)
                const uint32_t nc = hc_cnt[0], nd = hc_cnt[1];
                u64 *gkc = wj_kc(J, s), *gkd = wj_kd(J, s);
                for (uint32_t i = (uint32_t)tid; i < nc && i < (uint32_t)WJ_WINS; i += NT) put_dev64(gkc + i, KC[i]);
                for (uint32_t i = (uint32_t)tid; i < nd && i < (uint32_t)WJ_WINS; i += NT) put_dev64(gkd + i, KD[i]);
                if (tid == 0) {   // (above WJ_WINS: the owner takes the general path)
                    put_dev32(wj_cnt(J, 1) + s, nc);
                    put_dev32(wj_cnt(J, 2) + s, nd);
                    u64 tb = 0, tc = 0, td = 0;
#pragma unroll
                    for (int v = 0; v < NWAVES; ++v) { tb += hc_s[0][v]; tc += hc_s[1][v]; td += hc_s[2][v]; }
                    put_dev64(wj_sums(J, s), tb);
                    put_dev64(wj_sums(J, s) + WJ_S, tc);
                    put_dev64(wj_sums(J, s) + 2 * WJ_S, td);
                }
                q = &J->q2;
                done = &J->done2;
            }
            // the next slice of this pass, claimed while the results are acknowledged
            if (tid == 0) hc_slice = wj_claim_back(q, S);
            wj_done(done);
            __syncthreads();
            s = hc_slice;
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------- fp16 rows, top-k off
//
// An fp16 logit is one of 65536 values, and for 2^-100 < |T| < 2^100 its
// tempered value fl32(x / T) is a strictly monotone function of them:
// neighbouring fp16 values differ by at least 2^-11 relative, far more than
// the fp32 rounding of the quotient moves them, and no quotient leaves the
// normal range.  -0 and +0 are the one pair with equal values.  So the
// sorted order of sampling.py:56-57 (value desc, index asc) is the order of
// the values' ranks R = 0, 1, ..., the elements of one rank in index order,
// and one pass that counts each rank's elements (16-bit counters, two per
// LDS word) gives every prefix mass: each rank's mass is its count times one
// mass_of, computed once per value present.  The top-p cut and the draw
// search the ranks' masses in chunks of 128 ranks; the only other pass over
// the row marks the elements of the drawn rank to find the one at the drawn
// position in index order.
//
// The penalized history ids (at most HCAP) leave their raw ranks and are
// placed by their penalized values: an id whose value equals rank R's joins
// R's tie group (same mass, index order), one strictly between the values of
// R and R + 1 follows R's group.  Each thread keeps up to HQ of them in
// registers.
//
// The counts overwrite the history bitmap and list, which are rebuilt when
// a row falls back to the general path: a rank holding 65536 or more
// elements, or a draw or cut among more than GCAP history values that lie
// between the same two ranks.
//
// Ranks: R = h ^ KP for an fp16 pattern h >= 0, h ^ KN for h < 0, with
// (KP, KN) = (0x7FFF, 0) for T > 0 and (0x8000, 0xFFFF) for T < 0.  R < 0x3FF
// and R > 0xFC00 are NaN patterns, 0x3FF holds the value +inf and 0xFC00 the
// value -inf; ranks 0x7FFF and 0x8000 both hold 0 and the counts of 0x8000
// move to 0x7FFF after the pass.
constexpr int RCH = 256;                    // ranks per chunk: four per lane of a wave
constexpr int NCH = 65536 / RCH;            // chunks
constexpr int KC_CS = 131072;               // NCH x u64: mass of each chunk
constexpr int KC_HS = KC_CS + 8 * NCH;      // NCH x u64: penalized history mass placed in each chunk
constexpr int KC_G = KC_HS + 8 * NCH;       // history values between two ranks: values, ids, masses
constexpr int GCAP = 256;
constexpr int KC_PM = KC_G + 16 * GCAP;     // RCH x u64: history mass placed at each rank of one chunk
constexpr int KC_PN = KC_PM + 8 * RCH;      // RCH x u32: history values tied with each rank of one chunk
constexpr int HQ = 4;
constexpr uint32_t RK_PINF = 0x3FFu, RK_NINF = 0xFC00u, RK_ZERO = 0x7FFFu;
constexpr int FC_MIN_V = 32768;             // shorter rows take the general path
static_assert(KC_PN + 4 * RCH <= KF_LDS_BYTES, "chunk history arrays");
static_assert(HCAP <= HQ * NT, "history ids held in registers");
static_assert(RCH == 256 && NCH <= NT, "chunk layout");
static_assert(MXS_MAX_VOCAB / 8 <= 32768, "two index bitmaps in the counts' area");

// An element at a mass position of the sorted order.
struct CPick {
    u64 E;          // mass before it
    u64 w;          // its mass
    u64 i;          // a raw element: its position among rank R's tie group, in index order
    uint32_t R;     // its rank (a history element: the rank it follows or ties)
    uint32_t id;    // a history element: its id; else 0xFFFFFFFF
    float l;        // its tempered value
    uint32_t ok;
};

// a / b for a < 2^62 and 0 < b (a double estimate, corrected)
__device__ __forceinline__ u64 udiv_est(u64 a, u64 b)
{
    u64 q = (u64)((double)a / (double)b);
    while (q > 0 && q * b > a) --q;
    while ((q + 1) * b <= a) ++q;
    return q;
}

// Returns false (history bitmap and list restored, rs restarted) when the
// row must take the general path.
__device__ __forceinline__ bool finish_counts(const Params& p, int r, RowStream<__half>& rs, float T, bool neg,
                                              float top_p, float u, float pen, bool pen_on, uint32_t* bm,
                                              uint32_t* hl, uint32_t nh, unsigned char* smem,
                                              int64_t& tok, int32_t& st)
{
    __shared__ uint32_t s_csum, s_flag, s_ng, s_own, s_rtop, s_nb, s_bR, s_bflag;
    __shared__ float s_bl;
    __shared__ u64 s_ownE, s_btb;
    __shared__ CPick s_pick;
    const int tid = threadIdx.x, lane = lane_id();
    const int V = p.V;
    const __half* rowp = (const __half*)p.logits + (size_t)r * (size_t)p.ld;
    uint32_t* cnt = (uint32_t*)smem;
    u64* CS = (u64*)(smem + KC_CS);
    u64* HS = (u64*)(smem + KC_HS);
    float* GL = (float*)(smem + KC_G);
    uint32_t* GI = (uint32_t*)(smem + KC_G + 4 * GCAP);
    u64* GW = (u64*)(smem + KC_G + 8 * GCAP);
    u64* PM = (u64*)(smem + KC_PM);
    uint32_t* PN = (uint32_t*)(smem + KC_PN);
    const uint32_t KP = neg ? 0x8000u : 0x7FFFu, KN = neg ? 0xFFFFu : 0u;
    const uint32_t KPAIR = KP * 0x10001u;
    const uint32_t XA = neg ? 0xFFFFu : 0x7FFFu, XB = neg ? 0x8000u : 0u;   // inverse: h = R ^ (R < 0x8000 ? XA : XB)
    constexpr uint32_t OVF = 1u, NANB = 2u;
    auto rank_of = [&](uint32_t h) { return h ^ ((h & 0x8000u) ? KN : KP); };
    auto count_of = [&](uint32_t R) { return (cnt[R >> 1] >> ((R & 1u) << 4)) & 0xFFFFu; };
    auto inc_of = [](uint32_t R) { return 1u + (R & 1u) * 0xFFFFu; };
    auto val_fin = [&](uint32_t R) { return VecIO<__half>::h2f(R ^ (R < 0x8000u ? XA : XB)) / T; };
    auto val_of = [&](uint32_t R) -> float {   // monotone over all ranks (NaN ranks: +-inf)
        const float v = val_fin(R);
        return R < RK_PINF ? INFINITY : (R > RK_NINF ? -INFINITY : v);
    };

    // the history ids, HQ per thread, and their raw values
    int hid[HQ];
    float hx[HQ];
#pragma unroll
    for (int q = 0; q < HQ; ++q) {
        const uint32_t i = (uint32_t)(tid + q * NT);
        hid[q] = (pen_on && i < nh) ? (int)hl[i] : -1;
    }
#pragma unroll
    for (int q = 0; q < HQ; ++q) hx[q] = VecIO<__half>::one(rowp, hid[q] >= 0 ? hid[q] : 0);
    const uint32_t nhe = pen_on ? nh : 0u;
    auto restore = [&]() {   // the general path's history bitmap and list
        __syncthreads();
        if (pen_on) {
            const int words = (V + 31) >> 5;
            for (int w = tid; w < words; w += NT) bm[w] = 0;
            __syncthreads();
#pragma unroll
            for (int q = 0; q < HQ; ++q)
                if (hid[q] >= 0) {
                    atomicOr(&bm[hid[q] >> 5], 1u << (hid[q] & 31));
                    hl[tid + q * NT] = (uint32_t)hid[q];
                }
        }
        __syncthreads();
        rs.restart();
    };
    __syncthreads();   // (the list lies in the counts' area)
    {
        uint4* c4 = (uint4*)smem;
#pragma unroll
        for (int i = 0; i < KC_CS / 16 / NT; ++i) c4[tid + i * NT] = uint4{0u, 0u, 0u, 0u};
        if (tid < NCH) { HS[tid] = 0; CS[tid] = 0; }
        if (tid == 0) { s_csum = 0; s_flag = 0; s_ng = 0; s_own = 0xFFFFFFFFu; }
    }
    __syncthreads();

    // sampling.py:56: the row's values, counted by rank
    auto ranks2 = [&](uint32_t wd) {   // the ranks of a word's two values, in its two halves
        const uint32_t s = (wd >> 15) & 0x00010001u;
        return wd ^ (((s << 15) - s) ^ KPAIR);
    };
    uint32_t rmin = 0xFFFFu;
    rs.run_raw(
        [&](const RowStream<__half>::vec_t& v, int) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t Rp = ranks2(v[k]);
                const uint32_t r0 = Rp & 0xFFFFu, r1 = Rp >> 16;
                rmin = min(rmin, min(r0, r1));
                atomicAdd(&cnt[r0 >> 1], inc_of(r0));
                atomicAdd(&cnt[r1 >> 1], inc_of(r1));
            }
        },
        [&](uint32_t h, int) {
            const uint32_t R = rank_of(h);
            rmin = R < rmin ? R : rmin;
            atomicAdd(&cnt[R >> 1], inc_of(R));
        });
    // the history ids leave their raw ranks (sampling.py:38-45 penalizes them)
    uint32_t hraw[HQ], hR[HQ];
    float hv[HQ];
    uint32_t hkey = 0, hnan = 0;
#pragma unroll
    for (int q = 0; q < HQ; ++q) {
        hraw[q] = rank_of((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hx[q]));
        hv[q] = penalize(hx[q], pen) / T;
        if (hid[q] >= 0) {
            atomicSub(&cnt[hraw[q] >> 1], inc_of(hraw[q]));
            if (hv[q] != hv[q]) hnan = 1u;
            else hkey = max(hkey, okey(hv[q]) + 1u);   // 0: none
        }
    }
    const Reduced rd = block_reduce(hkey, rmin, hnan);   // (its barriers publish the counts)
    if (tid == 0) {   // -0 joins +0
        const uint32_t z = cnt[0x8000u >> 1] & 0xFFFFu;
        const uint32_t t0 = (cnt[RK_ZERO >> 1] >> 16) + z;
        if (t0 > 0xFFFFu) s_flag = OVF;
        cnt[RK_ZERO >> 1] = (cnt[RK_ZERO >> 1] & 0xFFFFu) | (t0 << 16);
        cnt[0x8000u >> 1] &= 0xFFFF0000u;
    }
    // a NaN, or +inf at the top (sampling.py:57-58)
    if (rd.any || rd.min <= RK_PINF) { st = MXS_ROW_NONFINITE; tok = -1; return true; }
    __syncthreads();
    // the row's maximum: the first rank still holding elements, or a history value
    uint32_t rtop = rd.min == 0x8000u ? RK_ZERO : rd.min;
    if (count_of(rtop) == 0u) {
        if (wave_id() == 0) {
            uint32_t found = 0xFFFFFFFFu;
            for (uint32_t base = (rtop + 1u) & ~127u; base < 65536u && found == 0xFFFFFFFFu; base += 128u) {
                const uint32_t R0 = base + 2u * (uint32_t)lane;
                const uint32_t wd = cnt[R0 >> 1];
                const uint32_t c0 = R0 > rtop ? (wd & 0xFFFFu) : 0u, c1 = R0 + 1u > rtop ? (wd >> 16) : 0u;
                const u64 m0 = __ballot(c0 != 0u), m1 = __ballot(c1 != 0u);
                if (m0 | m1) {
                    const int l0 = m0 ? __builtin_ctzll(m0) : 64, l1 = m1 ? __builtin_ctzll(m1) : 64;
                    found = l0 <= l1 ? base + 2u * (uint32_t)l0 : base + 2u * (uint32_t)l1 + 1u;
                }
            }
            if (lane == 0) s_rtop = found;
        }
        __syncthreads();
        rtop = s_rtop;
    }
    float m = rtop != 0xFFFFFFFFu ? val_of(rtop) : -INFINITY;
    if (rd.max) {
        const float mh = okey_inv(rd.max - 1u);
        m = mh > m ? mh : m;
    }
    if (!__builtin_isfinite(m)) { st = MXS_ROW_NONFINITE; tok = -1; return true; }
    // (the chunk masses take their quotients by rT: exact in d = l - m for
    // these m, see div_by_rT)
    if (m != 0.0f && __builtin_fabsf(m) < 0x1p-101f) { restore(); return false; }
    const double rT = 1.0 / (double)T;
    auto val_q = [&](uint32_t R) { return div_by_rT(VecIO<__half>::h2f(R ^ (R < 0x8000u ? XA : XB)), rT); };

    // each history value's place: the last rank whose value is >= it, from
    // the rank of fp16(l * T) (the place itself or a neighbour)
    {
        float va[HQ], vb[HQ], vc[HQ];   // the values of ranks R - 1, R, R + 1
#pragma unroll
        for (int q = 0; q < HQ; ++q) {
            uint32_t R = rank_of((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(hv[q] * T)));
            R = R < 1u ? 1u : (R > 0xFFFEu ? 0xFFFEu : R);
            hR[q] = R;
            va[q] = val_of(R - 1u);
            vb[q] = val_of(R);
            vc[q] = val_of(R + 1u);
        }
#pragma unroll
        for (int q = 0; q < HQ; ++q) {
            uint32_t R = hR[q];
            const float l = hv[q];
            if (vb[q] >= l && !(vc[q] >= l)) {
            } else if (va[q] >= l && !(vb[q] >= l)) {
                R -= 1u;
            } else if (hid[q] >= 0) {
                while (R > 0u && val_of(R) < l) --R;
                while (R < 0xFFFFu && val_of(R + 1u) >= l) ++R;
            }
            hR[q] = R == 0x8000u ? RK_ZERO : R;
        }
    }

    // sampling.py:57-58: the masses, per chunk of RCH ranks (chunks dealt
    // round-robin to the waves; a wave skips a chunk with no elements)
    {
        uint32_t csum = 0, nanb = 0;
        static_assert(NCH % (2 * NWAVES) == 0, "chunk pairs");
        for (int c2 = wave_id(); c2 < NCH; c2 += 2 * NWAVES) {
            uint2 wq[2];   // (both chunks' counts requested together)
#pragma unroll
            for (int q = 0; q < 2; ++q) wq[q] = *(const uint2*)&cnt[(RCH / 2) * (c2 + q * NWAVES) + 2 * lane];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int c = c2 + q * NWAVES;
                const uint2 wd = wq[q];
                if (__ballot((wd.x | wd.y) != 0u)) {
                    const uint32_t R0 = (uint32_t)(RCH * c) + 4u * (uint32_t)lane;
                    const uint32_t k0 = wd.x & 0xFFFFu, k1 = wd.x >> 16, k2 = wd.y & 0xFFFFu, k3 = wd.y >> 16;
                    u64 acc = count_mass(k0, val_q(R0) - m) + count_mass(k1, val_q(R0 + 1u) - m) +
                              count_mass(k2, val_q(R0 + 2u) - m) + count_mass(k3, val_q(R0 + 3u) - m);
                    csum += k0 + k1 + k2 + k3;
                    // (RK_NINF is a multiple of 4: the ranks above it are NaN values)
                    nanb |= R0 > RK_NINF ? (wd.x | wd.y) : (R0 == RK_NINF ? (k1 | wd.y) : 0u);
                    // the sums of the wave's four rows of 16 lanes (every sum
                    // of masses is below 2^63), added into the chunk's total
#pragma unroll
                    for (int step = 0; step < 4; ++step) acc += dpp_step(acc, 0ull, step);
                    if ((lane & 15) == 15) atomicAdd((unsigned long long*)&CS[c], (unsigned long long)acc);
                }
            }
        }
        csum = wave_sum_u32(csum);
        if (lane == 0) atomicAdd(&s_csum, csum);
        if (__ballot(nanb != 0u) && lane == 0) atomicOr(&s_flag, NANB);
#pragma unroll
        for (int q = 0; q < HQ; ++q)
            if (hid[q] >= 0) atomicAdd(&HS[hR[q] / RCH], mass_of(hv[q] - m));
    }
    __syncthreads();
    if (s_csum != (uint32_t)V - nhe || (s_flag & OVF)) { restore(); return false; }
    if (s_flag & NANB) { st = MXS_ROW_NONFINITE; tok = -1; return true; }
    const u64 S = tid < NCH ? CS[tid] + HS[tid] : 0ull;
    u64 W;
    const u64 E0 = block_incl_scan<u64>(S, &W) - S;

    // The element at mass position t < W: the chunk holding t; its ranks'
    // masses (count x mass, and the penalized history placed there, added
    // per rank with LDS atomics) in wave 0; if t falls on history values
    // between two ranks, those values ranked among themselves.
    auto pick = [&](u64 t) -> CPick {
        if (tid < RCH) { PM[tid] = 0; PN[tid] = 0; }
        if (E0 <= t && t - E0 < S) { s_own = (uint32_t)tid; s_ownE = E0; }
        if (tid == 0) { s_ng = 0; s_pick.ok = 0; s_bflag = 0; }
        __syncthreads();
        const uint32_t c = s_own;
        const u64 Ec = s_ownE;
#pragma unroll
        for (int q = 0; q < HQ; ++q)
            if (hid[q] >= 0 && hR[q] / RCH == c) {
                const uint32_t o = hR[q] % RCH;
                atomicAdd(&PM[o], mass_of(hv[q] - m));
                if (hv[q] == val_of(hR[q])) atomicAdd(&PN[o], 1u);
            }
        __syncthreads();
        if (tid == 0) s_own = 0xFFFFFFFFu;
        if (c < (uint32_t)NCH && wave_id() == 0) {
            const u64 tr = t - Ec;
            const uint32_t R0 = (uint32_t)RCH * c + 4u * (uint32_t)lane;
            const uint2 wd = *(const uint2*)&cnt[R0 >> 1];
            const uint32_t kc[4] = {wd.x & 0xFFFFu, wd.x >> 16, wd.y & 0xFFFFu, wd.y >> 16};
            uint32_t n[4];   // tie groups
            float lv[4];
            u64 wv[4], M[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lv[j] = val_of(R0 + (uint32_t)j);
                wv[j] = mass_of(lv[j] - m);
                n[j] = kc[j] + PN[4 * lane + j];
                M[j] = (u64)kc[j] * wv[j] + PM[4 * lane + j];
            }
            const u64 tot = M[0] + M[1] + M[2] + M[3];
            const u64 incl = wave_prefix_u64(tot);
            const u64 P = incl - tot;
            const bool here = P <= tr && tr < incl;
            if (here) {
                u64 t2 = tr - P;
                uint32_t R = R0 + 3u;
                float lR = lv[3];
                u64 wR = wv[3];
                uint32_t nR = n[3];
                bool found = false;
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    if (!found && t2 < M[j]) { found = true; R = R0 + (uint32_t)j; lR = lv[j]; wR = wv[j]; nR = n[j]; }
                    if (!found) t2 -= M[j];
                }
                const u64 tie = (u64)nR * wR;
                if (t2 < tie) {
                    const u64 i = udiv_est(t2, wR);
                    s_pick = CPick{t - (t2 - i * wR), wR, i, R, 0xFFFFFFFFu, lR, 1u};
                } else {   // a penalized history value strictly between ranks R and R + 1
                    s_bR = R; s_bl = lR; s_btb = t2 - tie; s_bflag = 1u;
                }
            }
        }
        __syncthreads();
        if (s_bflag) {
            // those placed after rank Rs, in order of (value desc, index asc)
            const uint32_t Rs = s_bR;
            const float ls = s_bl;
            const u64 tb = s_btb;
#pragma unroll
            for (int q = 0; q < HQ; ++q)
                if (hid[q] >= 0 && hR[q] == Rs && hv[q] < ls) {
                    const uint32_t g = atomicAdd(&s_ng, 1u);
                    if (g < (uint32_t)GCAP) { GL[g] = hv[q]; GI[g] = (uint32_t)hid[q]; GW[g] = mass_of(hv[q] - m); }
                }
            __syncthreads();
            const uint32_t ng = s_ng;
            if (ng <= (uint32_t)GCAP && wave_id() == 0) {
                auto key_at = [&](uint32_t g) { return ((u64)vkey(GL[g]) << 32) | (u64)(0xFFFFFFFFu - GI[g]); };
                for (uint32_t g0 = 0; g0 < ng; g0 += 64u) {
                    const uint32_t g = g0 + (uint32_t)lane;
                    const bool cand = g < ng;
                    const u64 key = cand ? key_at(g) : 0ull, wg = cand ? GW[g] : 0ull;
                    u64 Eh = 0;   // the mass of those ranked before it
                    for (uint32_t g1 = 0; g1 < ng; g1 += 64u) {
                        const uint32_t g2 = g1 + (uint32_t)lane;
                        const bool in2 = g2 < ng;
                        const u64 k2 = in2 ? key_at(g2) : 0ull, w2 = in2 ? GW[g2] : 0ull;
                        for (u64 msk = __ballot(in2); msk; msk &= msk - 1ull) {
                            const int b = __builtin_ctzll(msk);
                            Eh += readlane64(k2, b) > key ? readlane64(w2, b) : 0ull;
                        }
                    }
                    if (cand && Eh <= tb && tb - Eh < wg) s_pick = CPick{t - tb + Eh, wg, 0ull, Rs, GI[g], GL[g], 1u};
                }
            }
            __syncthreads();
        }
        const CPick res = s_pick;
        __syncthreads();
        return res;
    };

    bool bounded = false;
    CPick cut{0, 0, 0, 0, 0xFFFFFFFFu, 0.0f, 1u};
    u64 Wk = W;
    if (top_p < 1.0f) {   // sampling.py:56-63
        if (!(top_p > 0.0f)) { st = MXS_ROW_EMPTY_NUCLEUS; tok = -1; return true; }
        cut = pick(ceil_mul(top_p, W) - 1);
        if (!cut.ok) { restore(); return false; }
        bounded = true;
        Wk = cut.E + cut.w;
    }
    const u64 D = floor_mul(clamp_uniform(u), Wk);   // sampling.py:69
    const CPick dp = pick(D);
    if (!dp.ok) { restore(); return false; }

    // the index of a raw element: the i-th marked one of its rank
    uint32_t tid_d = dp.id, tid_c = cut.id;
    const bool need_d = dp.id == 0xFFFFFFFFu;
    const bool need_c = p.out_probs && bounded && cut.id == 0xFFFFFFFFu;
    if (need_d || need_c) {
        rs.restart();
        uint32_t* Bd = (uint32_t*)smem;
        uint32_t* Bc = (uint32_t*)(smem + 32768);
        const int words = (V + 31) >> 5;
        for (int w = tid; w < words; w += NT) { Bd[w] = 0; Bc[w] = 0; }
        __syncthreads();
        const uint32_t Rd = need_d ? dp.R : 0xFFFFFFFFu, Rc = need_c ? cut.R : 0xFFFFFFFFu;
        const uint32_t zd = Rd == RK_ZERO ? 1u : 0u, zc = Rc == RK_ZERO ? 1u : 0u;   // (rank 0x8000 is 0 too)
        // A group's raw fp16 patterns, in both halves of P: its value's, or
        // +0 and -0 for rank RK_ZERO (M masks the sign off); for a group not
        // looked for, a NaN pattern, which no row that gets here holds.
        auto pattern = [&](bool need, uint32_t R, uint32_t& P, uint32_t& M) {
            P = !need ? 0x7E007E00u : (R == RK_ZERO ? 0u : (R ^ (R < 0x8000u ? XA : XB)) * 0x10001u);
            M = need && R == RK_ZERO ? 0x7FFF7FFFu : 0xFFFFFFFFu;
        };
        uint32_t Pd, Md, Pc, Mc;
        pattern(need_d, Rd, Pd, Md);
        pattern(need_c, Rc, Pc, Mc);
        // The elements of a vector that match, a bit each (bits 2k and
        // 2k + 1: the halves of word k).  Almost no vector holds one, which
        // a test for a zero half in the four words shows first.
        auto match8 = [](const RowStream<__half>::vec_t& v, uint32_t P, uint32_t M) -> uint32_t {
            uint32_t x[4], z = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                x[k] = (v[k] ^ P) & M;
                z |= (x[k] - 0x00010001u) & ~x[k];
            }
            uint32_t b = 0;
            if (z & 0x80008000u) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    b |= ((x[k] & 0xFFFFu) == 0u ? 1u : 0u) << (2 * k) | ((x[k] >> 16) == 0u ? 2u : 0u) << (2 * k);
            }
            return b;
        };
        // the bits of a vector's eight elements, one LDS atomic per bitmap
        // when any is set (elements e .. e + 7 share one bitmap word)
        auto marks = [&](auto both) {
            rs.run_raw(
                [&](const RowStream<__half>::vec_t& v, int e) {
                    const uint32_t md = match8(v, Pd, Md);
                    const uint32_t mc = decltype(both)::value ? match8(v, Pc, Mc) : 0u;
                    if (md) atomicOr(&Bd[e >> 5], md << (e & 31));
                    if (mc) atomicOr(&Bc[e >> 5], mc << (e & 31));
                },
                [&](uint32_t h, int e) {
                    const uint32_t R = rank_of(h);
                    if (R - Rd <= zd) atomicOr(&Bd[e >> 5], 1u << (e & 31));
                    if (R - Rc <= zc) atomicOr(&Bc[e >> 5], 1u << (e & 31));
                });
        };
        if (need_c) marks(std::true_type{});
        else marks(std::false_type{});
        __syncthreads();
#pragma unroll
        for (int q = 0; q < HQ; ++q)   // history ids are not in their raw ranks' groups ...
            if (hid[q] >= 0) {
                const uint32_t bit = 1u << (hid[q] & 31);
                if (hraw[q] - Rd <= zd) atomicAnd(&Bd[hid[q] >> 5], ~bit);
                if (hraw[q] - Rc <= zc) atomicAnd(&Bc[hid[q] >> 5], ~bit);
            }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < HQ; ++q)   // ... but in the group whose value they equal
            if (hid[q] >= 0) {
                const uint32_t bit = 1u << (hid[q] & 31);
                if (hR[q] == Rd && hv[q] == dp.l) atomicOr(&Bd[hid[q] >> 5], bit);
                if (hR[q] == Rc && hv[q] == cut.l) atomicOr(&Bc[hid[q] >> 5], bit);
            }
        __syncthreads();
        auto nth_bit = [&](const uint32_t* B, u64 i) -> uint32_t {
            const int per = (words + NT - 1) / NT;
            const int w0 = tid * per;
            uint32_t c = 0;
            for (int k = 0; k < per; ++k)
                if (w0 + k < words) c += (uint32_t)__builtin_popcount(B[w0 + k]);
            if (tid == 0) s_nb = 0xFFFFFFFFu;
            uint32_t tot;
            const uint32_t incl = block_incl_scan<uint32_t>(c, &tot);
            u64 before = incl - c;
            if (before <= i && i < (u64)incl) {
                for (int k = 0; k < per; ++k) {
                    uint32_t b = B[w0 + k];
                    const uint32_t pc = (uint32_t)__builtin_popcount(b);
                    if (i < before + pc) {
                        for (u64 j = before; j < i; ++j) b &= b - 1u;
                        s_nb = (uint32_t)(32 * (w0 + k) + __builtin_ctz(b));
                        break;
                    }
                    before += pc;
                }
            }
            __syncthreads();
            const uint32_t res = s_nb;
            __syncthreads();
            return res;
        };
        if (need_d) tid_d = nth_bit(Bd, dp.i);
        if (need_c) tid_c = nth_bit(Bc, cut.i);
        if (tid_d >= (uint32_t)V || (need_c && tid_c >= (uint32_t)V)) { restore(); return false; }
    }
    tok = (int64_t)tid_d;
    st = MXS_ROW_OK;
    if (p.out_probs) {   // sampling.py:68
        __syncthreads();
        if (pen_on) {   // the history bitmap again (its area held the counts)
            const int words = (V + 31) >> 5;
            for (int w = tid; w < words; w += NT) bm[w] = 0;
            __syncthreads();
#pragma unroll
            for (int q = 0; q < HQ; ++q)
                if (hid[q] >= 0) atomicOr(&bm[hid[q] >> 5], 1u << (hid[q] & 31));
            __syncthreads();
        }
        const u64 bound = ((u64)vkey(cut.l) << 32) | (u64)(0xFFFFFFFFu - tid_c);
        float* out = p.out_probs + (size_t)r * (size_t)V;
        stream_row_pen<__half>(rowp, V, bm, pen_on, pen,
            [&](int, int e, float x) {
                const float l = x / T;
                const u64 key = ((u64)vkey(l) << 32) | (u64)(0xFFFFFFFFu - (uint32_t)e);
                if (!bounded || key >= bound) out[e] = (float)((double)mass_of(l - m) / (double)Wk);
            },
            [&](auto&&) { return false; });
    }
    return true;
}

// sampling.py:52-54, step 1 of the top-k path: a conservative estimate est of
// the row's k-th largest selection key from its NSAMP-logit sample (this
// thread's NS logits sx, the first at index se0): the lower edge of the
// histogram bin holding the sample's j-th largest, j well above the expected
// k * NSAMP / V; and theta = widen(est).  It only steers the stream; the
// count pass checks it.  hist (2048) must be zero; s_cs (64) receives the
// sums of its groups of 32 bins; called by the whole workgroup.
__device__ __forceinline__ void sample_bound(const float (&sx)[NSAMP / NT], int se0, uint32_t kk, int V, float T,
                                             bool neg, bool pen_inline, float pen, const uint32_t* bm,
                                             uint32_t* hist, uint32_t* s_cs, uint32_t& est, uint32_t& theta)
{
    constexpr int NS = NSAMP / NT;
    uint32_t sk4[NS], smax = 0, smin = 0xFFFFFFFFu;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        const int e = se0 + q;   // (< V: rows that sample are long)
        float x = sx[q];
        if (pen_inline && ((bm[e >> 5] >> (e & 31)) & 1u)) x = penalize(x, pen);
        sk4[q] = selkey(x, neg);
        smax = sk4[q] > smax ? sk4[q] : smax;
        smin = sk4[q] < smin ? sk4[q] : smin;
    }
    // The sample holds about Poisson(ks) of the row's top k; the bound fails
    // (the row streams again) when js or more of them are sampled: at most
    // 5e-6 per row for k <= 1024 with this margin of 4.5 standard
    // deviations and 3 (6 of them gave 1.2e-7, for 13 % more candidates).
    const float ks = (float)kk * (float)NSAMP / (float)V;
    uint32_t js = (uint32_t)ceilf(ks + 4.5f * sqrtf(ks) + 3.0f);
    js = js < (uint32_t)NSAMP ? js : (uint32_t)NSAMP;
    const Reduced sr = block_reduce(smax, smin, 0u);   // (its barriers also order the zeroed hist)
    const uint32_t span = sr.max - sr.min;
    const int sh = span >= 2048u ? (32 - __builtin_clz(span)) - 11 : 0;
    // Most of a sample crowds into a few bins at its low end, where lanes of
    // one atomic instruction that hit the same counter serialize: each
    // thread adds its equal bins at once, and the group sums are formed
    // from the bins afterwards instead of by atomics of their own.
    uint32_t b4[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) b4[q] = (sk4[q] - sr.min) >> sh;
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        bool first = true;
        uint32_t c = 1;
#pragma unroll
        for (int q2 = 0; q2 < NS; ++q2) {
            if (q2 < q) first = first && b4[q2] != b4[q];
            if (q2 > q) c += b4[q2] == b4[q] ? 1u : 0u;
        }
        if (first) atomicAdd(&hist[b4[q]], c);
    }
    __syncthreads();
    group_sums<uint32_t>(hist, s_cs);
    // (every wave finds the bin by itself)
    const WHit hb = wave_find_desc<uint32_t>(hist, (u64)s_cs[lane_id()], (u64)(js - 1u));
    est = sr.min + ((uint32_t)hb.bin << sh);
    if (est < SK_MIN) est = SK_MIN;
    theta = widen_threshold(est, T, neg);
}

// ---------------------------------------------------------------- small batches
//
// With few rows, one workgroup per row leaves most CUs idle and each row's
// stream runs at one CU's share of bandwidth.  For B <= SPLIT_MAX_B the
// launch (k_split, at the end of this file) cuts every top-k row that can
// defer its penalty (and every greedy row without one) into G slices of
// consecutive logits, one workgroup per slice (slice_row).  Every slice
// computes the row's sampled bound from the same sample with the same code,
// so all slices agree on it; a slice streams its logits and writes the keys
// that reach the bound with their ids, its key extremes and the bound (a
// greedy slice: its packed maximum) to a header and a candidate list in the
// workspace.  The row's last slice to finish then loads the row's
// candidates into its wave segments in place of a stream of its own and
// goes on from the count pass (fused_row); a row with a full slice, or one
// the slices did not take, streams there as usual.

// The slice's arrays: in the dynamic LDS of the launch, which the row's
// finish (fused_row) reuses once every slice is done.
constexpr int SL_LDS_HIST = 0;                                // 2048 bin counts
constexpr int SL_LDS_CS = SL_LDS_HIST + 4 * 2048;             // 64 group sums
constexpr int SL_LDS_N = SL_LDS_CS + 4 * 64;                  // the list's length
constexpr int SL_LDS_KEY = SL_LDS_N + 16;                     // SLICE_CAP keys
constexpr int SL_LDS_ID = SL_LDS_KEY + 4 * SLICE_CAP;         // SLICE_CAP ids
static_assert(SL_LDS_ID + 4 * SLICE_CAP <= KF_LDS_BYTES, "a slice's arrays fit the row's LDS");

// The hand-over is written with device-scope stores, which write through
// this XCD's L2: once they are acknowledged, the row's finish (on any XCD)
// reads them from memory after its acquire, and no L2 write-back is needed.
__device__ __forceinline__ void put_dev(uint32_t* a, uint32_t v)
{
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename TIn>
__device__ __forceinline__ void slice_row(const Params p, const int g, const int r, const int G, uint32_t* hdr_all,
                                          uint32_t* ent_all, unsigned char* sm)
{
    uint32_t* s_hist = (uint32_t*)(sm + SL_LDS_HIST);
    uint32_t* s_cs = (uint32_t*)(sm + SL_LDS_CS);
    uint32_t& s_n = *(uint32_t*)(sm + SL_LDS_N);
    uint32_t* s_key = (uint32_t*)(sm + SL_LDS_KEY);
    uint32_t* s_id = (uint32_t*)(sm + SL_LDS_ID);
    const int tid = threadIdx.x, lane = lane_id();
    const int V = p.V;
    const TIn* rowp = (const TIn*)p.logits + (size_t)r * (size_t)p.ld;
    uint32_t* hdr = hdr_all + (size_t)(r * G + g) * SL_HDR;
    uint32_t* ent = ent_all + (size_t)(r * G + g) * SLICE_CAP * 2;
    const float T = p.T[r];
    const int k = p.K[r];
    const float pen = p.PEN[r];
    int h0, h1;
    bool hbad;
    history_range(p, p.hoff ? p.hoff[r] : 0, p.hoff ? (p.hend ? p.hend[r] : p.hoff[r + 1]) : 0, pen, h0, h1, hbad);
    const RowMode mode = classify(T, k, V);
    const bool neg = T < 0.0f;
    const bool pen_on = (pen != 1.0f) && (h1 > h0);
    const bool defer = pen_on && !neg && pen >= 1.0f && pen <= 3.402823466e38f;
    const bool topk = mode == MODE_TOPK && V >= FAST_MIN_V && (!pen_on || defer);
    // (a greedy row with the LM head's maximum needs no slices)
    const bool greedy = mode == MODE_GREEDY && !pen_on && !p.pre_best;
    if ((!topk && !greedy) || hbad) {
        if (tid == 0) put_dev(hdr, SL_NONE);
        return;
    }
    // the slice: whole multiples of 8 logits (16-byte vectors of either dtype)
    const int L = (((V + G - 1) / G) + 7) & ~7;
    const int s0 = g * L < V ? g * L : V;
    const int n = (s0 + L < V ? s0 + L : V) - s0;
    if (greedy) {   // sampling.py:47-48: the slice's first maximum
        uint32_t bk = 0, bi = 0;
        RowStream<TIn> rs(rowp + s0, n);
        rs.template run<false>(nullptr, 1.0f,
            [&](int, int e, float x) {
                const uint32_t gk = (x != x) ? 0xFFFFFFFFu : vkey(x);   // NaN is the maximum
                if (gk > bk) { bk = gk; bi = (uint32_t)(s0 + e); }
            },
            [&](auto&&) { return false; });
        const u64 best = block_max<u64>(bk ? (((u64)bk << 32) | (u64)(0xFFFFFFFFu - bi)) : 0ull);
        if (tid == 0) { put_dev(hdr + 5, (uint32_t)best); put_dev(hdr + 6, (uint32_t)(best >> 32)); put_dev(hdr, 0u); }
        return;
    }
    constexpr int NS = NSAMP / NT;
    float sx[NS];
    const int se0 = (((tid >> 3) * (V >> 6)) & ~31) + (tid & 7) * NS;   // (the sample of k_fused)
#pragma unroll
    for (int q = 0; q < NS; ++q) sx[q] = VecIO<TIn>::one(rowp, se0 + q < V ? se0 + q : V - 1);
    for (int b = tid; b < 2048; b += NT) s_hist[b] = 0;
    if (tid < 64) s_cs[tid] = 0;
    if (tid == 0) s_n = 0;
    uint32_t est, theta;
    sample_bound(sx, se0, (uint32_t)k, V, T, neg, false, pen, nullptr, s_hist, s_cs, est, theta);
    // sampling.py:52-54: the slice's keys that reach the bound (raw keys: a
    // deferred penalty never raises one), appended with one LDS atomic per
    // wave and tile
    uint32_t omax = 0, omin = 0xFFFFFFFFu, hm = 0;
    uint32_t tk[FPT];
    RowStream<TIn> rs(rowp + s0, n);
    rs.template run<false>(nullptr, 1.0f,
        [&](int i, int, float x) {
            const uint32_t sk = selkey(x, neg);
            omax = sk > omax ? sk : omax;
            omin = sk < omin ? sk : omin;
            tk[i] = sk;
            hm |= (sk >= theta ? 1u : 0u) << i;
        },
        [&](auto&& id) -> bool {
            const uint32_t c = (uint32_t)__builtin_popcount(hm);
            const uint32_t incl = wave_prefix_u32(c);
            const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            if (tot) {
                uint32_t base = 0;
                if (lane == 63) base = atomicAdd(&s_n, tot);
                uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)base, 63) + incl - c;
#pragma unroll
                for (int i = 0; i < FPT; ++i) {
                    if ((hm >> i) & 1u) {
                        if (o < (uint32_t)SLICE_CAP) { s_key[o] = tk[i]; s_id[o] = (uint32_t)(s0 + id(i)); }
                        ++o;
                    }
                }
            }
            hm = 0;
            return false;
        });
    const Reduced rd = block_reduce(omax, omin, 0u);   // (its barriers publish the list)
    const uint32_t nh = s_n;
    if (nh <= (uint32_t)SLICE_CAP)
        for (uint32_t j = (uint32_t)tid; j < nh; j += NT)
            __hip_atomic_store((u64*)ent + j, (u64)s_key[j] | ((u64)s_id[j] << 32), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
        put_dev(hdr, nh <= (uint32_t)SLICE_CAP ? nh : SL_NONE);
        put_dev(hdr + 1, rd.max);
        put_dev(hdr + 2, rd.min);
        put_dev(hdr + 3, est);
        put_dev(hdr + 4, theta);
    }
}

// Rows that finish_counts serves: fp16, top-k off, long, a temperature
// that keeps every tempered value distinct and normal, and a finite positive
// penalty whose history fits the list.
template <typename TIn>
__device__ __forceinline__ bool counted_row(const Params& p, RowMode mode, int k, float T, float pen, bool pen_on,
                                            uint32_t nh)
{
    if constexpr (sizeof(TIn) != 2) {
        return false;
    } else {
        const float aT = __builtin_fabsf(T);
        return mode == MODE_LARGE && (k <= 0 || k >= p.V) && p.V >= FC_MIN_V && aT > 0x1p-100f && aT < 0x1p100f &&
               (!pen_on || (pen > 0.0f && pen <= 3.402823466e38f && nh <= (uint32_t)HCAP));
    }
}

template <typename TIn>
__device__ __forceinline__ bool finish_counts_as(const Params& p, int r, RowStream<TIn>& rs, float T, bool neg,
                                                 float top_p, float u, float pen, bool pen_on, uint32_t* bm,
                                                 uint32_t* hl, uint32_t nh, unsigned char* smem, int64_t& tok,
                                                 int32_t& st)
{
    if constexpr (sizeof(TIn) != 2) {
        return false;
    } else {
        return finish_counts(p, r, rs, T, neg, top_p, u, pen, pen_on, bm, hl, nh, smem, tok, st);
    }
}

// One row's chain in one workgroup.  SPLIT: the row's slices (slice_row)
// are done, and their candidates may replace the row's stream; the
// instance without it has none of that code.
template <typename TIn, bool SPLIT, bool SHARE = false>
__device__ __forceinline__ void fused_row(const Params p, const int r, unsigned char* smem)
{
    uint32_t* ck = (uint32_t*)(smem + KF_CK);   // candidate selection keys
    uint32_t* ci = (uint32_t*)(smem + KF_CI);   // candidate ids
    uint32_t* bm = (uint32_t*)(smem + KF_BM);   // history bitmap
    uint32_t* hist = (uint32_t*)(smem + KF_H);
    __shared__ uint32_t s_cnt[3];               // appends per tile, rotating
    __shared__ uint32_t s_seg[NWAVES];          // entries per buffer segment
    __shared__ uint32_t s_ovf;                  // a segment ran full
    __shared__ uint32_t s_nh;                   // distinct history ids listed in hl
    __shared__ u64 s_ms[64];                    // masses per group of 32 bins
    __shared__ uint32_t s_cs[64];               // counts per group of 32 bins
    __shared__ u64 s_rp[NWAVES], s_hp[NWAVES];  // raw_extremes: per-wave results
    __shared__ uint32_t s_mn[NWAVES];
    __shared__ uint32_t s_r[5][NWAVES];         // per-wave reductions after the stream

    const int tid = threadIdx.x, lane = lane_id();
    const int V = p.V;
    const TIn* rowp = (const TIn*)p.logits + (size_t)r * (size_t)p.ld;
    // Loads are issued in the order they are needed: the row's parameters,
    // the sample for a top-k row's first bound, then the row's first two
    // tiles (every valid row streams from its start, and the set-up below
    // overlaps them).  Requests are served in issue order, so the tiles, the
    // bulk, go last.
    //
    // The parameters: one gathered load, lane i of every wave reading
    // parameter i (an absent optional array reads a valid dummy instead);
    // they are read out of the lanes once the other loads are in flight.
    const uint32_t* pa = (const uint32_t*)(p.T + r);
    pa = lane == 1 ? (const uint32_t*)(p.K + r) : pa;
    pa = lane == 2 ? (const uint32_t*)(p.PEN + r) : pa;
    pa = lane == 3 ? (const uint32_t*)(p.P + r) : pa;
    pa = (lane == 4 && p.hoff) ? (const uint32_t*)(p.hoff + r) : pa;
    pa = (lane == 5 && p.hoff) ? (const uint32_t*)(p.hend ? p.hend + r : p.hoff + r + 1) : pa;
    pa = (lane == 6 && p.U) ? (const uint32_t*)(p.U + r) : pa;
    const uint32_t pv = *pa;
    // k_fused: the batch's rows with top-k off (whether rows are shared),
    // among the first NT rows, each wave counting 64; read with the parameters
    int kb = 0;
    float tb = 0.0f;
    if constexpr (!SPLIT && SHARE) {
        const int i = tid < p.B ? tid : 0;
        kb = p.K[i];
        tb = p.T[i];
    }
    // the slice headers of this row (a slice count per lane)
    uint32_t sln = 0;
    if constexpr (SPLIT) sln = p.sl_hdr[(size_t)(r * p.G + (lane < p.G ? lane : 0)) * SL_HDR];
    // The sample: NSAMP logits in 64 groups of 32 consecutive ones spread
    // over the row (a group is one 128-byte line of an fp32 row), 4 per
    // thread.  It is requested before the row's mode is known, so that it
    // does not queue behind the tiles; rows that do not use it waste 8 KB.
    // (After the slices it is requested only for a row they did not take:
    // the hand-over's loads would otherwise wait behind it.)
    constexpr int NS = NSAMP / NT;
    static_assert(NSAMP == 64 * 32 && NS * 8 == 32, "sample layout");
    float sx[NS];
    const int se0 = (((tid >> 3) * (V >> 6)) & ~31) + (tid & 7) * NS;   // this thread's first sample
    auto load_sample = [&]() {
#pragma unroll
        for (int q = 0; q < NS; ++q) sx[q] = VecIO<TIn>::one(rowp, se0 + q < V ? se0 + q : V - 1);
    };
    if constexpr (!SPLIT) load_sample();
    // (after the slices, or with the LM head's maxima: issued later, for the rows that stream)
    const bool early = !SPLIT && !p.pre_best;
    RowStream<TIn> rs(rowp, V, early);
    __builtin_amdgcn_sched_barrier(0);   // (the loads above stay ahead of the reads below)
    const float T = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_readlane((int)pv, 0));
    const int k = __builtin_amdgcn_readlane((int)pv, 1);
    const float pen = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_readlane((int)pv, 2));
    const float top_p = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_readlane((int)pv, 3));
    const int hv0 = __builtin_amdgcn_readlane((int)pv, 4);
    const int hv1 = __builtin_amdgcn_readlane((int)pv, 5);
    const float uv = __builtin_bit_cast(float, (uint32_t)__builtin_amdgcn_readlane((int)pv, 6));
    if constexpr (!SPLIT && SHARE) {
        const bool wd = sizeof(TIn) == 4 && tid < p.B && tb != 0.0f && tb == tb && (kb <= 0 || kb >= V) &&
                        V >= FAST_MIN_V;
        const u64 wm = __ballot(wd);
        if (lane == 0) g_wide[wave_id()] = wm;
    }
    int h0, h1;
    bool hbad;
    history_range(p, hv0, hv1, pen, h0, h1, hbad);
    const float u = p.U ? uv : 0.0f;
    RowMode mode = classify(T, k, V);
    // every slice of the row handed over its part: the candidates replace the stream
    bool split = false;
    if constexpr (SPLIT) {
        split = !__ballot(lane < p.G && sln == SL_NONE);
        if (!split) load_sample();
    }
    const bool neg = T < 0.0f;
    const bool pen_on = (pen != 1.0f) && (h1 > h0);
    // a greedy row without a penalty takes the LM head's maximum (sampling.py:47-48)
    const bool head_best = p.pre_best && mode == MODE_GREEDY && !pen_on && !hbad;
    if (!early && !split && !head_best) rs.restart();
    int64_t tok = -1;
    int32_t st = hbad ? MXS_ROW_BAD_HISTORY : MXS_ROW_OK;

    const bool sampled = mode == MODE_TOPK && V >= FAST_MIN_V;
    if (sampled) {
        for (int b = tid; b < 2048; b += NT) hist[b] = 0;
        if (tid < 64) s_cs[tid] = 0;
    }
    // With 1 <= pen < inf and T > 0 the penalty never raises a selection
    // key, so a top-k row's stream may compare raw keys: the raw hits include
    // every penalized hit.  Buffered history ids get their penalized keys
    // afterwards, and the history bitmap is first needed after the stream.
    const bool defer = pen_on && !neg && pen >= 1.0f && pen <= 3.402823466e38f;
    const bool late_bm = sampled && defer;
    if (p.out_probs) {
        float* o = p.out_probs + (size_t)r * (size_t)V;
        for (int i = tid; i < V; i += NT) o[i] = 0.0f;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");   // before the writes of the kept probabilities
    }
    if (tid < 3) s_cnt[tid] = 0;
    if (tid == 0) s_ovf = 0u;   // (a barrier follows before any wave may set it)

    // sampling.py:38-45: the row's history ids, each once (sorted(set())).
    // The first HB per thread are requested now and held in registers.
    // Rows with top-k off also list them (the thread that sets an id's bit
    // appends it) for the passes that correct raw values to penalized ones.
    constexpr int HB = 4;
    int hv[HB];
    uint32_t* hl = (uint32_t*)(smem + KF_HL);
    if (tid == 0) s_nh = 0;
    if (pen_on) {
        // (unconditional loads, clamped into the row's history: writing a
        // default into a register with a load pending would wait for every
        // load in flight; build_bitmap skips the clamped ones)
#pragma unroll
        for (int q = 0; q < HB; ++q) {
            const int h = h0 + tid + q * NT;
            hv[q] = p.hids[h < h1 ? h : h1 - 1];
        }
        const int words = (V + 31) >> 5;
        for (int w = tid; w < words; w += NT) bm[w] = 0;
    }
    // Sets the bits of the row's history (after a barrier that follows the
    // clearing above); returns whether this thread saw an id outside [0, V).
    auto build_bitmap = [&]() -> bool {
        bool bad = false;
        if (pen_on) {
            const bool list = mode == MODE_LARGE || mode == MODE_GREEDY;
            // (called by whole waves: the ids new to the bitmap take list
            // slots with one atomic per wave)
            auto add = [&](int id, bool valid) {
                bool fresh = false;
                if (valid) {
                    if (id < 0 || id >= V) {
                        bad = true;
                    } else {
                        const uint32_t bit = 1u << (id & 31);
                        fresh = !(atomicOr(&bm[id >> 5], bit) & bit);
                    }
                }
                if (list) {
                    const u64 fm = __ballot(fresh);
                    if (fm) {
                        const int first = __builtin_ctzll(fm);
                        uint32_t base = 0;
                        if (lane == first) base = atomicAdd(&s_nh, (uint32_t)__builtin_popcountll(fm));
                        const uint32_t slot = (uint32_t)__builtin_amdgcn_readlane((int)base, first) + lanes_below(fm);
                        if (fresh && slot < (uint32_t)HCAP) hl[slot] = (uint32_t)id;
                    }
                }
            };
#pragma unroll
            for (int q = 0; q < HB; ++q) add(hv[q], h0 + tid + q * NT < h1);
            for (int hb = h0 + HB * NT; hb < h1; hb += NT) {
                const int h = hb + tid;
                add(h < h1 ? p.hids[h] : 0, h < h1);
            }
        }
        return bad;
    };
    if (!late_bm) {
        __syncthreads();
        if (block_max<uint32_t>(build_bitmap() ? 1u : 0u)) st = MXS_ROW_BAD_HISTORY;   // (its barriers publish bm)
    }
    if (st == MXS_ROW_OK && mode == MODE_INVALID) st = MXS_ROW_BAD_PARAM;

    // A top-k row's first bound (step 1 below) is taken here, on the straight
    // path from the kernel's entry: at a join of the row modes' paths the
    // compiler's wait for the sample would also wait for the first tiles
    // (other paths leave loads pending into the same registers), which held
    // every row for the tiles' arrival.  (A row with an error computes it too;
    // nothing reads it then.)
    uint32_t est0 = 0, theta0 = 0;
    if (sampled && !split)
        sample_bound(sx, se0, (uint32_t)k, V, T, neg, pen_on && !defer, pen, bm, hist, s_cs, est0, theta0);

    // The penalized row's extremes from a raw stream (no penalty branch per
    // element): key_of(x) ranks a value; best gets the packed maximum
    // (key << 32 | ~index: the first index among equal keys), kmin the
    // smallest key over the raw row and the penalized history values (a
    // bound, and a witness of NaNs and infinities).  The history ids'
    // penalized values are folded in from the deduplicated list.  Returns
    // false when the raw maximum is itself a history id (the largest of the
    // other elements is then unknown): the caller streams again with the
    // penalty applied.  Requires the list (greedy and top-k-off rows) and a
    // penalty in (0, inf).
    const bool raw_ok = pen_on && pen > 0.0f && pen <= 3.402823466e38f &&
                        (mode == MODE_GREEDY || mode == MODE_LARGE);
    auto raw_extremes = [&](auto key_of, u64& best, uint32_t& kmin) -> bool {
        uint32_t bk = 0, bi = 0, mn = 0xFFFFFFFFu;
        rs.template run<false>(bm, pen,
            [&](int, int e, float x) {
                const uint32_t g = key_of(x);
                if (g > bk) { bk = g; bi = (uint32_t)e; }   // ascending e: the first maximum
                mn = g < mn ? g : mn;
            },
            [&](auto&&) { return false; });
        u64 hp = 0;
        const uint32_t nh = s_nh;
        auto fold = [&](int id, float x0) {
            const uint32_t g = key_of(penalize(x0, pen));
            const u64 pk = ((u64)g << 32) | (u64)(0xFFFFFFFFu - (uint32_t)id);
            hp = pk > hp ? pk : hp;
            mn = g < mn ? g : mn;
        };
        if (nh <= (uint32_t)HCAP) {
            for (uint32_t i0 = tid; i0 < nh; i0 += 4 * NT) {   // loads four at a time
                int id[4];
                float xv[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t i = i0 + (uint32_t)(q * NT);
                    id[q] = i < nh ? (int)hl[i] : -1;
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) xv[q] = VecIO<TIn>::one(rowp, id[q] >= 0 ? id[q] : 0);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (id[q] >= 0) fold(id[q], xv[q]);
            }
        } else {
            const int words = (V + 31) >> 5;
            for (int wd = tid; wd < words; wd += NT) {
                uint32_t bits = bm[wd];
                while (bits) {
                    const int bi2 = __builtin_ctz(bits);
                    bits &= bits - 1u;
                    fold(wd * 32 + bi2, VecIO<TIn>::one(rowp, wd * 32 + bi2));
                }
            }
        }
        const u64 rp = bk ? (((u64)bk << 32) | (u64)(0xFFFFFFFFu - bi)) : 0ull;
        const u64 a0 = wave_max<u64>(rp), a1 = wave_max<u64>(hp);
        const uint32_t a2 = wave_min_u32(mn);
        if (lane == 0) { s_rp[wave_id()] = a0; s_hp[wave_id()] = a1; s_mn[wave_id()] = a2; }
        __syncthreads();
        u64 rb = 0, hb = 0;
        kmin = 0xFFFFFFFFu;
#pragma unroll
        for (int v = 0; v < NWAVES; ++v) {
            rb = s_rp[v] > rb ? s_rp[v] : rb;
            hb = s_hp[v] > hb ? s_hp[v] : hb;
            kmin = s_mn[v] < kmin ? s_mn[v] : kmin;
        }
        __syncthreads();   // (the arrays may be read again)
        const uint32_t arg = 0xFFFFFFFFu - (uint32_t)rb;
        if (rb && ((bm[arg >> 5] >> (arg & 31)) & 1u)) return false;
        best = rb > hb ? rb : hb;
        return true;
    };

    if (st == MXS_ROW_OK && mode == MODE_GREEDY) {   // sampling.py:47-48
        auto gkey = [](float x) -> uint32_t { return (x != x) ? 0xFFFFFFFFu : vkey(x); };   // NaN is the maximum
        u64 best = head_best ? p.pre_best[r] : 0ull;
        uint32_t kmin;
        bool have = head_best || split || (raw_ok && raw_extremes(gkey, best, kmin));
        if (split) {   // the slices' maxima
            const uint32_t* h = p.sl_hdr + (size_t)(r * p.G + (lane < p.G ? lane : 0)) * SL_HDR;
            const u64 sb = lane < p.G ? (((u64)h[6] << 32) | h[5]) : 0ull;
            best = wave_max<u64>(sb);
        }
        if (!have) {
            if (raw_ok) rs.restart();
            uint32_t bk = 0, bi = 0;
            rs.run_pen(bm, pen_on, pen,
                [&](int, int e, float x) {
                    const uint32_t g = gkey(x);
                    if (g > bk) { bk = g; bi = (uint32_t)e; }   // ascending e: the first maximum
                },
                [&](auto&&) { return false; });
            best = block_max<u64>(bk ? (((u64)bk << 32) | (u64)(0xFFFFFFFFu - bi)) : 0ull);
        }
        tok = (int64_t)(0xFFFFFFFFu - (uint32_t)best);
        if (p.out_probs && tid == 0) p.out_probs[(size_t)r * (size_t)V + (size_t)tok] = 1.0f;
    } else if (st == MXS_ROW_OK && counted_row<TIn>(p, mode, k, T, pen, pen_on, s_nh) &&
               finish_counts_as<TIn>(p, r, rs, T, neg, top_p, u, pen, pen_on, bm, hl, s_nh, smem, tok, st)) {
        // an fp16 row with top-k off, finished from its value counts
    } else if (st == MXS_ROW_OK) {
        // selection keys of the penalized row: extremes (NaN and infinity
        // tests, the row maximum) and, for top-k rows, the candidates
        uint32_t omax = 0, omin = 0xFFFFFFFFu;
        uint32_t theta = 0, Nc = 0;
        int cidx = 0;
        bool overflow = false;
        const uint32_t kk = (uint32_t)k;
        // deferred penalty: buffered history ids get their penalized keys
        // (fix_up) before any bound is taken from the buffer
        uint32_t Nfix = 0;   // buffer entries [0, Nfix) hold penalized keys
        auto fix_up = [&]() {
            if (defer) {
                for (uint32_t j = Nfix + tid; j < Nc; j += NT) {
                    const uint32_t id = ci[j];
                    if ((bm[id >> 5] >> (id & 31)) & 1u) ck[j] = okey(penalize(okey_inv(ck[j]), pen));
                }
                __syncthreads();
            }
            Nfix = Nc;
        };
        uint32_t est = 0, cmax = 0;   // the sampled estimate; the buffer's largest penalized key
        int wide2 = -1;               // finish_wide2: 1 done, 0 general path, -1 not taken
        bool segs = false;            // the candidates are in the stream's per-wave segments
        bool binned = false;          // ... and carry their bins, counts and final masses
        bool have_rd = false;         // rd holds the penalized row's extremes
        float m0 = 0.0f, lest = 0.0f;
        Reduced rd{0u, 0xFFFFFFFFu, 0u};
        u64* MH = (u64*)(smem + KF_MH);
        if (mode == MODE_TOPK) {
            // 1. A conservative estimate of the k-th largest key from a strided
            //    sample of NSAMP logits: the lower edge of the histogram bin
            //    holding the sample's j-th largest, j well above the expected
            //    k * NSAMP / V.  It only steers the stream; step 3 checks it.
            //    (Computed before the row modes branch, as est0 / theta0.)
            bool fast = sampled;
            if (fast && split) {   // the slices computed the same bound
                est = p.sl_hdr[(size_t)r * p.G * SL_HDR + 3];
                theta = p.sl_hdr[(size_t)r * p.G * SL_HDR + 4];
                __syncthreads();   // (s_ovf is cleared before any wave may set it)
            } else if (fast) {
                est = est0;
                theta = theta0;
            }
            if (fast) {
                // 2. The stream: each wave appends its hits to its own segment
                //    of the buffer, so no barrier is needed.  A full segment
                //    stops every wave (step 4 takes over).
                const int w = wave_id();
                uint32_t* wck = ck + w * FSEG;
                uint32_t* wci = ci + w * FSEG;
                uint32_t cw = 0;   // (wave-uniform) entries in this wave's segment
                constexpr uint32_t SEG_USE = FSEG - 64;   // [SEG_USE, FSEG): the dummy words
                if (split) {
                    // the candidates of slices w, w + NWAVES, ... into this wave's
                    // segment: the slices' headers one per lane and, in the same
                    // round trip, entry `lane` of each of the wave's slices (most
                    // slices hand over fewer than 64); then the offsets by a wave
                    // prefix.  A slice with more than 64 takes the general loop,
                    // eight loads per lane at a time (clamped indices: no load
                    // behind a branch).
                    constexpr int SPW = 64 / NWAVES;   // slices per wave at most (G <= 64)
                    static_assert(SPW * NWAVES == 64, "every slice has a wave");
                    const int nsw = w < p.G ? (p.G - w + NWAVES - 1) / NWAVES : 0;   // (<= SPW)
                    const int gh = w + NWAVES * (lane < nsw ? lane : 0);   // (a wave without slices reads slice G - 1)
                    const uint32_t* h = p.sl_hdr + (size_t)(r * p.G + (gh < p.G ? gh : p.G - 1)) * SL_HDR;
                    const bool mine = lane < nsw;
                    const uint32_t hn = h[0], hmx = h[1], hmn = h[2];
                    uint2 sp[SPW];
#pragma unroll
                    for (int i = 0; i < SPW; ++i) {
                        const int si = w + NWAVES * (i < nsw ? i : 0);
                        sp[i] = ((const uint2*)(p.sl_ent + (size_t)(r * p.G + (si < p.G ? si : p.G - 1)) * SLICE_CAP * 2))[lane];
                    }
                    const uint32_t ng = mine ? hn : 0u;
                    omax = wave_max_u32(mine ? hmx : 0u);
                    omin = wave_min_u32(mine ? hmn : 0xFFFFFFFFu);
                    const uint32_t incl = wave_prefix_u32(ng);
                    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
                    const uint32_t excl = incl - ng;
                    const bool small = wave_max_u32(ng) <= 64u;
                    if (total > SEG_USE) {
                        if (lane == 0) __hip_atomic_store(&s_ovf, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                    } else if (small) {
#pragma unroll
                        for (int i = 0; i < SPW; ++i) {
                            if (i < nsw) {
                                const uint32_t ni = (uint32_t)__builtin_amdgcn_readlane((int)ng, i);
                                const uint32_t ei = (uint32_t)__builtin_amdgcn_readlane((int)excl, i);
                                if ((uint32_t)lane < ni) { wck[ei + lane] = sp[i].x; wci[ei + lane] = sp[i].y; }
                            }
                        }
                        cw = total;
                    } else {
                        for (uint32_t q0 = 0; q0 < total; q0 += 512u) {
                            uint2 v[8];
#pragma unroll
                            for (int i = 0; i < 8; ++i) {
                                uint32_t q = q0 + (uint32_t)lane + 64u * (uint32_t)i;
                                q = q < total ? q : total - 1u;
                                // the slice holding position q: the last one that starts at or below it
                                int ls = 0;
                                uint32_t base = 0;
                                for (int l = 1; l < nsw; ++l) {
                                    const uint32_t el = (uint32_t)__builtin_amdgcn_readlane((int)excl, l);
                                    if (q >= el) { ls = l; base = el; }
                                }
                                const uint2* e = (const uint2*)(p.sl_ent + (size_t)(r * p.G + w + NWAVES * ls) * SLICE_CAP * 2);
                                v[i] = e[q - base];
                            }
#pragma unroll
                            for (int i = 0; i < 8; ++i) {
                                const uint32_t q = q0 + (uint32_t)lane + 64u * (uint32_t)i;
                                if (q < total) { wck[q] = v[i].x; wci[q] = v[i].y; }
                            }
                        }
                        cw = total;
                    }
                } else {
                    // A hit is tested on the value itself: x >= tf (x <= tf for
                    // T < 0), tf the value of theta.  Every key >= theta passes;
                    // the test adds at most zeros of the other sign at a bound
                    // of +0 (-0 for T < 0), which widening never leaves (it
                    // goes past the other zero then).  The
                    // row's extremes are NaN-propagating maxima and minima of
                    // the values, and the segments take the values' raw bits
                    // (the count pass turns them into keys).  Each lane counts
                    // its hits; at the tile's end one wave prefix gives each
                    // lane its offset in the segment, and every slot is written
                    // without a branch (a miss writes a per-lane dummy word at
                    // the segment's end).  No barrier, no atomics.
                    const float tf = sel_inv(theta, neg);
                    float fmx = -INFINITY, fmn = INFINITY;
                    float tx[FPT];      // this tile's values
                    uint32_t nhit = 0;  // this lane's hits in the tile
                    auto stream = [&](auto negc) {
                        constexpr bool NEG = decltype(negc)::value;
                        auto hit = [&](float x) { return NEG ? x <= tf : x >= tf; };
                        // (every slot is visited: a slot past the row's end holds
                        // NaN, never a hit, instead of the last tile's value)
                        rs.run_pen_all(bm, pen_on && !defer, pen,
                            [&](int i, int, float x, bool valid) {
                                fmx = __builtin_elementwise_maximum(fmx, x);
                                fmn = __builtin_elementwise_minimum(fmn, x);
                                tx[i] = valid ? x : __builtin_nanf("");
                                nhit += hit(tx[i]) ? 1u : 0u;
                            },
                            [&](auto&& id) -> bool {
                                const uint32_t incl = wave_prefix_u32(nhit);
                                const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
                                if (__builtin_expect(cw + tot > SEG_USE, 0)) {
                                    if (lane == 0) __hip_atomic_store(&s_ovf, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                                    return true;
                                }
                                uint32_t o = cw + incl - nhit;
                                const uint32_t dummy = SEG_USE + (uint32_t)lane;
#pragma unroll
                                for (int i = 0; i < FPT; ++i) {
                                    const bool h = hit(tx[i]);
                                    const uint32_t a = h ? o : dummy;
                                    wck[a] = f2u(tx[i]);
                                    wci[a] = (uint32_t)id(i);
                                    o += h ? 1u : 0u;
                                }
                                nhit = 0;
                                cw += tot;
                                return __hip_atomic_load(&s_ovf, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u;
                            });
                    };
                    if (neg) stream(std::integral_constant<bool, true>{});
                    else stream(std::integral_constant<bool, false>{});
                    if (fmx != fmx) {   // a NaN (both extremes carry it): keys that say so
                        omax = 0xFFFFFFFFu;
                        omin = 0u;
                    } else {
                        omax = neg ? selkey(fmn, true) : selkey(fmx, false);
                        omin = neg ? selkey(fmx, true) : selkey(fmn, false);
                    }
                }
                if (lane == 0) s_seg[w] = cw;
                bool bad = false;
                if (late_bm) bad = build_bitmap();
                for (int b = tid; b < 2048; b += NT) { MH[b] = 0; hist[b] = 0; }
                {
                    const uint32_t a2 = wave_max_u32(omax), a3 = wave_min_u32(omin);
                    if (lane == 0) { s_r[2][w] = a2; s_r[3][w] = a3; }
                }
                __syncthreads();   // (publishes bm, s_seg, the cleared histograms)
                rd = Reduced{0u, 0xFFFFFFFFu, 0u};
#pragma unroll
                for (int v = 0; v < NWAVES; ++v) {
                    rd.max = s_r[2][v] > rd.max ? s_r[2][v] : rd.max;
                    rd.min = s_r[3][v] < rd.min ? s_r[3][v] : rd.min;
                }
                // 3. One pass over each wave's own segment: the penalty of its
                //    history ids (deferred penalty), the segment's largest key,
                //    the keys that reach the estimate, and for every element
                //    with l >= l_est = l(est) its bin (linear in d = l - m0 on
                //    [l_est - m0, 0], m0 the tempered row maximum before the
                //    deferred penalty), count and mass.  The estimate stands
                //    if at least k keys reach it: then the k-th largest key is
                //    >= est, and every element that ties with it after x / T
                //    is >= widen(est) = theta, so it is in the buffer.  The
                //    masses are final when the penalty left the maximum alone.
                m0 = sel_inv(rd.max, neg) / T;
                lest = sel_inv(est, neg) / T;
                const float dlo = lest - m0;
                const float scale = 2047.0f / -dlo;
                binned = dlo < 0.0f && dlo > -INFINITY && __builtin_isfinite(scale) && __builtin_isfinite(m0);
                uint32_t cmx = 0, nr = 0;
                // four entries per lane at a time, their loads issued together
                for (uint32_t j0 = (uint32_t)lane; j0 < cw; j0 += 256) {
                    uint32_t key[4], id[4], bw[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t j = j0 + 64u * q < cw ? j0 + 64u * q : j0;
                        key[q] = wck[j];
                        id[q] = wci[j];
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) bw[q] = defer ? bm[id[q] >> 5] : 0u;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t j = j0 + 64u * q;
                        if (j >= cw) continue;
                        // (the stream left raw values; the slices' candidates are keys)
                        float x = split ? sel_inv(key[q], neg) : u2f(key[q]);
                        const bool hp = (bw[q] >> (id[q] & 31)) & 1u;
                        if (hp) x = penalize(x, pen);
                        if (!split || hp) {
                            key[q] = selkey(x, neg);
                            wck[j] = key[q];
                        }
                        cmx = key[q] > cmx ? key[q] : cmx;
                        nr += key[q] >= est ? 1u : 0u;
                        if (binned) {
                            const float l = sel_inv(key[q], neg) / T;
                            if (l >= lest) {
                                const float f = ((l - m0) - dlo) * scale;
                                const uint32_t b = f < 2047.0f ? (uint32_t)f : 2047u;
                                atomicAdd(&hist[b], 1u);
                                wci[j] = id[q] | ((b + 1u) << TAG_SHIFT);
                            }
                        }
                    }
                }
                {
                    const uint32_t a0 = wave_max_u32(cmx), a1 = wave_sum_u32(nr), a4 = wave_max_u32(bad ? 1u : 0u);
                    if (lane == 0) { s_r[0][w] = a0; s_r[1][w] = a1; s_r[4][w] = a4; }
                }
                __syncthreads();
                uint32_t reach = 0, badw = 0;
                cmax = 0;
                Nc = 0;
#pragma unroll
                for (int v = 0; v < NWAVES; ++v) {
                    cmax = s_r[0][v] > cmax ? s_r[0][v] : cmax;
                    reach += s_r[1][v];
                    badw |= s_r[4][v];
                    Nc += s_seg[v];
                }
                if (badw) st = MXS_ROW_BAD_HISTORY;
                fast = st == MXS_ROW_OK && s_ovf == 0u && reach >= kk;
                segs = fast;
                if (__builtin_expect(segs && binned && cmax != rd.max, 0)) {
                    // the penalty lowered the row's maximum: the bins and
                    // masses again, relative to the penalized maximum
                    m0 = sel_inv(cmax, neg) / T;
                    const float dlo2 = lest - m0;
                    const float scale2 = 2047.0f / -dlo2;
                    binned = dlo2 < 0.0f && dlo2 > -INFINITY && __builtin_isfinite(scale2) && __builtin_isfinite(m0);
                    for (int b = tid; b < 2048; b += NT) hist[b] = 0;
                    __syncthreads();
                    for (uint32_t j = (uint32_t)lane; j < cw; j += 64) {
                        const uint32_t id = wci[j] & ID_MASK;
                        uint32_t word = id;
                        const float l = sel_inv(wck[j], neg) / T;
                        if (binned && l >= lest) {
                            const float f = ((l - m0) - dlo2) * scale2;
                            const uint32_t b = f < 2047.0f ? (uint32_t)f : 2047u;
                            atomicAdd(&hist[b], 1u);
                            word = id | ((b + 1u) << TAG_SHIFT);
                        }
                        wci[j] = word;
                    }
                    __syncthreads();
                }
            }
            if (__builtin_expect(!fast && st == MXS_ROW_OK, 0)) {
                // 4. The stream again with one shared buffer and a running
                //    bound raised by compaction whenever it nears capacity.
                theta = 0;
                Nc = 0;
                Nfix = 0;
                cidx = 0;
                if (tid < 3) s_cnt[tid] = 0;
                __syncthreads();
                uint32_t tk[FPT], te[FPT], hm = 0;   // this tile's keys, ids and hits
                if (sampled) rs.restart();
                rs.run_pen(bm, pen_on && !defer, pen,
                    [&](int i, int e, float x) {
                        const uint32_t sk = selkey(x, neg);
                        omax = sk > omax ? sk : omax;
                        omin = sk < omin ? sk : omin;
                        tk[i] = sk;
                        te[i] = (uint32_t)e;
                        hm |= (sk >= theta ? 1u : 0u) << i;
                    },
                    [&](auto&&) -> bool {
                        // after massive ties the rest of the row is still
                        // streamed, for its extremes (the row maximum and the
                        // NaN and infinity tests need every element), but
                        // nothing more is appended
                        if (overflow) { hm = 0; return false; }
                        // append this tile's hits: one LDS atomic per wave
                        uint32_t wtot;
                        const uint32_t pre = wave_excl_small((uint32_t)__builtin_popcount(hm), wtot);
                        if (wtot) {
                            uint32_t base = 0;
                            if (lane == 0) base = atomicAdd(&s_cnt[cidx], wtot);
                            uint32_t o = Nc + (uint32_t)__builtin_amdgcn_readfirstlane((int)base) + pre;
#pragma unroll
                            for (int i = 0; i < FPT; ++i) {
                                const bool h = (hm >> i) & 1u;
                                if (__ballot(h)) {
                                    if (h) { ck[o] = tk[i]; ci[o] = te[i]; ++o; }
                                }
                            }
                        }
                        hm = 0;
                        __syncthreads();
                        Nc += s_cnt[cidx];
                        cidx = cidx == 2 ? 0 : cidx + 1;
                        // the counter of the tile after next: every wave has read it
                        if (tid == 0) s_cnt[cidx == 2 ? 0 : cidx + 1] = 0;
                        if (Nc <= (uint32_t)(FCAP - FTILE)) return false;
                        // raise theta from the buffer, then compact it
                        fix_up();
                        uint32_t mx = 0, mn = 0xFFFFFFFFu;
                        for (uint32_t j = tid; j < Nc; j += NT) {
                            const uint32_t key = ck[j];
                            mx = key > mx ? key : mx;
                            mn = key < mn ? key : mn;
                        }
                        const Reduced rd = block_reduce(mx, mn, 0u);
                        const uint32_t lo = rd.min, span = rd.max - rd.min;
                        const int sh = span >= 2048u ? (32 - __builtin_clz(span)) - 11 : 0;
                        for (int b = tid; b < 2048; b += NT) hist[b] = 0;
                        __syncthreads();
                        for (uint32_t j = tid; j < Nc; j += NT) atomicAdd(&hist[(ck[j] - lo) >> sh], 1u);
                        __syncthreads();
                        const BinHit hb = find_desc<uint32_t>(hist, 2048, (u64)(kk - 1u));
                        uint32_t bound = lo + ((uint32_t)hb.bin << sh);
                        if (bound < SK_MIN) bound = SK_MIN;
                        const uint32_t nt = widen_threshold(bound, T, neg);
                        theta = nt > theta ? nt : theta;
                        constexpr int PER = FCAP / NT;
                        uint32_t kv[PER], iv[PER], keep = 0;
#pragma unroll
                        for (int q = 0; q < PER; ++q) {
                            const uint32_t j = (uint32_t)(tid + q * NT);
                            kv[q] = j < Nc ? ck[j] : 0u;
                            iv[q] = j < Nc ? ci[j] : 0u;
                            keep += (j < Nc && kv[q] >= theta) ? 1u : 0u;
                        }
                        uint32_t total;
                        uint32_t o = block_incl_scan<uint32_t>(keep, &total) - keep;   // its barriers end the reads
#pragma unroll
                        for (int q = 0; q < PER; ++q) {
                            const uint32_t j = (uint32_t)(tid + q * NT);
                            if (j < Nc && kv[q] >= theta) { ck[o] = kv[q]; ci[o] = iv[q]; ++o; }
                        }
                        Nc = total;
                        Nfix = total;
                        __syncthreads();
                        if (Nc > (uint32_t)(FCAP - FTILE)) overflow = true;   // massive ties
                        return false;
                    });
                if (!overflow) fix_up();
            }
        } else if (mode == MODE_LARGE && (k <= 0 || k >= V) && V >= FAST_MIN_V &&
                   (wide2 = finish_wide2<TIn, !SPLIT && SHARE>(p, r, rs, T, neg, top_p, u, pen, pen_on, bm, sx, se0, h0, h1, smem, hist,
                                              rd, tok, st)) >= 0) {
            // top-k off, two passes (done, or rd holds the extremes for the general path)
            have_rd = true;
        } else {
            u64 best = 0;
            uint32_t kmin = 0;
            if (raw_ok && raw_extremes([&](float x) { return selkey(x, neg); }, best, kmin)) {
                rd = Reduced{(uint32_t)(best >> 32), kmin, 0u};
                have_rd = true;
            } else {
                if (raw_ok) rs.restart();
                rs.run_pen(bm, pen_on, pen,
                    [&](int, int, float x) {
                        const uint32_t sk = selkey(x, neg);
                        omax = sk > omax ? sk : omax;
                        omin = sk < omin ? sk : omin;
                    },
                    [&](auto&&) { return false; });
            }
        }
        if (!segs && !have_rd) rd = block_reduce(omax, omin, 0u);
        // NaN keys lie above the key of +inf and below that of -inf (the
        // reversed keys of T < 0 swap the two ranges)
        const bool has_nan = rd.max > 0xFF800000u || rd.min < 0x007FFFFFu;
        const bool has_inf = rd.max >= 0xFF800000u || rd.min <= 0x007FFFFFu;
        if (wide2 == 1 || st != MXS_ROW_OK) {
            // finished by finish_wide2, or a history id outside [0, V) found after the stream
        } else if (__builtin_expect(has_nan || (has_inf && __builtin_isinf(T)), 0)) {
            st = MXS_ROW_NONFINITE;   // a NaN tempered logit heads the order (sampling.py:57-58)
        } else {
            bool done = false;
            uint32_t thk = 0;
            bool thk_known = false;
            if (segs) {
                if (binned) {
                    // (its kept list goes where the history bitmap was)
                    done = finish_segs(p, r, ck, ci, s_seg, T, neg, kk, m0, top_p, u, MH, hist, s_ms,
                                       (u64*)(smem + KF_BM), tok, st);
                    if (__builtin_expect(!done && pen_on, 0)) {   // the general path needs the bitmap again
                        const int words = (V + 31) >> 5;
                        for (int w2 = tid; w2 < words; w2 += NT) bm[w2] = 0;
                        __syncthreads();
                        (void)build_bitmap();
                        __syncthreads();
                    }
                }
                if (__builtin_expect(!done, 0)) {
                    // compact the segments (ids without their bin tags): the
                    // buffer becomes [0, Nc) for the general path
                    constexpr int PERW = FSEG / 64;
                    const int w = wave_id();
                    const uint32_t cw = s_seg[w];
                    uint32_t off = 0;
#pragma unroll
                    for (int v = 0; v < NWAVES; ++v) off += v < w ? s_seg[v] : 0u;
                    uint32_t kv[PERW], iv[PERW];
#pragma unroll
                    for (int q = 0; q < PERW; ++q) {
                        const uint32_t j = (uint32_t)(lane + 64 * q);
                        kv[q] = j < cw ? ck[w * FSEG + j] : 0u;
                        iv[q] = j < cw ? ci[w * FSEG + j] & ID_MASK : 0u;
                    }
                    __syncthreads();
#pragma unroll
                    for (int q = 0; q < PERW; ++q) {
                        const uint32_t j = (uint32_t)(lane + 64 * q);
                        if (j < cw) { ck[off + j] = kv[q]; ci[off + j] = iv[q]; }
                    }
                    Nfix = Nc;
                    __syncthreads();
                }
            }
            if (__builtin_expect(mode == MODE_TOPK && !overflow && !done, 0)) {
                auto visit = [&](auto&& f) {
                    for (uint32_t j = tid; j < Nc; j += NT) f(ck[j]);
                };
                // sampling.py:52-54: the k-th largest, then everything that rounds onto it.
                // At least k buffered keys lie in [theta, row maximum] (keys that
                // the penalty took below theta are not among the top k).
                uint32_t sk_k = select_exact_in(kk, visit, hist, neg, theta, rd.max);
                if (sk_k < SK_MIN) sk_k = SK_MIN;
                thk = widen_threshold(sk_k, T, neg);
                thk_known = true;
                uint32_t mine = 0;
                visit([&](uint32_t sk) { mine += sk >= thk ? 1u : 0u; });
                uint32_t n1u;
                uint32_t o = block_incl_scan<uint32_t>(mine, &n1u) - mine;
                if (n1u <= (uint32_t)SORT_CAP) {
                    u64* keys = (u64*)(smem + KF_BM);
                    for (uint32_t j = tid; j < Nc; j += NT) {
                        const uint32_t sk = ck[j];
                        if (sk >= thk) {
                            const uint32_t vk = vkey(sel_inv(sk, neg) / T);
                            keys[o++] = ((u64)vk << 32) | (u64)(0xFFFFFFFFu - ci[j]);
                        }
                    }
                    __syncthreads();
                    done = finish_kept(p, r, keys, (u64*)(smem + KF_CK), (int)n1u, top_p, u,
                                       (u64*)(smem + KF_MH), hist, tok, st);
                }
            }
            if (!done && mode == MODE_LARGE && (k <= 0 || k >= V) && wide2 < 0) {
                __syncthreads();
                done = finish_wide<TIn>(p, r, T, neg, top_p, u, pen, pen_on, bm, hl, s_nh, rd.max, rd.min,
                                        (u64*)(smem + KF_MH),
                                        hist, (u64*)(smem + KF_CK), (u64*)(smem + KF_CK + 8 * LCAP),
                                        (u64*)(smem + KF_CK + 16 * LCAP),
                                        (uint32_t*)(smem + KF_CK + 16 * LCAP + 8 * 2048), tok, st);
            }
            if (__builtin_expect(!done, 0)) {
                __syncthreads();
                const LargeLds lds{bm, (u64*)(smem + KF_MH), (u64*)(smem + KF_CK), hist};
                const uint32_t skmax = rd.max;
                const bool raw_max = defer && mode == MODE_TOPK;   // then the maximum is taken again
                finish_large<TIn>(p, r, T, k, top_p, pen, pen_on, skmax, !raw_max, thk_known, thk, u, lds,
                                  tok, st);
            }
        }
    }
    if (tid == 0) {
        p.out_tok[r] = st == MXS_ROW_OK ? tok : -1;
        if (p.out_status) p.out_status[r] = st;
    }
}

// Batches above SPLIT_MAX_B rows: one workgroup per row.  SHARE (the
// caller's flag MXS_FLAG_SHARE_ROWS, fp32): rows with top-k off share their
// passes, and every workgroup then helps with those still running
// (help_rows).  The instance without it has none of that code: its
// presence alone costs the other rows about a microsecond.
template <typename TIn, bool SHARE>
__global__ __launch_bounds__(NT, 1) void k_fused(Params p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    fused_row<TIn, false, SHARE>(p, (int)blockIdx.x, smem);
    if constexpr (SHARE) {
        if (p.wj) {
            __syncthreads();   // (the row's LDS is free)
            help_rows<TIn>(p, smem);
        }
    }
}

// Batches of up to SPLIT_MAX_B rows, in one launch: workgroup (g, r) runs
// slice g of row r, and the row's last slice to finish (one counter per
// row in the workspace, zero before the launch, which that workgroup
// returns to zero) goes on with the row's chain from the slices'
// hand-over.  No workgroup waits for another.  The hand-over is written
// through to memory (put_dev) and every wave waits until its stores are
// acknowledged before the count (a release fence would also write back
// this XCD's whole L2, about a microsecond); in the last workgroup one
// thread acquires the other slices' writes after it (invalidating the
// caches its waves read through).
template <typename TIn>
__global__ __launch_bounds__(NT, 1) void k_split(Params p)
{
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ uint32_t s_last;
    const int G = (int)gridDim.x, g = (int)blockIdx.x, r = (int)blockIdx.y;
    slice_row<TIn>(p, g, r, G, (uint32_t*)p.sl_hdr, (uint32_t*)p.sl_ent, smem);
    __builtin_amdgcn_s_waitcnt(0);   // (all counters: this wave's stores are acknowledged)
    __syncthreads();
    if (threadIdx.x == 0) {
        // the counter: the unused last word of the header of the row's slice 0
        uint32_t* cnt = (uint32_t*)p.sl_hdr + (size_t)r * G * SL_HDR + SL_CNT_WORD;
        const uint32_t before = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = before == (uint32_t)(G - 1);
        if (last) {
            __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        s_last = last ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    fused_row<TIn, true>(p, r, smem);
}

}  // namespace
}  // namespace mxs
