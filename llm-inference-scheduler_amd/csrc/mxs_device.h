// mxs_device.h -- device building blocks of the gfx950 sampler kernels.
//
// Everything here runs inside one 512-thread workgroup (8 wave64s).  The
// arithmetic helpers (keys, mass, exact thresholds) are the same operation
// sequences the CPU oracle uses, so results agree bit for bit; the file must
// be compiled with -ffp-contract=off so that the only fused multiply-adds are
// the explicit __builtin_fmaf calls.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxs {

typedef unsigned long long u64;
typedef unsigned __int128 u128;

constexpr int NT = 512;                 // threads per workgroup
constexpr int NWAVES = NT / 64;
constexpr int KMAX = 1024;              // largest top_k served by the candidate path
constexpr int SORT_CAP = 4096;          // top-k survivors sorted in LDS (= 8 per thread)
constexpr int LCAP = 4096;              // elements collected per refinement step (= 8 per thread)
constexpr int MASS_SHIFT = 20;          // masses carry 44 fractional bits: 24-bit P << (20 + n)
constexpr uint32_t SK_MIN = 0x007FFFFFu;  // selection key of -inf (T > 0) or +inf (T < 0)

// LDS map of the one-workgroup-per-row kernel.
constexpr int FCAP = 12288;                     // candidates held while streaming
constexpr int FTILE = 8192;                     // logits streamed between capacity checks
constexpr int FSEG = FCAP / NWAVES;             // buffer segment of one wave
constexpr int NSAMP = 2048;                     // logits sampled for the first bound
constexpr int FAST_MIN_V = 8 * NSAMP;           // rows shorter than this skip the sample
constexpr int KF_CK = 0;                        // FCAP candidate keys; later SORT_CAP masses
constexpr int KF_CI = KF_CK + 4 * FCAP;         // FCAP candidate ids
constexpr int KF_HL = 90112;                    // top-k-off rows: distinct history ids (in the candidate area)
constexpr int HCAP = (2 * 4 * FCAP - KF_HL) / 4; // 2048 of them
constexpr int KF_BM = KF_CI + 4 * FCAP;         // history bitmap (MXS_MAX_VOCAB bits); later sort keys
constexpr int KF_MH = KF_BM + 32768;            // 2048 x u64
constexpr int KF_H = KF_MH + 16384;             // 2048 x u32
constexpr int KF_LDS_BYTES = KF_H + 8192;

__host__ __device__ __forceinline__ uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ __forceinline__ float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// Order-preserving key: a < b (non-NaN)  =>  okey(a) < okey(b).
__host__ __device__ __forceinline__ uint32_t okey(float f)
{
    const uint32_t u = f2u(f);   // negative: all bits flipped; otherwise the sign bit set
    return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
}
__host__ __device__ __forceinline__ float okey_inv(uint32_t k)
{
    return u2f((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
// Value key: -0 and +0 compare equal, so they share the key of +0.
__host__ __device__ __forceinline__ uint32_t vkey(float f) { return okey(f == 0.0f ? 0.0f : f); }

// Selection key of a penalized logit x: ordered like x / T (reversed for T < 0).
__device__ __forceinline__ uint32_t selkey(float x, bool neg)
{
    return okey(x) ^ (neg ? 0xFFFFFFFFu : 0u);
}
__device__ __forceinline__ float sel_inv(uint32_t s, bool neg) { return okey_inv(neg ? ~s : s); }

// Integer softmax numerator of d = fl32(l - m) <= 0: floor(exp(d) * 2^44), with
// exp evaluated as 2^n * q(r): n = rint(d log2 e), r = d - n ln2 (Cody-Waite,
// two fma), q = degree-7 Taylor polynomial of exp(r) in Horner form.
__host__ __device__ __forceinline__ u64 mass_of(float d)
{
    if (!(d >= -104.0f)) return 0;
    float t = d * 0x1.715476p+0f;
    float n = __builtin_rintf(t);
    float r = __builtin_fmaf(n, -0x1.62e4p-1f, d);
    r = __builtin_fmaf(n, -0x1.7f7d1cp-20f, r);
    float q = 0x1.a01a02p-13f;
    q = __builtin_fmaf(q, r, 0x1.6c16c2p-10f);
    q = __builtin_fmaf(q, r, 0x1.111112p-7f);
    q = __builtin_fmaf(q, r, 0x1.555556p-5f);
    q = __builtin_fmaf(q, r, 0x1.555556p-3f);
    q = __builtin_fmaf(q, r, 0.5f);
    q = __builtin_fmaf(q, r, 1.0f);
    q = __builtin_fmaf(q, r, 1.0f);
    uint32_t P = (uint32_t)(q * 16777216.0f);
    int s = MASS_SHIFT + (int)n;
    if (s >= 0) return (u64)P << s;
    if (s <= -26) return 0;
    return (u64)(P >> (-s));
}

// c * mass_of(d) for c < 2^16 and d <= 0 (0 for NaN), without branches: P (< 2^25)
// is shifted right first when the exponent is negative, as mass_of does.
__device__ __forceinline__ u64 count_mass(uint32_t c, float d)
{
    const float dc = __builtin_fminf(d, 0.0f);   // (d itself for d <= 0; keeps n finite)
    const float t = dc * 0x1.715476p+0f;
    const float n = __builtin_rintf(t);
    float r = __builtin_fmaf(n, -0x1.62e4p-1f, dc);
    r = __builtin_fmaf(n, -0x1.7f7d1cp-20f, r);
    float q = 0x1.a01a02p-13f;
    q = __builtin_fmaf(q, r, 0x1.6c16c2p-10f);
    q = __builtin_fmaf(q, r, 0x1.111112p-7f);
    q = __builtin_fmaf(q, r, 0x1.555556p-5f);
    q = __builtin_fmaf(q, r, 0x1.555556p-3f);
    q = __builtin_fmaf(q, r, 0.5f);
    q = __builtin_fmaf(q, r, 1.0f);
    q = __builtin_fmaf(q, r, 1.0f);
    const uint32_t P = (uint32_t)(q * 16777216.0f);
    const int s = MASS_SHIFT + (int)n;   // (n >= -152 where d >= -104)
    const uint32_t ce = d >= -104.0f ? c : 0u;
    const uint32_t Ps = s >= 0 ? P : P >> (-s < 31 ? -s : 31);
    const uint32_t sh = s >= 0 ? (uint32_t)s : 0u;
    return ((u64)ce * (u64)Ps) << sh;
}

// v in [0, 1) as M * 2^-sh, M < 2^24.
__host__ __device__ __forceinline__ void split_unit(float v, uint32_t& M, int& sh)
{
    uint32_t b = f2u(v), e = (b >> 23) & 0xFFu, f = b & 0x7FFFFFu;
    if (e == 0) { M = f; sh = 149; }
    else        { M = f | 0x800000u; sh = 150 - (int)e; }
}

// ceil(p * W) for 0 < p < 1, exact.
__host__ __device__ __forceinline__ u64 ceil_mul(float p, u64 W)
{
    uint32_t M; int sh;
    split_unit(p, M, sh);
    u128 prod = (u128)M * W;
    if (prod == 0) return 0;
    if (sh >= 100) return 1;
    u128 one = (u128)1 << sh;
    return (u64)((prod + one - 1) >> sh);
}

// floor(u * W) for 0 <= u < 1, exact.
__host__ __device__ __forceinline__ u64 floor_mul(float u, u64 W)
{
    uint32_t M; int sh;
    split_unit(u, M, sh);
    if (sh >= 100) return 0;
    return (u64)(((u128)M * W) >> sh);
}

__host__ __device__ __forceinline__ float clamp_uniform(float u)
{
    if (!(u >= 0.0f)) return 0.0f;
    if (u >= 1.0f) return 0x1.fffffep-1f;
    return u;
}

// ---------------------------------------------------------------- wave/block

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// ---------------------------------------------------------------- DPP wave operations
//
// Wave-wide prefix operations through DPP lane moves, which stay in the
// vector ALU (no LDS round trips): shifts by 1, 2, 4 and 8 within each row of
// 16 lanes, then row 0's result into row 1 and row 2's into row 3
// (row_bcast:15), then lane 31's into rows 2 and 3 (row_bcast:31).  Lanes
// without a source receive the operation's identity.  Every lane of the wave
// must be active.
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_move_or(uint32_t v, uint32_t id)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)id, (int)v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ u64 dpp_move64_or(u64 v, u64 id)
{
    const uint32_t lo = dpp_move_or<CTRL, ROWS>((uint32_t)v, (uint32_t)id);
    const uint32_t hi = dpp_move_or<CTRL, ROWS>((uint32_t)(v >> 32), (uint32_t)(id >> 32));
    return ((u64)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t dpp_step(uint32_t v, uint32_t id, int step)
{
    switch (step) {
    case 0: return dpp_move_or<0x111, 0xF>(v, id);
    case 1: return dpp_move_or<0x112, 0xF>(v, id);
    case 2: return dpp_move_or<0x114, 0xF>(v, id);
    case 3: return dpp_move_or<0x118, 0xF>(v, id);
    case 4: return dpp_move_or<0x142, 0xA>(v, id);
    default: return dpp_move_or<0x143, 0xC>(v, id);
    }
}
__device__ __forceinline__ u64 dpp_step(u64 v, u64 id, int step)
{
    switch (step) {
    case 0: return dpp_move64_or<0x111, 0xF>(v, id);
    case 1: return dpp_move64_or<0x112, 0xF>(v, id);
    case 2: return dpp_move64_or<0x114, 0xF>(v, id);
    case 3: return dpp_move64_or<0x118, 0xF>(v, id);
    case 4: return dpp_move64_or<0x142, 0xA>(v, id);
    default: return dpp_move64_or<0x143, 0xC>(v, id);
    }
}
// Inclusive prefix of op over the wave (32- or 64-bit unsigned values).
template <typename T, class Op>
__device__ __forceinline__ T wave_prefix_op(T v, T id, Op op)
{
#pragma unroll
    for (int step = 0; step < 6; ++step) v = op(v, dpp_step(v, id, step));
    return v;
}
template <typename T>
__device__ __forceinline__ T lane63(T v)
{
    if constexpr (sizeof(T) == 8) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((u64)v >> 32), 63);
        return (T)(((u64)hi << 32) | lo);
    } else {
        return (T)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    }
}
// Wave-wide results, in every lane.
template <typename T> __device__ __forceinline__ T wave_max(T v)
{
    return lane63(wave_prefix_op<T>(v, (T)0, [](T a, T b) { return a > b ? a : b; }));
}
template <typename T> __device__ __forceinline__ T wave_sum(T v)
{
    return lane63(wave_prefix_op<T>(v, (T)0, [](T a, T b) { return a + b; }));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) { return wave_max<uint32_t>(v); }
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) { return wave_sum<uint32_t>(v); }
// The sum of v < 2^63 over the wave as three 32-bit sums of 21-bit parts
// (each part's sum stays below 2^27).
__device__ __forceinline__ u64 wave_sum_u64(u64 v)
{
    const uint32_t a = wave_sum_u32((uint32_t)v & 0x1FFFFFu);
    const uint32_t b = wave_sum_u32((uint32_t)(v >> 21) & 0x1FFFFFu);
    const uint32_t c = wave_sum_u32((uint32_t)(v >> 42));
    return (u64)a + ((u64)b << 21) + ((u64)c << 42);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
    return lane63(wave_prefix_op<uint32_t>(v, 0xFFFFFFFFu, [](uint32_t a, uint32_t b) { return a < b ? a : b; }));
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v)
{
    return lane63(wave_prefix_op<uint32_t>(v, 0u, [](uint32_t a, uint32_t b) { return a | b; }));
}
__device__ __forceinline__ uint32_t wave_prefix_u32(uint32_t v)
{
    return wave_prefix_op<uint32_t>(v, 0u, [](uint32_t a, uint32_t b) { return a + b; });
}
__device__ __forceinline__ u64 wave_prefix_u64(u64 v)
{
    return wave_prefix_op<u64>(v, 0ull, [](u64 a, u64 b) { return a + b; });
}

// ---------------------------------------------------------------- block operations

template <typename T>
__device__ __forceinline__ T block_max(T v)
{
    __shared__ T s[NWAVES];
    v = wave_max<T>(v);
    __syncthreads();
    if (lane_id() == 0) s[wave_id()] = v;
    __syncthreads();
    T t = s[0];
#pragma unroll
    for (int i = 1; i < NWAVES; ++i) t = s[i] > t ? s[i] : t;
    return t;
}

// Number of set bits of `mask` below this lane.
__device__ __forceinline__ uint32_t lanes_below(u64 mask)
{
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

template <typename T>
__device__ __forceinline__ T block_sum(T v)
{
    __shared__ T s[NWAVES];
    v = wave_sum<T>(v);
    __syncthreads();
    if (lane_id() == 0) s[wave_id()] = v;
    __syncthreads();
    T t = 0;
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) t += s[i];
    return t;
}

// Inclusive scan of one value per thread, in thread order; *total gets the sum.
template <typename T>
__device__ __forceinline__ T block_incl_scan(T v, T* total)
{
    __shared__ T s[NWAVES];
    const int w = wave_id();
    v = wave_prefix_op<T>(v, (T)0, [](T a, T b) { return a + b; });
    __syncthreads();
    if (lane_id() == 63) s[w] = v;
    __syncthreads();
    T off = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) {
        if (i < w) off += s[i];
        tot += s[i];
    }
    *total = tot;
    return v + off;
}

struct BinHit {
    int bin;
    u64 above;   // sum of the bins above `bin`
};

// Descending search over h[0..nb): the bin b with  above(b) <= t < above(b) + h[b],
// where above(b) = sum of h over bins > b.  nb must be a multiple of NT.
template <typename T>
__device__ __forceinline__ BinHit find_desc(const T* h, int nb, u64 t)
{
    __shared__ BinHit s_hit;
    const int per = nb / NT;
    const int b0 = threadIdx.x * per;
    if (threadIdx.x == 0) s_hit = BinHit{0, 0};   // ordered before the search by the scan's barriers
    T mine = 0;
    for (int i = 0; i < per; ++i) mine += h[b0 + i];
    T total;
    T incl = block_incl_scan<T>(mine, &total);
    u64 a = (u64)(total - incl);   // sum of the bins above this thread's range
    for (int b = b0 + per - 1; b >= b0; --b) {
        u64 hb = (u64)h[b];
        if (a <= t && t < a + hb) s_hit = BinHit{b, a};
        a += hb;
    }
    __syncthreads();
    BinHit r = s_hit;
    __syncthreads();
    return r;
}

// kk-th largest (1-based) 32-bit key among the keys a workgroup enumerates,
// by an MSD radix select with digits of 11, 11 and 10 bits and a 2048-entry
// LDS histogram.  `visit(f)` must call f(key) once for every key owned by the
// calling thread (together the threads cover the whole set).  When the bin
// holding the answer has at most `small` keys the search stops and returns
// that bin's lower edge (a valid lower bound); small = 0 gives the exact key.
template <class Visit>
__device__ __forceinline__ uint32_t block_select_desc_v(uint32_t kk, Visit visit, uint32_t* hist, uint32_t small)
{
    const int shifts[3] = {21, 10, 0};
    const int widths[3] = {11, 11, 10};
    uint32_t prefix = 0;
    for (int lev = 0; lev < 3; ++lev) {
        const int sh = shifts[lev], nb = 1 << widths[lev];
        const int hsh = sh + widths[lev];
        for (int b = threadIdx.x; b < nb; b += NT) hist[b] = 0;
        __syncthreads();
        visit([&](uint32_t k) {
            if (lev == 0 || (k >> hsh) == prefix) atomicAdd(&hist[(k >> sh) & (nb - 1)], 1u);
        });
        __syncthreads();
        BinHit hit = find_desc<uint32_t>(hist, nb, (u64)(kk - 1));
        kk -= (uint32_t)hit.above;
        prefix = (prefix << widths[lev]) | (uint32_t)hit.bin;
        uint32_t cnt = hist[hit.bin];
        __syncthreads();
        if (cnt <= small || lev == 2) return prefix << sh;
    }
    return prefix;
}

// Indexed form: keys key(i) for i in [0, n).
template <class KeyF>
__device__ __forceinline__ uint32_t block_select_desc(int n, uint32_t kk, KeyF key, uint32_t* hist, uint32_t small)
{
    return block_select_desc_v(kk, [&](auto&& f) {
        for (int i = threadIdx.x; i < n; i += NT) f(key(i));
    }, hist, small);
}

// Bitonic sort of P (power of two) u64 keys in LDS, descending.
__device__ __forceinline__ void bitonic_sort_desc(u64* a, int P)
{
    for (int k = 2; k <= P; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < P; i += NT) {
                int ixj = i ^ j;
                if (ixj > i) {
                    u64 x = a[i], y = a[ixj];
                    bool up = (i & k) != 0;   // this sub-block ascends
                    if (up ? (x > y) : (x < y)) { a[i] = y; a[ixj] = x; }
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ int pow2_ceil(int n)
{
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}

}  // namespace mxs
