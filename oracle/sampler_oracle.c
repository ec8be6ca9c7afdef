/*
 * sampler_oracle.c -- CPU oracle for the sampler chain.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: it is loaded by
 * tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg,
 * and by nothing else.  The product (the HIP library and the Python package)
 * never links, imports or calls it.
 *
 * It restates the reference chain, mini_engine/sampling.py:30-69, one row at
 * a time, in plain C with every rounding step written out, so that the GPU
 * kernels can be required to reproduce its results bit for bit:
 *
 *   sampling.py:36     logits.float()            fp16 rows are upcast exactly by
 *                                                 the caller (numpy) before this file
 *   sampling.py:38-45  repetition penalty         x>0 ? fl32(x/pen) : fl32(x*pen),
 *                                                 once per unique history id
 *   sampling.py:47-48  greedy (T == 0)            first index of the maximum,
 *                                                 NaN counts as the maximum
 *   sampling.py:50     temperature                fl32(x / T), IEEE division
 *   sampling.py:52-54  top-k                      kth = k-th largest value;
 *                                                 keep !(l < kth) (ties at kth kept)
 *   sampling.py:56-66  top-p                      stable sort (value desc, index asc);
 *                                                 drop j when the mass before j
 *                                                 is >= top_p of the total
 *   sampling.py:68     softmax                    fl32(w_j / W_kept)
 *   sampling.py:69     draw                       inverse CDF over the kept list in
 *                                                 sorted order, from one uniform u
 *
 * Departures from torch's numerics, each deliberate (the reference's own
 * fp32 softmax and cumsum bits cannot be reproduced outside torch's CPU
 * kernels, so the oracle fixes an exact, order-independent definition):
 *
 *  - Softmax numerators are integer masses.  w = floor(exp(l - m) * 2^44),
 *    where exp is the fp32 function below (Cody-Waite reduction by ln2,
 *    degree-7 Taylor polynomial evaluated with fma, 2^n applied as an integer
 *    shift).  Sums of masses are exact 64-bit integer sums, so any summation
 *    order gives the same bits.  V <= 2^19 keeps every sum below 2^63.
 *  - torch's cut `fl32(cumsum(p) - p) >= fl32(top_p)` is evaluated exactly:
 *    E_j >= top_p * W  <=>  E_j >= ceil(top_p * W), with E_j the exclusive
 *    prefix mass in sorted order and the product formed in 128-bit integers.
 *  - torch.multinomial's exponential race (V draws from the generator) is
 *    replaced by one uniform u per row: the token is the first j in sorted
 *    order whose inclusive prefix mass C_j exceeds floor(u * W_kept).
 *  - Ties in the top-p sort go to the lowest index (torch.sort(stable=True));
 *    the reference uses stable=False.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).  The
 * -ffp-contract=off flag matters: every fused multiply-add in this file is an
 * explicit fmaf(), exactly as in the device code.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

enum {
    ORC_ROW_OK = 0,
    ORC_ROW_BAD_HISTORY = 1,   /* history id outside [0, V) */
    ORC_ROW_BAD_PARAM = 2,     /* temperature is NaN */
    ORC_ROW_NONFINITE = 3,     /* a tempered logit is NaN, or the maximum is infinite */
    ORC_ROW_EMPTY_NUCLEUS = 4  /* top_p <= 0 removes every token */
};

#define ORC_MASS_BITS 44
#define ORC_MAX_V (1 << 19)

typedef struct {
    int32_t status;
    int32_t n_topk;     /* tokens left after top-k (all V when top-k is off) */
    int32_t n_kept;     /* tokens left after top-p */
    int32_t draw_pos;   /* position of the drawn token in the sorted kept list */
    uint64_t W;         /* total mass of the top-k survivors */
    uint64_t W_kept;    /* mass of the final kept set */
    uint64_t T_mass;    /* ceil(top_p * W), 0 when top-p is off */
    uint64_t D_mass;    /* floor(u * W_kept) */
    float m;            /* max tempered logit */
    float kth;          /* top-k threshold value (tempered), NaN when off */
    double p_margin;    /* min(T_mass - E_last, E_next - T_mass) / W; +inf when top-p off */
    double u_margin;    /* min(D_mass - E_draw, C_draw - D_mass) / W_kept */
} orc_info;

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* Order-preserving key: for non-NaN a < b  =>  okey(a) < okey(b). */
static inline uint32_t okey(float f)
{
    uint32_t u = f2u(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* Value key: like okey, but -0 and +0 (equal values) share one key. */
uint32_t orc_vkey(float f) { return okey(f == 0.0f ? 0.0f : f); }

/* Integer softmax numerator for d = fl32(l - m) <= 0.
 *   n = rint(d * log2(e)); r = d - n*ln2 (two fma, Cody-Waite split);
 *   q = 1 + r + r^2/2! + ... + r^7/7! (Horner with fma) in [0.70, 1.42];
 *   w = floor(q * 2^(44 + n)) = floor(P * 2^(20 + n)) with P = q * 2^24,
 *   an exact integer because q >= 0.5 has no bits below 2^-24. */
uint64_t orc_mass(float d)
{
    if (!(d >= -104.0f)) return 0;                 /* NaN, -inf, deep underflow */
    const float log2e = 0x1.715476p+0f;   /* fl32(log2 e) */
    const float ln2_hi = 0x1.62e4p-1f;    /* ln2 with its low 9 bits cleared */
    const float ln2_lo = 0x1.7f7d1cp-20f; /* fl32(ln2 - ln2_hi) */
    float t = d * log2e;
    float n = rintf(t);
    float r = fmaf(n, -ln2_hi, d);
    r = fmaf(n, -ln2_lo, r);
    float q = 0x1.a01a02p-13f;            /* fl32(1/5040) */
    q = fmaf(q, r, 0x1.6c16c2p-10f);      /* fl32(1/720)  */
    q = fmaf(q, r, 0x1.111112p-7f);       /* fl32(1/120)  */
    q = fmaf(q, r, 0x1.555556p-5f);       /* fl32(1/24)   */
    q = fmaf(q, r, 0x1.555556p-3f);       /* fl32(1/6)    */
    q = fmaf(q, r, 0.5f);
    q = fmaf(q, r, 1.0f);
    q = fmaf(q, r, 1.0f);
    uint32_t P = (uint32_t)(q * 16777216.0f);
    int s = (ORC_MASS_BITS - 24) + (int)n;
    if (s >= 0) return (uint64_t)P << s;
    if (s <= -26) return 0;
    return (uint64_t)(P >> (-s));
}

/* Split a finite fp32 in [0, 1) into M * 2^-sh with M < 2^24. */
static void split_unit(float v, uint32_t* M, int* sh)
{
    uint32_t b = f2u(v);
    uint32_t e = (b >> 23) & 0xFFu;
    uint32_t f = b & 0x7FFFFFu;
    if (e == 0) { *M = f; *sh = 149; }
    else        { *M = f | 0x800000u; *sh = 150 - (int)e; }
}

/* ceil(p * W) for 0 < p < 1, exact. */
uint64_t orc_ceil_mul(float p, uint64_t W)
{
    uint32_t M; int sh;
    split_unit(p, &M, &sh);
    u128 prod = (u128)M * W;
    if (prod == 0) return 0;
    if (sh >= 100) return 1;                       /* 0 < p*W < 2^-12 */
    u128 one = (u128)1 << sh;
    return (uint64_t)((prod + one - 1) >> sh);
}

/* floor(u * W) for 0 <= u < 1, exact. */
uint64_t orc_floor_mul(float u, uint64_t W)
{
    uint32_t M; int sh;
    split_unit(u, &M, &sh);
    u128 prod = (u128)M * W;
    if (sh >= 100) return 0;
    return (uint64_t)(prod >> sh);
}

/* Uniforms outside [0, 1) are clamped into it; NaN reads as 0. */
float orc_clamp_uniform(float u)
{
    if (!(u >= 0.0f)) return 0.0f;
    if (u >= 1.0f) return 0.99999994039535522461f;     /* largest float < 1 */
    return u;
}

static int cmp_u64(const void* a, const void* b)
{
    uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
    return (x > y) - (x < y);
}

/* torch.argmax semantics: first index of the maximum; a NaN is the maximum. */
static int64_t argmax_first(const float* x, int V)
{
    int64_t best = 0;
    float bv = x[0];
    for (int i = 1; i < V && !isnan(bv); ++i) {
        float v = x[i];
        if (isnan(v) || v > bv) { best = i; bv = v; }
    }
    return best;
}

typedef struct {
    float* x;        /* V: penalized logits */
    float* l;        /* V: tempered logits */
    uint64_t* ord;   /* V: sort keys, low 32 bits = index after sorting */
    uint64_t* w;     /* V: masses in sorted order */
    uint8_t* seen;   /* V: dedup flags for the penalty */
} row_scratch;

static int sample_row(const float* xin, int V, float T, int k, float p, float pen,
                      const int32_t* hist, int H, float u, int64_t* tok,
                      float* probs, orc_info* info, row_scratch* s)
{
    orc_info inf;
    memset(&inf, 0, sizeof inf);
    inf.kth = NAN;
    inf.p_margin = INFINITY;
    inf.u_margin = INFINITY;
    *tok = -1;
    if (probs) memset(probs, 0, sizeof(float) * (size_t)V);

    /* sampling.py:36 */
    memcpy(s->x, xin, sizeof(float) * (size_t)V);
    float* x = s->x;

    /* sampling.py:38-45: once per unique id (sorted(set(ids))) */
    if (pen != 1.0f && H > 0) {
        memset(s->seen, 0, (size_t)V);
        for (int h = 0; h < H; ++h) {
            int32_t id = hist[h];
            if (id < 0 || id >= V) { inf.status = ORC_ROW_BAD_HISTORY; goto done; }
            if (s->seen[id]) continue;
            s->seen[id] = 1;
            float v = x[id];
            x[id] = (v > 0.0f) ? v / pen : v * pen;
        }
    }

    /* sampling.py:47-48 */
    if (T == 0.0f) {
        *tok = argmax_first(x, V);
        inf.n_topk = inf.n_kept = 1;
        if (probs) probs[*tok] = 1.0f;
        goto done;
    }
    if (isnan(T)) { inf.status = ORC_ROW_BAD_PARAM; goto done; }

    /* sampling.py:50 */
    float* l = s->l;
    /* a NaN anywhere (a NaN logit, or an infinite one over an infinite T)
     * makes torch's softmax NaN throughout and multinomial reject the row,
     * whatever the NaN's sign bit (sampling.py:58, 68-69) */
    int any_nan = 0;
    for (int i = 0; i < V; ++i) { l[i] = x[i] / T; any_nan |= isnan(l[i]); }
    if (any_nan) { inf.status = ORC_ROW_NONFINITE; goto done; }

    /* sort by (value desc, index asc): ascending (~vkey, index) */
    uint64_t* ord = s->ord;
    for (int i = 0; i < V; ++i)
        ord[i] = ((uint64_t)(~orc_vkey(l[i])) << 32) | (uint32_t)i;
    qsort(ord, (size_t)V, sizeof(uint64_t), cmp_u64);
#define IDX(j) ((int)(uint32_t)ord[(j)])

    /* sampling.py:52-54 */
    int n1 = V;
    if (k > 0) {
        int kk = k < V ? k : V;
        float kth = l[IDX(kk - 1)];
        inf.kth = kth;
        n1 = kk;
        while (n1 < V && !(l[IDX(n1)] < kth)) ++n1;
    }
    inf.n_topk = n1;

    float m = l[IDX(0)];
    inf.m = m;
    if (!isfinite(m)) { inf.status = ORC_ROW_NONFINITE; goto done; }

    /* sampling.py:57-59: softmax numerators and their exact total */
    uint64_t* w = s->w;
    uint64_t W = 0;
    for (int j = 0; j < n1; ++j) { w[j] = orc_mass(l[IDX(j)] - m); W += w[j]; }
    inf.W = W;

    /* sampling.py:56, 60-66 */
    int nstar = n1;
    if (p < 1.0f) {
        if (!(p > 0.0f)) { inf.status = ORC_ROW_EMPTY_NUCLEUS; goto done; }
        uint64_t Tm = orc_ceil_mul(p, W);
        inf.T_mass = Tm;
        uint64_t E = 0;
        nstar = 0;
        while (nstar < n1 && E < Tm) { E += w[nstar]; ++nstar; }
        /* E is now the exclusive mass of position nstar (the first removed) */
        uint64_t E_last = E - w[nstar - 1];
        double lo = (double)(Tm - E_last);
        double hi = (nstar < n1) ? (double)(E - Tm) : INFINITY;
        inf.p_margin = (lo < hi ? lo : hi) / (double)W;
    }
    inf.n_kept = nstar;

    uint64_t Wk = 0;
    for (int j = 0; j < nstar; ++j) Wk += w[j];
    inf.W_kept = Wk;

    /* sampling.py:69 (inverse CDF in sorted order) */
    uint64_t D = orc_floor_mul(orc_clamp_uniform(u), Wk);
    inf.D_mass = D;
    uint64_t C = 0;
    int jd = 0;
    for (; jd < nstar; ++jd) {
        uint64_t Cn = C + w[jd];
        if (Cn > D) {
            double lo = (double)(D - C), hi = (double)(Cn - D);
            inf.u_margin = (lo < hi ? lo : hi) / (double)Wk;
            break;
        }
        C = Cn;
    }
    inf.draw_pos = jd;
    *tok = IDX(jd);

    /* sampling.py:68 */
    if (probs)
        for (int j = 0; j < nstar; ++j)
            probs[IDX(j)] = (float)((double)w[j] / (double)Wk);
#undef IDX

done:
    if (info) *info = inf;
    return inf.status;
}

/* Batched entry: row r reads x[r*ld .. r*ld+V) and history ids
 * hids[hoff[r] .. hoff[r+1]).  Error rows get token -1.  Returns the number
 * of error rows, or -1 for an invalid shape. */
int orc_sample(const float* x, int B, int V, int64_t ld,
               const float* T, const int32_t* k, const float* p, const float* pen,
               const int32_t* hoff, const int32_t* hids, const float* u,
               int64_t* out_tok, float* out_probs, int32_t* out_status,
               orc_info* info)
{
    if (B < 0 || V <= 0 || V > ORC_MAX_V || ld < V) return -1;
    int nerr = 0;
#pragma omp parallel reduction(+ : nerr)
    {
        row_scratch s;
        s.x = (float*)malloc(sizeof(float) * (size_t)V);
        s.l = (float*)malloc(sizeof(float) * (size_t)V);
        s.ord = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
        s.w = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
        s.seen = (uint8_t*)malloc((size_t)V);
#pragma omp for schedule(dynamic, 1)
        for (int r = 0; r < B; ++r) {
            int H = hoff ? hoff[r + 1] - hoff[r] : 0;
            const int32_t* hist = hoff ? hids + hoff[r] : NULL;
            int st = sample_row(x + (size_t)r * (size_t)ld, V, T[r], k[r], p[r], pen[r],
                                hist, H, u ? u[r] : 0.0f, &out_tok[r],
                                out_probs ? out_probs + (size_t)r * (size_t)V : NULL,
                                info ? &info[r] : NULL, &s);
            if (out_status) out_status[r] = st;
            if (st) ++nerr;
        }
        free(s.x); free(s.l); free(s.ord); free(s.w); free(s.seen);
    }
    return nerr;
}
