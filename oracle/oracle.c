/*
 * oracle.c -- CPU restatement of helix-lite's KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * Python drop-in packages) links, loads or calls this file.  It is the checker:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * nothing else may.
 *
 * Every function restates one piece of the reference's semantics and cites the
 * reference file:line it follows.  Arithmetic is plain IEEE binary32 in a fixed
 * order (compile with -O2 -fno-fast-math -ffp-contract=off) so results are
 * bit-reproducible and can be compared bit-for-bit with the GPU kernels.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   orc_nearest_code     -- known answer src/kvquant/tests/test_nuq_roundtrip.py:25-31,
 *                           torch.argmin (first-index-on-ties) over fp32 |v-p|,
 *                           brute force over all 65,536 fp16 inputs.
 *   orc_pack_k/_v        -- reference tests' outlier cases (test_nuq_roundtrip.py:34-39,65-75;
 *                           test_triton_kernels.py:120-129), torch restatement.
 *   orc_prep_table +
 *   orc_fast_eval        -- exhaustive equality with orc_nearest_code over all
 *                           65,536 fp16 inputs for random and adversarial tables.
 *   orc_page_stats       -- numpy amin/amax (value equality), test_reference.py:34-42.
 *   orc_page_bound       -- torch restatement within 4 ulp; bound >= true max
 *                           (test_reference.py:45-63); exact for one-hot queries.
 *   orc_topk_sinks       -- known answers test_reference.py:66-92, set validity,
 *                           torch.topk on distinct keys.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

float orc_h2f(uint16_t h)
{
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    float f;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else {
            f = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
            memcpy(&bits, &f, 4);
            bits |= s;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

/* float -> fp16, round to nearest even (the conversion `.to(tl.float16)` and
 * torch's `.to(torch.float16)` perform). */
uint16_t orc_f2h(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                        /* below 2^-14: subnormal */
        float a;
        memcpy(&a, &ax, 4);
        uint32_t m = (uint32_t)rintf(a * 16777216.0f);
        return (uint16_t)(sign | m);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

/* Signed ordered key of an fp16 bit pattern: increasing in value, -0 just
 * below +0, NaNs beyond +-inf. */
static inline int32_t hkey(uint16_t h)
{
    return (h & 0x8000u) ? -(int32_t)(h & 0x7fffu) - 1 : (int32_t)h;
}

static inline uint16_t hkey_inv(int32_t k)
{
    return k >= 0 ? (uint16_t)k : (uint16_t)(((-(k + 1)) & 0x7fff) | 0x8000);
}

/* --------------------------------------------------- a2: nearest pole */

/* Strict-'<' ascending scan over fp32 |v - pole|: the lowest level index wins
 * ties.  src/kvquant/triton_batched.py:65-72 (K5), :214-222 (K7),
 * src/kvquant/compact_pool.py:258-268 (K11), :198-205 (K10); the CPU spec
 * src/kvquant/nuq.py:36-37 (argmin returns the first minimum). */
int orc_nearest_code(float v, const float *poles, int L)
{
    float best = INFINITY;
    int idx = 0;
    for (int l = 0; l < L; l++) {
        float d = fabsf(v - poles[l]);
        if (d < best) {
            best = d;
            idx = l;
        }
    }
    return idx;
}

/* --------------------------------------- a3: dense-outlier pack (K, V) */

/* K per-channel pack, batched layout.  values (T,H,D) fp16 bits; poles
 * (H,D,L), upper/lower (H,D) upcast to fp32.  Outputs codes u8, outlier_v
 * fp16 (0 where not an outlier), outlier_m u8 -- all (T,H,D).
 * src/kvquant/triton_batched.py:28-82, wrapper :125-148. */
void orc_pack_k(const uint16_t *x, int64_t T, int H, int D, const float *poles,
                const float *upper, const float *lower, int L, uint8_t *codes,
                uint16_t *outv, uint8_t *outm)
{
    for (int64_t t = 0; t < T; t++)
        for (int h = 0; h < H; h++)
            for (int d = 0; d < D; d++) {
                int64_t i = (t * H + h) * D + d;
                int64_t s = (int64_t)h * D + d;
                float v = orc_h2f(x[i]);
                int o = (v > upper[s]) || (v < lower[s]);
                codes[i] = (uint8_t)orc_nearest_code(v, poles + s * L, L);
                outv[i] = o ? x[i] : 0;
                outm[i] = (uint8_t)o;
            }
}

/* V per-token pack.  poles (H,Tt,L), upper/lower (H,Tt).  Row t of head h uses
 * scale row min(pos[t], Tt-1) (pos == NULL means pos[t] = t).  With pos == NULL
 * and Tt == T this is src/kvquant/triton_batched.py:179-232 (caller-gathered
 * scales); with positions it is the pool's clamp, src/kvquant/compact_pool.py:
 * 467 and :190-205. */
void orc_pack_v(const uint16_t *x, int64_t T, int H, int D, const float *poles,
                const float *upper, const float *lower, int L, int64_t Tt,
                const int64_t *pos, uint8_t *codes, uint16_t *outv, uint8_t *outm)
{
    for (int64_t t = 0; t < T; t++) {
        int64_t r = pos ? pos[t] : t;
        if (r > Tt - 1) r = Tt - 1;
        if (r < 0) r = 0;
        for (int h = 0; h < H; h++) {
            int64_t s = (int64_t)h * Tt + r;
            for (int d = 0; d < D; d++) {
                int64_t i = (t * H + h) * D + d;
                float v = orc_h2f(x[i]);
                int o = (v > upper[s]) || (v < lower[s]);
                codes[i] = (uint8_t)orc_nearest_code(v, poles + s * L, L);
                outv[i] = o ? x[i] : 0;
                outm[i] = (uint8_t)o;
            }
        }
    }
}

/* ---------------------------------------------------- a6: dequantize */

/* where(outlier_m, outlier_v, fp16(pole[code])).  src/kvquant/triton_batched.py:
 * 85-122 (K6), :235-272 (K8); src/kvquant/nuq.py:155-156.  mode 0 = per-channel
 * table s = h*D+d, mode 1 = per-token table s = h*Tt + min(pos[t], Tt-1). */
void orc_unpack(const uint8_t *codes, const uint16_t *outv, const uint8_t *outm,
                int64_t T, int H, int D, const float *poles, int L, int mode,
                int64_t Tt, const int64_t *pos, uint16_t *out)
{
    for (int64_t t = 0; t < T; t++) {
        int64_t r = pos ? pos[t] : t;
        if (r > Tt - 1) r = Tt - 1;
        if (r < 0) r = 0;
        for (int h = 0; h < H; h++)
            for (int d = 0; d < D; d++) {
                int64_t i = (t * H + h) * D + d;
                int64_t s = mode == 0 ? (int64_t)h * D + d : (int64_t)h * Tt + r;
                /* a code without a level decodes to +0 (the reference's
                 * where-chain, src/kvquant/triton_batched.py:113-117) */
                out[i] = outm[i] ? outv[i]
                                 : (codes[i] >= L ? 0 : orc_f2h(poles[s * L + codes[i]]));
            }
    }
}

/* ------------------------------------ fast nearest-pole decision tables */

/* A decision table turns the L-level scan into a comparison against L-1
 * sorted fp16 breakpoints, valid for |x| <= xsafe.  The same construction runs
 * on the GPU; here it is restated so that the equivalence
 *     fast_eval(x) == orc_nearest_code(x)   for every fp16 x with |x| <= xsafe
 * can be checked exhaustively.  The construction is this build's own (the
 * reference always scans); see orc_prep_table for the argument. */
typedef struct {
    uint16_t bp[16];   /* bp[c-1]: smallest fp16 x with code(x) >= c; +inf if none */
    uint16_t pf16[16]; /* fp16(RNE) of each pole: the dequantised value of a code */
    uint16_t lo, up;   /* outlier iff x < lo || x > up (fp16 value compare) */
    uint16_t xsafe;    /* fast path valid iff |x| <= xsafe */
    uint16_t flags;    /* bit 0: fast path usable */
    uint16_t levels;
    uint16_t pad[3];
} orc_table; /* 80 bytes */

static float hval(int32_t k) { return orc_h2f(hkey_inv(k)); }

/* Smallest fp16 value (over -inf..+inf) that is >= t; NaN t -> -inf. */
static uint16_t h_ceil(float t)
{
    if (isnan(t)) return 0xfc00u;
    int32_t lo = hkey(0xfc00u), hi = hkey(0x7c00u); /* -inf, +inf */
    if (!(hval(hi) >= t)) return 0x7c00u;           /* unreachable for finite t */
    while (lo < hi) {
        int32_t mid = lo + (hi - lo) / 2;
        if (hval(mid) >= t) hi = mid; else lo = mid + 1;
    }
    return hkey_inv(lo);
}

/* Largest fp16 value (over -inf..+inf) that is <= t; NaN t -> +inf. */
static uint16_t h_floor(float t)
{
    if (isnan(t)) return 0x7c00u;
    int32_t lo = hkey(0xfc00u), hi = hkey(0x7c00u);
    if (!(hval(lo) <= t)) return 0xfc00u;
    while (lo < hi) {
        int32_t mid = hi - (hi - lo) / 2;
        if (hval(mid) <= t) lo = mid; else hi = mid - 1;
    }
    uint16_t r = hkey_inv(lo);
    return r == 0x8000u ? 0x0000u : r; /* a zero upper threshold is +0 */
}

/*
 * Build one decision table.  Correctness argument (checked exhaustively by the
 * tests): let the poles be finite and sorted, let delta be the smallest gap
 * between adjacent *distinct* pole values and 2^E <= delta.  For |x| <= xsafe
 * with xsafe + max|p| < 2^(E+23), every |x - p| < 2^(E+23), so its fp32
 * rounding error is below 2^(E-1) < delta/2.  A pole that is not one of the two
 * nearest distinct values is at least delta further away in exact arithmetic,
 * so it stays strictly worse after rounding; between the two nearest values
 * fl(x - p_lo) is non-decreasing and fl(p_hi - x) non-increasing in x.  Hence
 * the scan's code is a non-decreasing step function of x on [-xsafe, xsafe]
 * and equals the number of breakpoints <= x.
 */
void orc_prep_table(const float *p, int L, float upper, float lower, orc_table *t)
{
    memset(t, 0, sizeof(*t));
    t->levels = (uint16_t)L;
    for (int c = 0; c < 16; c++) t->bp[c] = 0x7c00u;
    for (int l = 0; l < L; l++) t->pf16[l] = orc_f2h(p[l]);
    t->lo = h_ceil(lower);
    if (t->lo == 0x0000u) t->lo = 0x8000u; /* a zero lower threshold is -0 */
    t->up = h_floor(upper);

    int ok = L >= 1 && L <= 16;
    double pmax = 0.0, delta = INFINITY;
    for (int l = 0; l < L && ok; l++) {
        if (!isfinite(p[l])) ok = 0;
        else {
            if (fabs((double)p[l]) > pmax) pmax = fabs((double)p[l]);
            if (l > 0) {
                if (p[l] < p[l - 1]) ok = 0;
                else if (p[l] > p[l - 1] && (double)p[l] - (double)p[l - 1] < delta)
                    delta = (double)p[l] - (double)p[l - 1];
            }
        }
    }
    double bound = 65504.0;
    if (ok && isfinite(delta)) {
        int E;
        frexp(delta, &E); /* delta = m * 2^E, m in [0.5,1) -> 2^(E-1) <= delta */
        double lim = ldexp(1.0, (E - 1) + 23) - pmax;
        if (lim < bound) bound = lim;
    }
    if (!ok || bound <= 0.0) {
        t->flags = 0;
        t->xsafe = 0;
        return;
    }
    /* largest fp16 strictly below bound (and <= 65504) */
    uint16_t xs = h_floor((float)bound);
    if ((xs & 0x8000u) || orc_h2f(xs) < 0.0f) { t->flags = 0; return; }
    while ((double)orc_h2f(xs) >= bound && xs > 0) xs--;
    if (xs >= 0x7c00u) xs = 0x7bffu;
    t->xsafe = xs;
    t->flags = 1;

    int32_t klo = hkey((uint16_t)(xs | 0x8000u)), khi = hkey(xs);
    for (int c = 1; c < L; c++) {
        if (orc_nearest_code(hval(khi), p, L) < c) {
            t->bp[c - 1] = 0x7c00u; /* never reached in the safe range */
            continue;
        }
        int32_t lo = klo, hi = khi;
        while (lo < hi) {
            int32_t mid = lo + (hi - lo) / 2;
            if (orc_nearest_code(hval(mid), p, L) >= c) hi = mid; else lo = mid + 1;
        }
        t->bp[c - 1] = hkey_inv(lo);
    }
}

void orc_prep_tables(const float *poles, const float *upper, const float *lower,
                     int64_t n, int L, orc_table *out)
{
    for (int64_t i = 0; i < n; i++)
        orc_prep_table(poles + i * L, L, upper[i], lower[i], out + i);
}

/* Fast-path evaluation as the GPU performs it.  Returns 1 and writes code and
 * outlier flag when the fast path applies to x, 0 when the caller must scan. */
int orc_fast_eval(uint16_t xb, const orc_table *t, int *code, int *outlier)
{
    if (!(t->flags & 1u)) return 0;
    if ((xb & 0x7fffu) > t->xsafe) return 0; /* also catches inf / NaN */
    float x = orc_h2f(xb);
    int c = 0;
    for (int i = 0; i + 1 < t->levels; i++) c += x >= orc_h2f(t->bp[i]);
    *code = c;
    *outlier = (x < orc_h2f(t->lo)) || (x > orc_h2f(t->up));
    return 1;
}

/* Exhaustive check of one table over all 65,536 fp16 inputs; returns the
 * number of inputs where the fast path applies but disagrees with the scan
 * (code or outlier flag), and the number of inputs it covers. */
int64_t orc_check_table_exhaustive(const float *p, int L, float upper, float lower,
                                   int64_t *covered)
{
    orc_table t;
    orc_prep_table(p, L, upper, lower, &t);
    int64_t bad = 0, cov = 0;
    for (uint32_t xb = 0; xb < 65536u; xb++) {
        int c, o;
        if (!orc_fast_eval((uint16_t)xb, &t, &c, &o)) continue;
        cov++;
        float v = orc_h2f((uint16_t)xb);
        int cr = orc_nearest_code(v, p, L);
        int orr = (v > upper) || (v < lower);
        if (c != cr || o != orr) bad++;
    }
    if (covered) *covered = cov;
    return bad;
}

/* ------------------------------------------------ a8: page statistics */

/* Total order used for min/max: -0 < +0; any NaN in a reduction yields NaN.
 * src/quest/reference.py:38-56 (amin/amax over the page-slot axis).  torch
 * leaves the choice between -0 and +0 unspecified; this build fixes it. */
static inline int32_t fkey(float f)
{
    int32_t b;
    memcpy(&b, &f, 4);
    return b >= 0 ? b : (int32_t)(b ^ 0x7fffffff);
}

/* K_pages (P,S,H,D) as fp32 values -> min/max (P,H,D) fp32. */
void orc_page_stats(const float *K, int64_t P, int S, int H, int D, float *kmin,
                    float *kmax)
{
    for (int64_t p = 0; p < P; p++)
        for (int h = 0; h < H; h++)
            for (int d = 0; d < D; d++) {
                float mn = K[((p * S) * H + h) * D + d], mx = mn;
                int nan = isnan(mn);
                for (int s = 1; s < S; s++) {
                    float v = K[((p * S + s) * H + h) * D + d];
                    if (isnan(v)) nan = 1;
                    if (fkey(v) < fkey(mn)) mn = v;
                    if (fkey(v) > fkey(mx)) mx = v;
                }
                if (nan) mn = mx = NAN;
                kmin[(p * H + h) * D + d] = mn;
                kmax[(p * H + h) * D + d] = mx;
            }
}

/* ------------------------------------------------ a9: upper bound */

static inline float clamp_pos(float q) { return q < 0.0f ? 0.0f : q; }  /* clamp(min=0) */
static inline float clamp_neg(float q) { return q > 0.0f ? 0.0f : q; }  /* clamp(max=0) */

/* Canonical fp32 evaluation order of one (page, head) bound: channels are cut
 * into chunks of 8; each chunk is summed left to right; the chunk sums (padded
 * with zeros to a power of two) are combined by a halving tree (chunk j with
 * chunk j + n/2, then j + n/4, ...).  The positive and negative halves are
 * summed separately and added last, as src/quest/reference.py:90-92 does.
 * Products are rounded before the add (no fused multiply-add). */
static float bound_one(const float *qp, const float *qn, const float *mn,
                       const float *mx, int D)
{
    float ps[64], ns[64];
    int nch = (D + 7) / 8, n2 = 1;
    while (n2 < nch) n2 <<= 1;
    for (int c = 0; c < n2; c++) {
        float a = 0.0f, b = 0.0f;
        for (int d = c * 8; d < c * 8 + 8 && d < D && c < nch; d++) {
            volatile float pa = qp[d] * mx[d];
            volatile float pb = qn[d] * mn[d];
            a = a + pa;
            b = b + pb;
        }
        ps[c] = a;
        ns[c] = b;
    }
    for (int off = n2 / 2; off >= 1; off /= 2)
        for (int c = 0; c < off; c++) {
            ps[c] = ps[c] + ps[c + off];
            ns[c] = ns[c] + ns[c + off];
        }
    float r = ps[0] + ns[0];
    return r + 0.0f; /* -0 -> +0 */
}

/* bound[p,h] = sum_d clamp(q,0)*Kmax + clamp(q,max=0)*Kmin.
 * src/quest/reference.py:59-93; fused form src/quest/triton_kernels.py:25-57.
 * q (H,D), Kmin/Kmax (P,H,D), all fp32 values; out (P,H) fp32. */
void orc_page_bound(const float *q, const float *kmin, const float *kmax, int64_t P,
                    int H, int D, float *out)
{
    float *qp = malloc(sizeof(float) * H * D), *qn = malloc(sizeof(float) * H * D);
    for (int i = 0; i < H * D; i++) {
        qp[i] = clamp_pos(q[i]);
        qn[i] = clamp_neg(q[i]);
    }
    for (int64_t p = 0; p < P; p++)
        for (int h = 0; h < H; h++)
            out[p * H + h] = bound_one(qp + h * D, qn + h * D, kmin + (p * H + h) * D,
                                       kmax + (p * H + h) * D, D);
    free(qp);
    free(qn);
}

/* GQA group-sum bound: the per-head bounds of the `group` query heads that
 * share KV head g, summed.  Evaluated in factorised form: Qp[d] = sum over the
 * group (ascending head order) of clamp(q,0), Qn likewise, then the canonical
 * single-head order above.  q (Hq,D) with Hq = Hkv*group; head h -> KV head
 * h / group.  (No reference counterpart: the reference averages the group's
 * queries, src/kvquant/compact_backend.py:225-231; the per-KV-head mode above
 * covers that path.) */
void orc_page_bound_group(const float *q, const float *kmin, const float *kmax,
                          int64_t P, int Hkv, int group, int D, float *out)
{
    float *qp = calloc((size_t)Hkv * D, sizeof(float));
    float *qn = calloc((size_t)Hkv * D, sizeof(float));
    for (int g = 0; g < Hkv; g++)
        for (int d = 0; d < D; d++) {
            float a = 0.0f, b = 0.0f;
            for (int j = 0; j < group; j++) {
                float v = q[(g * group + j) * D + d];
                a = a + clamp_pos(v);
                b = b + clamp_neg(v);
            }
            qp[g * D + d] = a;
            qn[g * D + d] = b;
        }
    for (int64_t p = 0; p < P; p++)
        for (int g = 0; g < Hkv; g++)
            out[p * Hkv + g] = bound_one(qp + g * D, qn + g * D, kmin + (p * Hkv + g) * D,
                                         kmax + (p * Hkv + g) * D, D);
    free(qp);
    free(qn);
}

/* ------------------------------------------------ a10: top-K + sinks */

/* Ordered key: NaN above +inf (torch.topk ranks NaN highest), -0 == +0. */
static inline uint32_t ukey(float f)
{
    if (isnan(f)) return 0xffffffffu;
    if (f == 0.0f) f = 0.0f;
    uint32_t b;
    memcpy(&b, &f, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

typedef struct { uint32_t key; int64_t idx; } kv_pair;

static int cmp_desc(const void *a, const void *b)
{
    const kv_pair *x = a, *y = b;
    if (x->key != y->key) return x->key > y->key ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

static int cmp_i64(const void *a, const void *b)
{
    int64_t x = *(const int64_t *)a, y = *(const int64_t *)b;
    return x < y ? -1 : (x > y);
}

/* src/quest/reference.py:96-133: sinks = min(sink_pages, P); k_eff =
 * min(k, P - sinks); the top k_eff non-sink pages per head plus the sinks,
 * sorted ascending.  Ties in the bound go to the lower page index (torch.topk
 * leaves this unspecified).  bound (P,H) fp32; out (sinks + k_eff, H) int64.
 * Returns sinks + k_eff. */
int64_t orc_topk_sinks(const float *bound, int64_t P, int H, int64_t k,
                       int64_t sink_pages, int64_t *out)
{
    int64_t s = sink_pages < 0 ? 0 : (sink_pages > P ? P : sink_pages);
    int64_t keff = k < 0 ? 0 : (k > P - s ? P - s : k);
    kv_pair *buf = malloc(sizeof(kv_pair) * (size_t)(P > 0 ? P : 1));
    int64_t *sel = malloc(sizeof(int64_t) * (size_t)(keff > 0 ? keff : 1));
    for (int h = 0; h < H; h++) {
        int64_t n = 0;
        for (int64_t p = s; p < P; p++) {
            buf[n].key = ukey(bound[p * H + h]);
            buf[n].idx = p;
            n++;
        }
        qsort(buf, (size_t)n, sizeof(kv_pair), cmp_desc);
        for (int64_t i = 0; i < keff; i++) sel[i] = buf[i].idx;
        qsort(sel, (size_t)keff, sizeof(int64_t), cmp_i64);
        for (int64_t i = 0; i < s; i++) out[i * H + h] = i;
        for (int64_t i = 0; i < keff; i++) out[(s + i) * H + h] = sel[i];
    }
    free(buf);
    free(sel);
    return s + keff;
}

/* Optimal 1-D k-means of n fp32 values into k clusters (the calibration fit
 * of the f4 row, solving the objective sklearn's KMeans approximates in
 * src/kvquant/calibration.py:106-123).  Dynamic programming over the sorted
 * values (Wang & Song 2011): D[0][i] = cost(0, i), D[m][i] = min over
 * m <= j <= i of D[m-1][j-1] + cost(j, i), with cost(j, i) the sum of squared
 * deviations of x[j..i] from their mean, from fp64 prefix sums.  Every
 * candidate j is tried (no monotone-argmin shortcut); D rows are rounded to
 * fp32, the leftmost minimum wins, rows m < k-1 cover i up to n-1-(k-1-m)
 * and the last row only i = n-1.  The prefix sums follow the device's order:
 * the sorted values cut into 256 chunks of ceil(n / 256), each chunk summed
 * in order from the sum of the earlier chunks' totals (themselves summed in
 * order).  centers: the clusters' means, fl32(fp64 sum / count), ascending.
 * n < k: the values and k - n zeros, sorted (calibration.py:116-119).
 * Returns 0, or -1 for n > 6144 (centres NaN). */
static int cmp_f32(const void *a, const void *b)
{
    float x = *(const float *)a, y = *(const float *)b;
    return (x > y) - (x < y);
}

int orc_kmeans_dp(const float *values, int64_t n64, int k, float *centers)
{
    if (n64 > 6144) {
        for (int l = 0; l < k; l++) centers[l] = NAN;
        return -1;
    }
    int n = (int)n64;
    float *x = malloc(sizeof(float) * (size_t)(n > k ? n : k));
    for (int i = 0; i < n; i++) x[i] = values[i];
    if (n < k) {
        for (int i = n; i < k; i++) x[i] = 0.0f;
        qsort(x, (size_t)k, sizeof(float), cmp_f32);
        for (int l = 0; l < k; l++) centers[l] = x[l];
        free(x);
        return 0;
    }
    qsort(x, (size_t)n, sizeof(float), cmp_f32);
    double *S1 = malloc(sizeof(double) * (size_t)(n + 1));
    double *S2 = malloc(sizeof(double) * (size_t)(n + 1));
    int per = (n + 255) / 256;
    double b1 = 0.0, b2 = 0.0;  /* totals of the earlier chunks */
    S1[0] = 0.0;
    S2[0] = 0.0;
    for (int t = 0; t < 256; t++) {
        int i0 = t * per, i1 = i0 + per < n ? i0 + per : n;
        double c1 = b1, c2 = b2, a1 = 0.0, a2 = 0.0;
        for (int i = i0; i < i1; i++) {
            double v = (double)x[i];
            c1 += v;
            c2 += v * v;
            a1 += v;
            a2 += v * v;
            S1[i + 1] = c1;
            S2[i + 1] = c2;
        }
        b1 += a1;
        b2 += a2;
    }
    float *Dp = malloc(sizeof(float) * (size_t)n), *Dc = malloc(sizeof(float) * (size_t)n);
    int *opt = malloc(sizeof(int) * (size_t)k * (size_t)n);
    for (int i = 0; i < n; i++) {
        double s = S1[i + 1], q = S2[i + 1];
        Dp[i] = (float)(q - s * s / (double)(i + 1));
    }
    int last = k - 1;
    for (int m = 1; m <= last; m++) {
        int ilo = m == last ? n - 1 : m, ihi = n - 1 - (last - m);
        for (int i = ilo; i <= ihi; i++) {
            double best = INFINITY;
            int bj = -1;
            for (int j = m; j <= i; j++) {
                double s = S1[i + 1] - S1[j], q = S2[i + 1] - S2[j];
                double c = (double)Dp[j - 1] + (q - s * s / (double)(i - j + 1));
                if (c < best) {
                    best = c;
                    bj = j;
                }
            }
            Dc[i] = (float)best;
            opt[(size_t)m * (size_t)n + (size_t)i] = bj;
        }
        float *t = Dp;
        Dp = Dc;
        Dc = t;
    }
    int i = n - 1;
    for (int m = last; m >= 1; m--) {
        int j = opt[(size_t)m * (size_t)n + (size_t)i];
        centers[m] = (float)((S1[i + 1] - S1[j]) / (double)(i - j + 1));
        i = j - 1;
    }
    centers[0] = (float)(S1[i + 1] / (double)(i + 1));
    free(x);
    free(S1);
    free(S2);
    free(Dp);
    free(Dc);
    free(opt);
    return 0;
}
