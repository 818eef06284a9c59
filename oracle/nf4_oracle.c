/*
 * C restatement of the NF4 blockwise quantize / pack / dequantize path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the timed CPU
 * baseline ("port") of bench.py. The product library never links this file.
 *
 * Follows the published bitsandbytes algorithm that the reference reaches at
 *   quantize:   stratum/upload.py:367-369 and :725-727 (CPU tensor, 2-D view)
 *   dequantize: stratum/upload.py:221, :946, :1038 and stratum/nf4_linear.py:46
 * It is written in a different form from oracle/nf4_oracle.py on purpose so the
 * two cross-check each other: a literal 16-way first-minimum scan for the
 * "argmin" rule and a literal binary comparison tree for the "threshold" rule.
 *
 * Build: make -C oracle   (gcc -O2 -fopenmp -ffp-contract=off, no fast-math)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };
enum { R_ARGMIN = 0, R_THRESHOLD = 1 };

static const float kCode[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f, 0.33791524171829224f,
    0.44070982933044434f, 0.5626170039176941f, 0.7229568362236023f, 1.0f};

/* fp32 midpoints of adjacent levels, computed in double then rounded once */
static float mid(int i) { return (float)(((double)kCode[i] + (double)kCode[i + 1]) * 0.5); }

static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { /* subnormal: value = m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* round-to-nearest-even fp32 -> fp16 */
static uint16_t f32_to_f16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);     /* NaN */
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);    /* rounds to inf */
    if (a < 0x38800000u) {                                      /* fp16 subnormal or zero */
        /* value / 2^-24, rounded to nearest even integer */
        float v;
        memcpy(&v, &a, 4);
        double q = (double)v * 16777216.0; /* exact */
        double fl = floor(q);
        double r = q - fl;
        uint32_t m = (uint32_t)fl;
        if (r > 0.5 || (r == 0.5 && (m & 1u))) m++;
        return (uint16_t)(sign | m);
    }
    uint32_t e = ((a >> 23) - 112u) << 10;
    uint32_t m = (a >> 13) & 0x3FFu;
    uint32_t rest = a & 0x1FFFu;
    uint32_t h = e | m;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

static float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static float load(const void* x, int dt, int64_t i) {
    if (dt == DT_F16) return f16_to_f32(((const uint16_t*)x)[i]);
    if (dt == DT_BF16) return bf16_to_f32(((const uint16_t*)x)[i]);
    return ((const float*)x)[i];
}

static int code_argmin(float s) {
    /* torch.clamp then argmin over fp32 |s - code|, first minimum wins */
    if (s != s) return 0;
    if (s < -1.0f) s = -1.0f;
    if (s > 1.0f) s = 1.0f;
    int best = 0;
    float bd = fabsf(s - kCode[0]);
    for (int j = 1; j < 16; ++j) {
        float d = fabsf(s - kCode[j]);
        if (d < bd) {
            bd = d;
            best = j;
        }
    }
    return best;
}

static int code_tree(float s) {
    /* binary comparison tree on fp32 midpoints, strict '>'; NaN walks to 0 */
    int lo = 0, hi = 15; /* code in [lo, hi] */
    while (lo < hi) {
        int m = (lo + hi) >> 1; /* threshold between code m and m+1 */
        if (s > mid(m))
            lo = m + 1;
        else
            hi = m;
    }
    return lo;
}

int nf4o_code(float s, int rounding) { return rounding == R_ARGMIN ? code_argmin(s) : code_tree(s); }

void nf4o_quantize(const void* x, int dt, int64_t n, int bs, int rounding, uint8_t* packed, float* absmax,
                   int nthreads) {
    int64_t nb = (n + bs - 1) / bs;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t b = 0; b < nb; ++b) {
        int64_t lo = b * bs, hi = lo + bs < n ? lo + bs : n;
        float a = 0.0f;
        for (int64_t i = lo; i < hi; ++i) {
            float v = fabsf(load(x, dt, i));
            if (v > a || v != v) a = (a != a) ? a : v; /* NaN sticks */
        }
        absmax[b] = a;
        float inv = 1.0f / a;
        for (int64_t i = lo; i < hi; i += 2) {
            int q0 = nf4o_code(load(x, dt, i) * inv, rounding);
            int q1 = (i + 1 < hi) ? nf4o_code(load(x, dt, i + 1) * inv, rounding) : 0;
            packed[i >> 1] = (uint8_t)((q0 << 4) | q1);
        }
    }
}

void nf4o_dequantize(const uint8_t* packed, const float* absmax, int64_t n, int bs, void* out, int out_dt,
                     int nthreads) {
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (int64_t i = 0; i < n; ++i) {
        uint8_t byte = packed[i >> 1];
        int q = (i & 1) ? (byte & 0x0F) : (byte >> 4);
        float v = kCode[q] * absmax[i / bs];
        if (out_dt == DT_F16)
            ((uint16_t*)out)[i] = f32_to_f16(v);
        else if (out_dt == DT_BF16)
            ((uint16_t*)out)[i] = f32_to_bf16(v);
        else
            ((float*)out)[i] = v;
    }
}

/*
 * Exhaustive check of a cell table of the form used by the product kernels:
 * for every fp32 s in [-1, 1] (and NaN, +-inf, values just outside), the code
 *   c = clamp(s) ; f = fma(c, 32, 2^21 + 32) ; j = (bits(f) & 0x3FC) >> 2 ;
 *   code = base[j] + (c >= bound[j])
 * must equal nf4o_code(s, rounding). (f lies in [2^21, 2^22), where the float
 * spacing is 1/4, so bits(f) & 0x3FC is 4 * floor(round(128 c + 128) / 4).)
 * Returns the number of mismatches and writes the first mismatching bit
 * pattern to *first_bad.
 */
static int cell_index(float c) {
    float f = fmaf(c, 32.0f, 2097184.0f);
    uint32_t u;
    memcpy(&u, &f, 4);
    return (int)((u & 0x3FCu) >> 2);
}

int64_t nf4o_check_cells(const float* bound, const uint8_t* base, int ncell, int rounding, uint32_t* first_bad) {
    int64_t bad = 0;
    uint32_t first = 0;
    const uint32_t one = 0x3F800000u;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) reduction(+ : bad)
#endif
    for (int64_t k = 0; k <= (int64_t)one + 16; ++k) {
        for (int sgn = 0; sgn < 2; ++sgn) {
            uint32_t u = (uint32_t)k | (sgn ? 0x80000000u : 0u);
            float s;
            memcpy(&s, &u, 4);
            float c = s != s ? -1.0f : (s < -1.0f ? -1.0f : (s > 1.0f ? 1.0f : s));
            int j = cell_index(c);
            if (j < 0 || j >= ncell) {
                bad++;
                continue;
            }
            int got = base[j] + (c >= bound[j] ? 1 : 0);
            if (got != nf4o_code(s, rounding)) {
                bad++;
#ifdef _OPENMP
#pragma omp critical
#endif
                {
                    if (first == 0) first = u;
                }
            }
        }
    }
    /* NaN and infinities */
    const uint32_t specials[3] = {0x7FC00000u, 0x7F800000u, 0xFF800000u};
    for (int t = 0; t < 3; ++t) {
        float s;
        memcpy(&s, &specials[t], 4);
        float c = s != s ? -1.0f : (s < -1.0f ? -1.0f : (s > 1.0f ? 1.0f : s));
        int j = cell_index(c);
        int got = base[j] + (c >= bound[j] ? 1 : 0);
        if (got != nf4o_code(s, rounding)) bad++;
    }
    if (first_bad) *first_bad = first;
    return bad;
}
