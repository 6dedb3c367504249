/*
 * ora_common.c -- fp16 conversion, counter-based random numbers, the
 * deterministic exp.  Test infrastructure (see oracle.h).
 */
#include "ora_internal.h"

#include <math.h>
#include <string.h>

/* IEEE binary16 -> binary32, exact for every input (normals, subnormals,
 * +-0, +-inf, NaN).  Same semantics as half_to_float,
 * src/inference/inference_engine.cpp:15-37. */
float ora_h2f(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) & 1u;
    uint32_t e = (uint32_t)(h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    float f;
    if (e == 0) {
        f = ldexpf((float)m, -24);
    } else if (e == 31) {
        f = m ? NAN : INFINITY;
    } else {
        f = ldexpf((float)(m + 1024u), (int)e - 25);
    }
    return s ? -f : f;
}

/* binary32 -> binary16, round to nearest, ties to even. */
uint16_t ora_f2h(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) { /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    int32_t e = (int32_t)(ax >> 23) - 127;
    uint32_t mant = ax & 0x7fffffu;
    if (e >= -14) { /* normal half */
        uint32_t hm = mant >> 13;
        uint32_t rem = mant & 0x1fffu;
        uint32_t he = (uint32_t)(e + 15);
        uint32_t r = (he << 10) | hm;
        if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) r += 1u;
        return (uint16_t)(sign | r);
    }
    /* subnormal half: value = mant_full * 2^(e-23); half ulp = 2^-24 */
    if (e < -25) return (uint16_t)sign; /* < 2^-25 rounds to 0 (2^-25 exactly is a tie -> 0) */
    uint32_t full = mant | 0x800000u;
    /* value / 2^-24 = full * 2^(e + 1); e in [-25, -15] -> right shift 14..24 */
    int shift = -(e + 1);
    uint32_t q = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

void ora_h2f_array(const uint16_t* h, float* f, size_t n)
{
    for (size_t i = 0; i < n; ++i) f[i] = ora_h2f(h[i]);
}

void ora_f2h_array(const float* f, uint16_t* h, size_t n)
{
    for (size_t i = 0; i < n; ++i) h[i] = ora_f2h(f[i]);
}

/* splitmix64 finalizer (Steele, Lea & Flood, "Fast splittable pseudorandom
 * number generators", OOPSLA 2014). */
uint64_t ora_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static inline uint64_t ora_counter(uint64_t seed, uint64_t idx)
{
    return ora_mix64(seed + (idx + 1u) * 0x9e3779b97f4a7c15ull);
}

float ora_uniform(uint64_t seed, uint64_t idx)
{
    return (float)(ora_counter(seed, idx) >> 40) * 0x1.0p-24f;
}

void ora_uniforms(uint64_t seed, uint64_t idx0, size_t n, float* out)
{
    for (size_t i = 0; i < n; ++i) out[i] = ora_uniform(seed, idx0 + i);
}

/* Normal pair i of stream s: u1, u2 from counters (2i, 2i+1) of the seed
 * mix64(seed ^ mix64(stream)); 53-bit uniforms in (0, 1]; Box-Muller in
 * double; fp32 output = (float)(mean + std * z). */
typedef struct {
    uint64_t key;
    size_t n;      /* one past the last normal index to write */
    size_t base;   /* normal index written to out[0] */
    double mean, std;
    float* out;
} normal_job;

static void normal_range(void* arg, int64_t lo, int64_t hi)
{
    normal_job* j = (normal_job*)arg;
    for (int64_t p = lo; p < hi; ++p) {
        uint64_t a = ora_counter(j->key, 2u * (uint64_t)p);
        uint64_t b = ora_counter(j->key, 2u * (uint64_t)p + 1u);
        double u1 = (double)((a >> 11) + 1u) * 0x1.0p-53; /* (0, 1] */
        double u2 = (double)(b >> 11) * 0x1.0p-53;        /* [0, 1) */
        double r = sqrt(-2.0 * log(u1));
        double t = 6.283185307179586476925286766559 * u2;
        size_t i0 = 2u * (size_t)p;
        if (i0 >= j->base) j->out[i0 - j->base] = (float)(j->mean + j->std * r * cos(t));
        if (i0 + 1u < j->n && i0 + 1u >= j->base) j->out[i0 + 1u - j->base] = (float)(j->mean + j->std * r * sin(t));
    }
}

static uint64_t normal_key(uint64_t seed, uint64_t stream)
{
    return ora_mix64(seed ^ ora_mix64(stream + 0x632be59bd9b4e019ull));
}

void ora_normals(uint64_t seed, uint64_t stream, size_t n, double mean, double std, float* out, int nthreads)
{
    normal_job j = { normal_key(seed, stream), n, 0, mean, std, out };
    ora_parallel_for(nthreads, (int64_t)((n + 1u) / 2u), normal_range, &j);
}

/* Normals i0 .. i0+n-1 of the stream, single thread. */
void ora_normals_range(uint64_t seed, uint64_t stream, uint64_t i0, size_t n, double mean, double std, float* out)
{
    normal_job j = { normal_key(seed, stream), n + (size_t)i0, (size_t)i0, mean, std, out };
    normal_range(&j, (int64_t)(i0 / 2u), (int64_t)((i0 + n + 1u) / 2u));
}

/* exp(x) for float x, the same sequence of IEEE fp32 operations as the
 * device's expf in universal-loader_amd/csrc/detmath.h, so the two agree bit
 * for bit.  Cody & Waite range reduction (x = n ln2 + r, |r| <= ln2/2, ln2
 * split in a 16-bit head and a tail), degree-7 Taylor polynomial of e^r
 * (truncation error < r^8/8! < 2e-9 relative), scaling by 2^n through the
 * exponent bits.  Inputs below -87 give 0 (so every nonzero result is a
 * normal float); above 88.72 give inf. */
float ora_expf(float x)
{
    if (!(x == x)) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.72f) return INFINITY;
    const float log2e = 1.44269504088896341f;
    const float shifter = 12582912.0f; /* 1.5 * 2^23: round-to-nearest-even trick */
    float t = fmaf(x, log2e, shifter);
    float n = t - shifter;
    const float ln2_hi = 0.693145751953125f;      /* 16 significant bits */
    const float ln2_lo = 1.428606820309417232e-06f; /* ln2 - ln2_hi */
    float r = fmaf(-n, ln2_hi, x);
    r = fmaf(-n, ln2_lo, r);
    float p = 1.98412698412698413e-04f;           /* 1/7! */
    p = fmaf(p, r, 1.38888888888888889e-03f);     /* 1/6! */
    p = fmaf(p, r, 8.33333333333333333e-03f);     /* 1/5! */
    p = fmaf(p, r, 4.16666666666666667e-02f);     /* 1/4! */
    p = fmaf(p, r, 1.66666666666666667e-01f);     /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int32_t ni = (int32_t)n;
    /* 2^n as two normal factors (n in [-126, 128]) */
    int32_t n1 = ni / 2;
    int32_t n2 = ni - n1;
    uint32_t b1 = (uint32_t)(n1 + 127) << 23;
    uint32_t b2 = (uint32_t)(n2 + 127) << 23;
    float s1, s2;
    memcpy(&s1, &b1, 4);
    memcpy(&s2, &b2, 4);
    return (p * s1) * s2;
}
