// detmath.h -- arithmetic that must give the same bits on the GPU as the
// CPU restatement of the sampling rule: exp from explicit IEEE fp32
// operations (no hardware transcendental), order-preserving float keys and
// the counter-based uniform generator.  Compiled with -ffp-contract=off.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ulspec {

// exp(x): Cody & Waite reduction x = n ln2 + r (ln2 split in a 16-bit head
// and a tail), degree-7 Taylor polynomial of e^r (error < r^8 / 8! < 2e-9
// relative on |r| <= ln2/2), 2^n applied as two normal factors.  x < -87
// gives 0 (every nonzero result is normal), x > 88.72 gives inf.
__host__ __device__ inline float det_expf(float x)
{
    if (!(x == x)) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.72f) return __builtin_inff();
    const float log2e = 1.44269504088896341f;
    const float shifter = 12582912.0f;  // 1.5 * 2^23: round to nearest even
    const float t = __builtin_fmaf(x, log2e, shifter);
    const float n = t - shifter;
    const float ln2_hi = 0.693145751953125f;
    const float ln2_lo = 1.428606820309417232e-06f;
    float r = __builtin_fmaf(-n, ln2_hi, x);
    r = __builtin_fmaf(-n, ln2_lo, r);
    float p = 1.98412698412698413e-04f;
    p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);
    p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);
    p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);
    p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int32_t ni = (int32_t)n;
    const int32_t n1 = ni / 2, n2 = ni - n1;
    const float s1 = __builtin_bit_cast(float, (uint32_t)(n1 + 127) << 23);
    const float s2 = __builtin_bit_cast(float, (uint32_t)(n2 + 127) << 23);
    return (p * s1) * s2;
}

// Larger key <=> larger float; -0.0 and +0.0 share a key (they compare equal).
__host__ __device__ inline uint32_t float_key(float f)
{
    uint32_t b = __builtin_bit_cast(uint32_t, f);
    if (b == 0x80000000u) b = 0u;
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__host__ __device__ inline float key_float(uint32_t k)
{
    const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __builtin_bit_cast(float, b);
}

// splitmix64 finalizer (Steele, Lea & Flood, OOPSLA 2014)
__host__ __device__ inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// u = top 24 bits of mix64(seed + (idx + 1) * golden) * 2^-24, in [0, 1)
__host__ __device__ inline float counter_uniform(uint64_t seed, uint64_t idx)
{
    return (float)(mix64(seed + (idx + 1u) * 0x9e3779b97f4a7c15ull) >> 40) * 0x1.0p-24f;
}

__host__ __device__ inline int bitlen64(uint64_t x)
{
    return x ? 64 - __builtin_clzll(x) : 0;
}

// fixed-point exponent S of the warp of a row of V tokens: E = trunc(e * 2^S)
__host__ __device__ inline int warp_shift(uint32_t V)
{
    return 63 - bitlen64(V);
}

}  // namespace ulspec
