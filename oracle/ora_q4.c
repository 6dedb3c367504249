/*
 * ora_q4.c -- GGUF Q4_0 / Q4_K blocks and the verify dequant-GEMM on the CPU.
 * Test infrastructure (see oracle.h).
 *
 * Block formats (public GGUF definition; type ids and elements per block as in
 * src/core/gguf_types.h:6-33,60-81, byte sizes corrected from the 6 / 12 of
 * gguf_types.h:39,47 to the GGUF 18 / 144):
 *   Q4_0 (type 2), 32 elements, 18 B: { fp16 d; u8 qs[16]; }
 *        x[j] = ((qs[j] & 15) - 8) * d,  x[j+16] = ((qs[j] >> 4) - 8) * d,  j < 16
 *   Q4_K (type 12), 256 elements, 144 B: { fp16 d; fp16 dmin; u8 scales[12]; u8 qs[128]; }
 *        (offsets as read in src/inference/inference_engine.cpp:900-921)
 *        sub-block j (32 elements) has 6-bit (sc_j, m_j):
 *          j < 4: sc = scales[j] & 63, m = scales[j+4] & 63
 *          j >= 4: sc = (scales[j+4] & 15) | ((scales[j-4] >> 6) << 4),
 *                  m  = (scales[j+4] >> 4) | ((scales[j] >> 6) << 4)
 *        chunk c < 4 uses qs[32c .. 32c+31]: element 64c+l = d*sc_{2c}*(qs[32c+l] & 15) - dmin*m_{2c},
 *        element 64c+32+l = d*sc_{2c+1}*(qs[32c+l] >> 4) - dmin*m_{2c+1}.
 * Types real Q4_K_M files mix in (ggml's published block layouts; the
 * reference's own dequantize_q6_k.glsl / dequantize_q8_0.glsl do not read the
 * GGUF bytes, src/core/gguf_types.h:43,49 has wrong sizes for them):
 *   F16  (type 1), 1 element, 2 B: IEEE half.
 *   Q8_0 (type 8), 32 elements, 34 B: { fp16 d; i8 qs[32]; }   x[j] = d * qs[j]
 *   Q6_K (type 14), 256 elements, 210 B: { u8 ql[128]; u8 qh[64]; i8 scales[16]; fp16 d; }
 *        for half h < 2 (elements 128h ..), ql += 64h, qh += 32h, sc = scales + 8h, l < 32:
 *          q1 = ((ql[l]    & 15) | (((qh[l] >> 0) & 3) << 4)) - 32 -> element 128h + l,      scale sc[l/16]
 *          q2 = ((ql[l+32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32 -> element 128h + 32 + l, scale sc[l/16 + 2]
 *          q3 = ((ql[l]    >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32 -> element 128h + 64 + l, scale sc[l/16 + 4]
 *          q4 = ((ql[l+32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32 -> element 128h + 96 + l, scale sc[l/16 + 6]
 *        x = d * scale * q.
 *   ggml itself (its ggml-quants.c dequantize_row_q8_0 / _q6_K) is neither in
 *   the reference tree nor in this image, and no GGUF fixture holding these
 *   types exists here: the Q8_0 / Q6_K element order is pinned by closed forms
 *   of the layout above (scale groups, the byte and bit behind each element),
 *   not against an independent decoder -- parity unpinned against ggml.
 */
#include "ora_internal.h"

#include <immintrin.h>
#include <math.h>
#include <string.h>

int ora_blck_size(int type)
{
    switch (type) {
    case ORA_F16: return 1;
    case ORA_Q4_0: case ORA_Q8_0: return 32;
    case ORA_Q4_K: case ORA_Q6_K: return 256;
    default: return 0;
    }
}

int ora_type_size(int type)
{
    switch (type) {
    case ORA_F16: return 2;
    case ORA_Q4_0: return 18;
    case ORA_Q8_0: return 34;
    case ORA_Q4_K: return 144;
    case ORA_Q6_K: return 210;
    default: return 0;
    }
}

size_t ora_row_bytes(int type, int64_t k)
{
    int bs = ora_blck_size(type);
    if (bs == 0 || k % bs) return 0;
    return (size_t)(k / bs) * (size_t)ora_type_size(type);
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* Q4_0 quantizer: the element of largest magnitude keeps its sign (max),
 * d = max / -8, q = min(15, (int)(x / d + 8.5)), d stored as fp16. */
static void quant_block_q4_0(const float* x, uint8_t* blk)
{
    float amax = 0.0f, vmax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        float a = fabsf(x[j]);
        if (a > amax) { amax = a; vmax = x[j]; }
    }
    float d = vmax / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    wr16(blk, ora_f2h(d));
    for (int j = 0; j < 16; ++j) {
        int q0 = (int)(x[j] * id + 8.5f);
        int q1 = (int)(x[j + 16] * id + 8.5f);
        if (q0 > 15) q0 = 15;
        if (q1 > 15) q1 = 15;
        if (q0 < 0) q0 = 0;
        if (q1 < 0) q1 = 0;
        blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

static void dequant_block_q4_0(const uint8_t* blk, float* y)
{
    float d = ora_h2f(rd16(blk));
    for (int j = 0; j < 16; ++j) {
        y[j] = (float)((blk[2 + j] & 15) - 8) * d;
        y[j + 16] = (float)((blk[2 + j] >> 4) - 8) * d;
    }
}

void ora_q4k_scale_min(const uint8_t* scales, int j, int* sc, int* m)
{
    if (j < 4) {
        *sc = scales[j] & 63;
        *m = scales[j + 4] & 63;
    } else {
        *sc = (scales[j + 4] & 15) | ((scales[j - 4] >> 6) << 4);
        *m = (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4);
    }
}

/* Q4_K quantizer (a simple affine one; any quantizer is valid because the
 * GPU and the CPU read the same bytes): per sub-block scale = (max - min)/15
 * with min clamped to <= 0, m = -min; d = max scale / 63, dmin = max m / 63
 * (fp16); 6-bit sc = round(scale / d), m6 = round(m / dmin);
 * q = round((x + dmin*m6) / (d*sc)) clamped to [0, 15]. */
static void quant_block_q4_k(const float* x, uint8_t* blk)
{
    float scale[8], mins[8];
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; ++j) {
        float mn = 0.0f, mx = x[32 * j];
        for (int l = 0; l < 32; ++l) {
            float v = x[32 * j + l];
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        if (mx < mn) mx = mn;
        scale[j] = (mx - mn) / 15.0f;
        mins[j] = -mn;
        if (scale[j] > max_scale) max_scale = scale[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    uint16_t d16 = ora_f2h(max_scale / 63.0f);
    uint16_t m16 = ora_f2h(max_min / 63.0f);
    float dq = ora_h2f(d16), mq = ora_h2f(m16);
    int sc[8], mm[8];
    for (int j = 0; j < 8; ++j) {
        int a = dq > 0.0f ? (int)(scale[j] / dq + 0.5f) : 0;
        int b = mq > 0.0f ? (int)(mins[j] / mq + 0.5f) : 0;
        sc[j] = a > 63 ? 63 : a;
        mm[j] = b > 63 ? 63 : b;
    }
    wr16(blk, d16);
    wr16(blk + 2, m16);
    uint8_t* s = blk + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mm[j] & 63) | ((mm[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mm[j + 4] & 15) << 4));
    }
    uint8_t q[256];
    for (int j = 0; j < 8; ++j) {
        float es = dq * (float)sc[j];
        float em = mq * (float)mm[j];
        for (int l = 0; l < 32; ++l) {
            int v = es > 0.0f ? (int)((x[32 * j + l] + em) / es + 0.5f) : 0;
            q[32 * j + l] = (uint8_t)(v < 0 ? 0 : v > 15 ? 15 : v);
        }
    }
    uint8_t* qs = blk + 16;
    for (int c = 0; c < 4; ++c)
        for (int l = 0; l < 32; ++l)
            qs[32 * c + l] = (uint8_t)(q[64 * c + l] | (q[64 * c + 32 + l] << 4));
}

static void dequant_block_q4_k(const uint8_t* blk, float* y)
{
    float d = ora_h2f(rd16(blk));
    float dmin = ora_h2f(rd16(blk + 2));
    const uint8_t* qs = blk + 16;
    for (int c = 0; c < 4; ++c) {
        int sc0, m0, sc1, m1;
        ora_q4k_scale_min(blk + 4, 2 * c, &sc0, &m0);
        ora_q4k_scale_min(blk + 4, 2 * c + 1, &sc1, &m1);
        float d0 = d * (float)sc0, mn0 = dmin * (float)m0;
        float d1 = d * (float)sc1, mn1 = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) {
            y[64 * c + l] = d0 * (float)(qs[32 * c + l] & 15) - mn0;
            y[64 * c + 32 + l] = d1 * (float)(qs[32 * c + l] >> 4) - mn1;
        }
    }
}

static void dequant_block_q8_0(const uint8_t* blk, float* y)
{
    float d = ora_h2f(rd16(blk));
    for (int j = 0; j < 32; ++j) y[j] = d * (float)(int8_t)blk[2 + j];
}

static void dequant_block_q6_k(const uint8_t* blk, float* y)
{
    const float d = ora_h2f(rd16(blk + 208));
    for (int h = 0; h < 2; ++h) {
        const uint8_t* ql = blk + 64 * h;
        const uint8_t* qh = blk + 128 + 32 * h;
        const int8_t* sc = (const int8_t*)(blk + 192 + 8 * h);
        float* yy = y + 128 * h;
        for (int l = 0; l < 32; ++l) {
            const int is = l / 16;
            const int q1 = ((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = ((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            yy[l] = d * (float)sc[is] * (float)q1;
            yy[l + 32] = d * (float)sc[is + 2] * (float)q2;
            yy[l + 64] = d * (float)sc[is + 4] * (float)q3;
            yy[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
    }
}

/* Q8_0 quantizer: d = amax / 127, q = round-half-away(x / d), d stored as fp16. */
static void quant_block_q8_0(const float* x, uint8_t* blk)
{
    float amax = 0.0f;
    for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    wr16(blk, ora_f2h(d));
    for (int j = 0; j < 32; ++j) {
        int q = (int)roundf(x[j] * id);
        blk[2 + j] = (uint8_t)(int8_t)(q > 127 ? 127 : (q < -127 ? -127 : q));
    }
}

/* Q6_K quantizer (simple, for synthetic tensors): per 16-element group g the
 * scale s_g = amax_g / 31; d = max_g s_g / 127, sc_g = round(s_g / d)
 * (int8, <= 127); q = clamp(round(x / (d sc_g)), -32, 31) + 32 split into
 * ql / qh by the layout above; d stored as fp16. */
static void quant_block_q6_k(const float* x, uint8_t* blk)
{
    float s[16], smax = 0.0f;
    for (int g = 0; g < 16; ++g) {
        float amax = 0.0f;
        for (int l = 0; l < 16; ++l) amax = fmaxf(amax, fabsf(x[16 * g + l]));
        s[g] = amax / 31.0f;
        smax = fmaxf(smax, s[g]);
    }
    float d = smax / 127.0f;
    uint16_t dh = ora_f2h(d);
    float dq = ora_h2f(dh);
    memset(blk, 0, 210);
    int8_t sc[16];
    for (int g = 0; g < 16; ++g) {
        int v = dq != 0.0f ? (int)roundf(s[g] / dq) : 0;
        sc[g] = (int8_t)(v > 127 ? 127 : v);
        blk[192 + g] = (uint8_t)sc[g];
    }
    wr16(blk + 208, dh);
    for (int e = 0; e < 256; ++e) {
        const int g = e / 16;
        const float step = dq * (float)sc[g];
        int q = step != 0.0f ? (int)roundf(x[e] / step) : 0;
        q = (q > 31 ? 31 : (q < -32 ? -32 : q)) + 32;
        /* element e: half h, position within the half p = e % 128 -> (quarter, l) */
        const int h = e / 128, p = e % 128, quarter = p / 32, l = p % 32;
        uint8_t* ql = blk + 64 * h;
        uint8_t* qh = blk + 128 + 32 * h;
        const int lo = q & 15, hi = q >> 4;
        if (quarter == 0) { ql[l] |= (uint8_t)lo; qh[l] |= (uint8_t)(hi << 0); }
        if (quarter == 1) { ql[l + 32] |= (uint8_t)lo; qh[l] |= (uint8_t)(hi << 2); }
        if (quarter == 2) { ql[l] |= (uint8_t)(lo << 4); qh[l] |= (uint8_t)(hi << 4); }
        if (quarter == 3) { ql[l + 32] |= (uint8_t)(lo << 4); qh[l] |= (uint8_t)(hi << 6); }
    }
}

static void quant_block(int type, const float* x, uint8_t* blk)
{
    switch (type) {
    case ORA_F16: wr16(blk, ora_f2h(x[0])); break;
    case ORA_Q4_0: quant_block_q4_0(x, blk); break;
    case ORA_Q8_0: quant_block_q8_0(x, blk); break;
    case ORA_Q4_K: quant_block_q4_k(x, blk); break;
    default: quant_block_q6_k(x, blk); break;
    }
}

static void dequant_block(int type, const uint8_t* blk, float* y)
{
    switch (type) {
    case ORA_F16: y[0] = ora_h2f(rd16(blk)); break;
    case ORA_Q4_0: dequant_block_q4_0(blk, y); break;
    case ORA_Q8_0: dequant_block_q8_0(blk, y); break;
    case ORA_Q4_K: dequant_block_q4_k(blk, y); break;
    default: dequant_block_q6_k(blk, y); break;
    }
}

int ora_quantize(int type, const float* x, int64_t n, uint8_t* out)
{
    int bs = ora_blck_size(type);
    if (bs == 0 || n % bs) return -1;
    int ts = ora_type_size(type);
    for (int64_t b = 0; b < n / bs; ++b) quant_block(type, x + b * bs, out + b * ts);
    return 0;
}

int ora_dequantize(int type, const uint8_t* in, int64_t n, float* out)
{
    int bs = ora_blck_size(type);
    if (bs == 0 || n % bs) return -1;
    int ts = ora_type_size(type);
    for (int64_t b = 0; b < n / bs; ++b) dequant_block(type, in + b * ts, out + b * bs);
    return 0;
}

/* ---- synthetic weights ---------------------------------------------------- */
typedef struct {
    int type;
    uint64_t seed, stream;
    int64_t K;
    double std;
    uint8_t* out;
} synth_job;

static void synth_rows(void* arg, int64_t lo, int64_t hi)
{
    synth_job* j = (synth_job*)arg;
    float* row = (float*)malloc(sizeof(float) * (size_t)j->K);
    size_t rb = ora_row_bytes(j->type, j->K);
    for (int64_t n = lo; n < hi; ++n) {
        /* element (n, k) is normal number n*K + k of stream (seed, stream) */
        ora_normals_range(j->seed, j->stream, (uint64_t)(n * j->K), (size_t)j->K, 0.0, j->std, row);
        ora_quantize(j->type, row, j->K, j->out + (size_t)n * rb);
    }
    free(row);
}

int ora_synth_q4(int type, uint64_t seed, uint64_t stream, int64_t N, int64_t K, double std,
                 uint8_t* out, int nthreads)
{
    if (ora_row_bytes(type, K) == 0 || N <= 0) return -1;
    synth_job j = { type, seed, stream, K, std, out };
    ora_parallel_for(nthreads, N, synth_rows, &j);
    return 0;
}

/* ---- float64 dequant-GEMM (pinning reference) ----------------------------- */
int ora_q4_gemm_f64(int type, const uint8_t* W, int64_t N, int64_t K,
                    const uint16_t* X, int64_t M, double* Y)
{
    size_t rb = ora_row_bytes(type, K);
    if (rb == 0 || N <= 0 || M <= 0) return -1;
    int bs = ora_blck_size(type), ts = ora_type_size(type);
    double* w = (double*)malloc(sizeof(double) * (size_t)K);
    double* x = (double*)malloc(sizeof(double) * (size_t)(M * K));
    for (int64_t i = 0; i < M * K; ++i) x[i] = (double)ora_h2f(X[i]);
    for (int64_t n = 0; n < N; ++n) {
        const uint8_t* row = W + (size_t)n * rb;
        for (int64_t b = 0; b < K / bs; ++b) {
            const uint8_t* blk = row + b * ts;
            double* wb = w + b * bs;
            if (type == ORA_F16) {
                wb[0] = (double)ora_h2f(rd16(blk));
            } else if (type == ORA_Q8_0) {
                double d = (double)ora_h2f(rd16(blk));
                for (int j = 0; j < 32; ++j) wb[j] = d * (double)(int8_t)blk[2 + j];
            } else if (type == ORA_Q6_K) {
                double d = (double)ora_h2f(rd16(blk + 208));
                for (int h = 0; h < 2; ++h) {
                    const uint8_t* ql = blk + 64 * h;
                    const uint8_t* qh = blk + 128 + 32 * h;
                    const int8_t* sc = (const int8_t*)(blk + 192 + 8 * h);
                    for (int l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        wb[128 * h + l] = d * sc[is] * (double)(((ql[l] & 15) | (((qh[l] >> 0) & 3) << 4)) - 32);
                        wb[128 * h + 32 + l] = d * sc[is + 2] * (double)(((ql[l + 32] & 15) | (((qh[l] >> 2) & 3) << 4)) - 32);
                        wb[128 * h + 64 + l] = d * sc[is + 4] * (double)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                        wb[128 * h + 96 + l] = d * sc[is + 6] * (double)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
                    }
                }
            } else if (type == ORA_Q4_0) {
                double d = (double)ora_h2f(rd16(blk));
                for (int j = 0; j < 16; ++j) {
                    wb[j] = (double)((blk[2 + j] & 15) - 8) * d;
                    wb[j + 16] = (double)((blk[2 + j] >> 4) - 8) * d;
                }
            } else {
                double d = (double)ora_h2f(rd16(blk)), dmin = (double)ora_h2f(rd16(blk + 2));
                for (int c = 0; c < 4; ++c) {
                    int sc0, m0, sc1, m1;
                    ora_q4k_scale_min(blk + 4, 2 * c, &sc0, &m0);
                    ora_q4k_scale_min(blk + 4, 2 * c + 1, &sc1, &m1);
                    for (int l = 0; l < 32; ++l) {
                        wb[64 * c + l] = d * sc0 * (double)(blk[16 + 32 * c + l] & 15) - dmin * m0;
                        wb[64 * c + 32 + l] = d * sc1 * (double)(blk[16 + 32 * c + l] >> 4) - dmin * m1;
                    }
                }
            }
        }
        for (int64_t m = 0; m < M; ++m) {
            double s = 0.0;
            const double* xm = x + m * K;
            for (int64_t k = 0; k < K; ++k) s += xm[k] * w[k];
            Y[m * N + n] = s;
        }
    }
    free(x);
    free(w);
    return 0;
}

/* ---- fp32 AVX2 dequant-GEMM (the timed CPU baseline) ----------------------- */
typedef struct {
    int type;
    const uint8_t* W;
    int64_t N, K, M;
    const float* x; /* fp32 copy of X */
    float* Y;
} gemm_job;

static inline float hsum256(__m256 v)
{
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    lo = _mm_add_ss(lo, _mm_shuffle_ps(lo, lo, 1));
    return _mm_cvtss_f32(lo);
}

/* 16 packed bytes -> 32 nibble values as 4 x 8 floats in element order. */
static inline void nibbles_to_f32(const uint8_t* qs, __m256 w[4], int offset8)
{
    __m128i b = _mm_loadu_si128((const __m128i*)qs);
    __m128i lo = _mm_and_si128(b, _mm_set1_epi8(15));
    __m128i hi = _mm_and_si128(_mm_srli_epi16(b, 4), _mm_set1_epi8(15));
    if (offset8) {
        lo = _mm_sub_epi8(lo, _mm_set1_epi8(8));
        hi = _mm_sub_epi8(hi, _mm_set1_epi8(8));
    }
    w[0] = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(lo));
    w[1] = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(lo, 8)));
    w[2] = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(hi));
    w[3] = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(hi, 8)));
}

#define ORA_MCHUNK 8

static void gemm_rows(void* arg, int64_t lo, int64_t hi)
{
    gemm_job* j = (gemm_job*)arg;
    const int64_t K = j->K, M = j->M, N = j->N;
    size_t rb = ora_row_bytes(j->type, K);
    for (int64_t n = lo; n < hi; ++n) {
        const uint8_t* row = j->W + (size_t)n * rb;
        for (int64_t m0 = 0; m0 < M; m0 += ORA_MCHUNK) {
            int mc = (int)(M - m0 < ORA_MCHUNK ? M - m0 : ORA_MCHUNK);
            __m256 acc[ORA_MCHUNK];
            for (int i = 0; i < mc; ++i) acc[i] = _mm256_setzero_ps();
            if (j->type != ORA_Q4_0 && j->type != ORA_Q4_K) {
                /* the other types: the row dequantized to fp32 (ora_dequantize), then fp32 dots */
                float* w = (float*)malloc(sizeof(float) * (size_t)K);
                ora_dequantize(j->type, row, K, w);
                for (int i = 0; i < mc; ++i) {
                    const float* xp = j->x + (m0 + i) * K;
                    __m256 a = _mm256_setzero_ps();
                    int64_t k = 0;
                    for (; k + 8 <= K; k += 8) a = _mm256_fmadd_ps(_mm256_loadu_ps(xp + k), _mm256_loadu_ps(w + k), a);
                    float tail = 0.0f;
                    for (; k < K; ++k) tail = fmaf(xp[k], w[k], tail);
                    acc[i] = _mm256_add_ps(a, _mm256_set_ps(0, 0, 0, 0, 0, 0, 0, tail));
                }
                free(w);
            } else if (j->type == ORA_Q4_0) {
                for (int64_t b = 0; b < K / 32; ++b) {
                    const uint8_t* blk = row + b * 18;
                    __m256 w[4];
                    nibbles_to_f32(blk + 2, w, 1);
                    __m256 d = _mm256_set1_ps(ora_h2f(rd16(blk)));
                    for (int i = 0; i < mc; ++i) {
                        const float* xp = j->x + (m0 + i) * K + b * 32;
                        __m256 t = _mm256_mul_ps(_mm256_loadu_ps(xp), w[0]);
                        t = _mm256_fmadd_ps(_mm256_loadu_ps(xp + 8), w[1], t);
                        t = _mm256_fmadd_ps(_mm256_loadu_ps(xp + 16), w[2], t);
                        t = _mm256_fmadd_ps(_mm256_loadu_ps(xp + 24), w[3], t);
                        acc[i] = _mm256_fmadd_ps(t, d, acc[i]);
                    }
                }
            } else {
                for (int64_t b = 0; b < K / 256; ++b) {
                    const uint8_t* blk = row + b * 144;
                    float d = ora_h2f(rd16(blk)), dmin = ora_h2f(rd16(blk + 2));
                    for (int c = 0; c < 4; ++c) {
                        int sc0, m0_, sc1, m1_;
                        ora_q4k_scale_min(blk + 4, 2 * c, &sc0, &m0_);
                        ora_q4k_scale_min(blk + 4, 2 * c + 1, &sc1, &m1_);
                        /* 32 bytes -> sub-block 2c (low nibbles) and 2c+1 (high nibbles) */
                        __m256 wl[4], wh[4];
                        __m256 q[8];
                        nibbles_to_f32(blk + 16 + 32 * c, q, 0);      /* bytes 0..15 */
                        nibbles_to_f32(blk + 16 + 32 * c + 16, q + 4, 0); /* bytes 16..31 */
                        /* element order: low nibbles of bytes 0..31 then high nibbles */
                        wl[0] = q[0]; wl[1] = q[1]; wl[2] = q[4]; wl[3] = q[5];
                        wh[0] = q[2]; wh[1] = q[3]; wh[2] = q[6]; wh[3] = q[7];
                        __m256 ds0 = _mm256_set1_ps(d * (float)sc0), dm0 = _mm256_set1_ps(dmin * (float)m0_);
                        __m256 ds1 = _mm256_set1_ps(d * (float)sc1), dm1 = _mm256_set1_ps(dmin * (float)m1_);
                        for (int t4 = 0; t4 < 4; ++t4) {
                            wl[t4] = _mm256_fmsub_ps(ds0, wl[t4], dm0);
                            wh[t4] = _mm256_fmsub_ps(ds1, wh[t4], dm1);
                        }
                        for (int i = 0; i < mc; ++i) {
                            const float* xp = j->x + (m0 + i) * K + b * 256 + 64 * c;
                            __m256 a = acc[i];
                            for (int t4 = 0; t4 < 4; ++t4) a = _mm256_fmadd_ps(_mm256_loadu_ps(xp + 8 * t4), wl[t4], a);
                            for (int t4 = 0; t4 < 4; ++t4) a = _mm256_fmadd_ps(_mm256_loadu_ps(xp + 32 + 8 * t4), wh[t4], a);
                            acc[i] = a;
                        }
                    }
                }
            }
            for (int i = 0; i < mc; ++i) j->Y[(m0 + i) * N + n] = hsum256(acc[i]);
        }
    }
}

int ora_q4_gemm_x32(int type, const uint8_t* W, int64_t N, int64_t K,
                    const float* X, int64_t M, float* Y, int nthreads)
{
    if (ora_row_bytes(type, K) == 0 || N <= 0 || M <= 0) return -1;
    gemm_job j = { type, W, N, K, M, X, Y };
    ora_parallel_for(nthreads, N, gemm_rows, &j);
    return 0;
}

int ora_q4_gemm_f32(int type, const uint8_t* W, int64_t N, int64_t K,
                    const uint16_t* X, int64_t M, float* Y, int nthreads)
{
    if (ora_row_bytes(type, K) == 0 || N <= 0 || M <= 0) return -1;
    float* x = (float*)malloc(sizeof(float) * (size_t)(M * K));
    ora_h2f_array(X, x, (size_t)(M * K));
    int rc = ora_q4_gemm_x32(type, W, N, K, x, M, Y, nthreads);
    free(x);
    return rc;
}
