/*
 * ane_oracle.c -- scalar CPU restatement of ane's quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker and the CPU baseline, never the
 * product).  Build: oracle/Makefile, flags -O2 -ffp-contract=off, no
 * -ffast-math, so every float operation below is one IEEE binary32 rounding
 * exactly as written.  See ane_oracle.h for what pins each function.
 */
#include "ane_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

int oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n <= 0) n = omp_get_num_procs();
    g_threads = n;
#else
    (void)n;
    g_threads = 1;
#endif
    return g_threads;
}

/* AArch64 FMAX/FMIN (not FMAXNM): NaN in -> NaN out; max(+0,-0) = +0,
 * min(+0,-0) = -0.  Used by the handlers at bytecode_interpreter.s:1900,
 * 1937-1938, 2293-2294. */
static inline float fmaxA(float a, float b) {
    if (isnan(a)) return a;
    if (isnan(b)) return b;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}
static inline float fminA(float a, float b) {
    if (isnan(a)) return a;
    if (isnan(b)) return b;
    if (a == b) return signbit(a) ? a : b;
    return a < b ? a : b;
}

/* FCVTZS to int32: NaN -> 0, truncation, saturation. */
static inline int32_t cvtzs(float x) {
    if (isnan(x)) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal half: renormalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400));
            man &= 0x3ff;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Pass 1 of bytecode_interpreter.s:1893-1905: amax = max |x| (fabs + FMAX,
 * NaN-propagating, order irrelevant). */
static float absmax_n(const float* src, size_t n) {
    float amax = 0.0f;
    for (size_t i = 0; i < n; i++) amax = fmaxA(amax, fabsf(src[i]));
    return amax;
}

/* bytecode_interpreter.s:1906-1920: zero guard then two IEEE divisions.
 * (fcmp s16,#0.0 / b.eq: a NaN amax is "not equal" and divides.) */
static void quant_params(float amax, float* scale, float* inv) {
    if (amax == 0.0f) {
        *scale = 1.0f;
        *inv = 127.0f;
    } else {
        *scale = amax / 127.0f;
        *inv = 127.0f / amax;
    }
}

/* bytecode_interpreter.s:1932-1944: fmul, fmax -127, fmin 127, frintn,
 * fcvtzs, st1b (low byte). */
static inline int8_t quant1(float x, float inv) {
    float t = x * inv;
    t = fmaxA(t, -127.0f);
    t = fminA(t, 127.0f);
    t = rintf(t); /* round-to-nearest-even in the default mode */
    return (int8_t)(uint8_t)(uint32_t)cvtzs(t);
}

void oracle_quantize_exact(size_t n, const float* src, int8_t* dst,
                           float* scale_out) {
    float scale, inv;
    quant_params(absmax_n(src, n), &scale, &inv);
    *scale_out = scale;
    for (size_t i = 0; i < n; i++) dst[i] = quant1(src[i], inv);
}

void oracle_quantize_fp32_i8(uint32_t count, const float* src, int8_t* dst,
                             float* scale_out) {
    /* do { 16 lanes } while (i < count): at least one vector. */
    size_t n = ((size_t)count + 15) & ~(size_t)15;
    if (n == 0) n = 16;
    oracle_quantize_exact(n, src, dst, scale_out);
}

void oracle_dequantize_i8_fp32(uint32_t count, float scale, const int8_t* src,
                               float* dst) {
    /* cbz count -> nothing; else 16-lane steps (count%16 != 0 never
     * terminates in the reference; this restatement stops at ceil16). */
    size_t n = ((size_t)count + 15) & ~(size_t)15;
    for (size_t i = 0; i < n; i++) dst[i] = (float)src[i] * scale;
}

void oracle_quantize_fp32_i8_channelwise(uint32_t rows, uint32_t cols,
                                         const float* src, int8_t* dst,
                                         float* scales) {
    size_t cpad = ((size_t)cols + 15) & ~(size_t)15;
    if (cpad == 0) cpad = 16;
    for (uint32_t r = 0; r < rows; r++) {
        const float* s = src + (size_t)r * cpad;
        int8_t* d = dst + (size_t)r * cpad;
        float scale, inv;
        quant_params(absmax_n(s, cpad), &scale, &inv);
        scales[r] = scale;
        for (size_t i = 0; i < cpad; i++) d[i] = quant1(s[i], inv);
    }
}

size_t oracle_packed_b_size(uint32_t K, uint32_t N) {
    size_t G = (((size_t)K + 3) & ~(size_t)3) / 4;
    size_t P = (((size_t)N + 15) & ~(size_t)15) / 16;
    return P * G * 64;
}

/* bytecode_interpreter.s:2459-2582: dst[(p*G+g)*64 + 4c + d] =
 * B[4g+d][16p+c], zero where 4g+d >= K or 16p+c >= N. */
void oracle_pack_b_i8(uint32_t K, uint32_t N, const int8_t* src, int8_t* dst) {
    size_t G = (((size_t)K + 3) & ~(size_t)3) / 4;
    size_t P = (((size_t)N + 15) & ~(size_t)15) / 16;
    for (size_t p = 0; p < P; p++)
        for (size_t g = 0; g < G; g++)
            for (size_t c = 0; c < 16; c++)
                for (size_t d = 0; d < 4; d++) {
                    size_t k = 4 * g + d, col = 16 * p + c;
                    dst[(p * G + g) * 64 + 4 * c + d] =
                        (k < K && col < N) ? src[k * N + col] : 0;
                }
}

/* bytecode_interpreter.s:1995-2446 (dense_i8) and 2849-3300 (dense_u8s8). */
void oracle_dense_i8(uint32_t M, uint32_t N, uint32_t K, float sa, float sb,
                     uint8_t flags, const void* A, const int8_t* Bp,
                     const float* bias, float* C, int a_unsigned) {
    size_t Kp = ((size_t)K + 63) & ~(size_t)63;      /* :2038-2039 */
    size_t Mp = ((size_t)M + 15) & ~(size_t)15;      /* :2033-2034 */
    if (Mp == 0) Mp = 16;                            /* do-while tile rows */
    size_t G = Kp / 4;
    float s = sa * sb;                               /* :2017 one fmul */
    float lo = (flags & 1) ? 0.0f : -3.40282347e+38f; /* :2021-2028 */
    const int8_t* As = (const int8_t*)A;
    const uint8_t* Au = (const uint8_t*)A;
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long ii = 0; ii < (long)Mp; ii++) {
        size_t i = (size_t)ii;
        for (size_t j = 0; j < N; j++) {
            uint32_t acc = 0; /* za tiles: wrapping int32 */
            const int8_t* panel = Bp + (j / 16) * G * 64 + (j % 16) * 4;
            for (size_t k = 0; k < Kp; k++) {
                int32_t a = a_unsigned ? (int32_t)Au[i * Kp + k]
                                       : (int32_t)As[i * Kp + k];
                int32_t b = (int32_t)panel[(k / 4) * 64 + (k % 4)];
                acc += (uint32_t)(a * b);
            }
            /* scvtf, fmul, fadd bias, fmax lo: :2269-2294, no fusion */
            float v = (float)(int32_t)acc;
            v = v * s;
            v = v + bias[j];
            C[i * N + j] = fmaxA(v, lo);
        }
    }
}

void oracle_gemm_s8_i32(uint32_t M, uint32_t N, uint32_t K, const int8_t* A,
                        uint32_t lda, const int8_t* B, uint32_t ldb,
                        int32_t* acc) {
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long ii = 0; ii < (long)M; ii++) {
        size_t i = (size_t)ii;
        uint32_t* row = (uint32_t*)malloc(sizeof(uint32_t) * (N ? N : 1));
        memset(row, 0, sizeof(uint32_t) * N);
        for (size_t k = 0; k < K; k++) {
            int32_t a = A[i * lda + k];
            const int8_t* b = B + k * ldb;
            for (size_t j = 0; j < N; j++) row[j] += (uint32_t)(a * (int32_t)b[j]);
        }
        for (size_t j = 0; j < N; j++) acc[i * N + j] = (int32_t)row[j];
        free(row);
    }
}

void oracle_dense_fused_rows(int32_t row0, int32_t row1, int32_t N, int32_t K,
                             float s, int relu, const int8_t* qA,
                             const int8_t* qB, float* C) {
    float lo = relu ? 0.0f : -3.40282347e+38f;
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long ii = row0; ii < (long)row1; ii++) {
        size_t i = (size_t)ii;
        uint32_t* row = (uint32_t*)malloc(sizeof(uint32_t) * (N ? N : 1));
        memset(row, 0, sizeof(uint32_t) * (size_t)N);
        for (size_t k = 0; k < (size_t)K; k++) {
            int32_t a = qA[i * (size_t)K + k];
            const int8_t* b = qB + k * (size_t)N;
            for (size_t j = 0; j < (size_t)N; j++)
                row[j] += (uint32_t)(a * (int32_t)b[j]);
        }
        for (size_t j = 0; j < (size_t)N; j++) {
            float v = (float)(int32_t)row[j];
            v = v * s;
            v = v + 0.0f; /* mirrors the zero-bias fadd: -0 -> +0 */
            C[i * (size_t)N + j] = fmaxA(v, lo);
        }
        free(row);
    }
}

void oracle_dense_fused_i8(int32_t M, int32_t N, int32_t K, float scale,
                           int relu, const float* A, const float* B, float* C) {
    if (M <= 0 || N <= 0) return;
    size_t na = (size_t)M * (size_t)(K > 0 ? K : 0);
    size_t nb = (size_t)(K > 0 ? K : 0) * (size_t)N;
    int8_t* qA = (int8_t*)malloc(na ? na : 1);
    int8_t* qB = (int8_t*)malloc(nb ? nb : 1);
    float sa, sb;
    oracle_quantize_exact(na, A, qA, &sa);
    oracle_quantize_exact(nb, B, qB, &sb);
    float s = sa * sb;
    s = s * scale;
    oracle_dense_fused_rows(0, M, N, K > 0 ? K : 0, s, relu, qA, qB, C);
    free(qA);
    free(qB);
}

/* FADDV over 16 fp32 lanes: recursive halving, lo + hi at every level
 * (bytecode_interpreter.s:7060; Arm ARM Reduce()).  Equals an xor-butterfly
 * with offsets 1, 2, 4, 8. */
static float faddv16(const float* a) {
    float t8[8], t4[4], t2[2];
    for (int l = 0; l < 8; l++) t8[l] = a[2 * l] + a[2 * l + 1];
    for (int l = 0; l < 4; l++) t4[l] = t8[2 * l] + t8[2 * l + 1];
    for (int l = 0; l < 2; l++) t2[l] = t4[2 * l] + t4[2 * l + 1];
    return t2[0] + t2[1];
}

/* bytecode_interpreter.s:7016-7063. */
void oracle_q8_0_gemv(uint32_t M, uint32_t K, const float* x,
                      const uint8_t* W, float* y) {
    size_t nb = K >> 5; /* :7026 lsr #5: K%32 ignored */
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long mm = 0; mm < (long)M; mm++) {
        size_t m = (size_t)mm;
        const uint8_t* row = W + m * nb * 34;
        float acc[16];
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t* blk = row + b * 34;
            uint16_t dh = (uint16_t)(blk[0] | (blk[1] << 8));
            float d = oracle_f16_to_f32(dh); /* fcvt s,h exact :7036-7038 */
            for (int h = 0; h < 2; h++)
                for (int l = 0; l < 16; l++) {
                    float w = (float)(int8_t)blk[2 + 16 * h + l] * d; /* scvtf, fmul */
                    acc[l] = fmaf(w, x[32 * b + 16 * h + l], acc[l]); /* fmla */
                }
        }
        y[m] = faddv16(acc); /* faddv s4, p0, z4.s (:7060) */
    }
}

void oracle_q8_0_quantize_x(uint32_t K, const float* x, int8_t* qx, float* dx) {
    size_t nb = K >> 5;
    for (size_t b = 0; b < nb; b++)
        oracle_quantize_exact(32, x + 32 * b, qx + 32 * b, dx + b);
}

void oracle_q8_0_mul_mat_g(uint32_t N, uint32_t K, uint32_t T, const float* x,
                           const uint8_t* W, float* y) {
    size_t nb = K >> 5;
    int8_t* qx = (int8_t*)malloc((size_t)T * nb * 32 + 1);
    float* dx = (float*)malloc(sizeof(float) * ((size_t)T * nb + 1));
    for (uint32_t t = 0; t < T; t++)
        oracle_q8_0_quantize_x(K, x + (size_t)t * K, qx + (size_t)t * nb * 32,
                               dx + (size_t)t * nb);
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long mm = 0; mm < (long)N; mm++) {
        size_t m = (size_t)mm;
        const uint8_t* row = W + m * nb * 34;
        for (uint32_t t = 0; t < T; t++) {
            const int8_t* q = qx + (size_t)t * nb * 32;
            const float* d = dx + (size_t)t * nb;
            float p[16];
            for (int l = 0; l < 16; l++) p[l] = 0.0f;
            for (size_t b = 0; b < nb; b++) {
                const uint8_t* blk = row + b * 34;
                float dw = oracle_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                int32_t isum = 0;
                for (int i = 0; i < 32; i++)
                    isum += (int32_t)(int8_t)blk[2 + i] * (int32_t)q[32 * b + i];
                float dd = dw * d[b];
                p[b % 16] = fmaf((float)isum, dd, p[b % 16]);
            }
            y[(size_t)t * N + m] = faddv16(p);
        }
    }
    free(qx);
    free(dx);
}

/* ------------------------------------------------------------ other Q formats
 * The reference's per-format GEMVs share the 0x57 skeleton: 16 fp32 lanes per
 * row, lane l accumulating with fmla in the order the handler visits the
 * elements, then the FADDV tree.  Only the unpacking differs. */

static inline float h2f(const uint8_t* p) { return oracle_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static inline uint32_t ld16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }
static inline uint32_t ld32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
/* SVE LSR (vectors): shift amounts >= the element size give 0. */
static inline uint32_t lsr_sve(uint32_t v, uint32_t sh) { return sh >= 32 ? 0u : v >> sh; }
static inline uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* 0x58  bytecode_interpreter.s:7071-7126. */
void oracle_q4_0_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y) {
    size_t nb = K >> 5; /* :7081 lsr #5 */
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long mm = 0; mm < (long)M; mm++) {
        const uint8_t* row = W + (size_t)mm * nb * 18;
        float acc[16];
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t* blk = row + b * 18;
            float d = h2f(blk); /* :7094-7095 */
            for (int l = 0; l < 16; l++) { /* low nibbles, :7101-7108 */
                float w = (float)((int)(blk[2 + l] & 15) - 8) * d;
                acc[l] = fmaf(w, x[32 * b + l], acc[l]);
            }
            for (int l = 0; l < 16; l++) { /* high nibbles, :7110-7117 */
                float w = (float)((int)(blk[2 + l] >> 4) - 8) * d;
                acc[l] = fmaf(w, x[32 * b + 16 + l], acc[l]);
            }
        }
        y[mm] = faddv16(acc); /* :7123 */
    }
}

/* The 6-bit (scale, min) pair of sub-block j from the 12-byte array of Q4_K
 * and Q5_K (bytecode_interpreter.s:11064-11089, 11406-11427). */
static void kq_scale_min(const uint8_t* s, int j, uint32_t* sc, uint32_t* m) {
    if (j < 4) {
        *sc = s[j] & 63u;
        *m = s[j + 4] & 63u;
    } else {
        *sc = (s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4);
        *m = (uint32_t)(s[j + 4] >> 4) | ((uint32_t)(s[j] >> 6) << 4);
    }
}

/* 0x75  bytecode_interpreter.s:11024-11131: 144-byte super-blocks
 * [d][dmin][scales 12][qs 128]; sub-block j (32 values) takes qs[16j+l]:
 * low nibble -> element 32j+l, high nibble -> 32j+16+l;
 * w = fl(fl(q * fl(d*sc)) + fl(-dmin*m)). */
void oracle_q4_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y) {
    size_t nsb = K >> 8; /* :11035 lsr #8 */
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long mm = 0; mm < (long)M; mm++) {
        const uint8_t* row = W + (size_t)mm * nsb * 144;
        float acc[16];
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = row + sb * 144;
            const float* xs = x + 256 * sb;
            float d = h2f(blk), nmin = -h2f(blk + 2); /* :11045-11049 fneg */
            for (int j = 0; j < 8; j++) {
                uint32_t sc, m;
                kq_scale_min(blk + 4, j, &sc, &m);
                float ds = d * (float)sc, dm = nmin * (float)m; /* :11092-11097 */
                const uint8_t* q = blk + 16 + 16 * j;
                for (int l = 0; l < 16; l++) { /* :11104-11112 */
                    float t = (float)(q[l] & 15) * ds;
                    float w = t + dm;
                    acc[l] = fmaf(w, xs[32 * j + l], acc[l]);
                }
                for (int l = 0; l < 16; l++) { /* :11114-11121 */
                    float t = (float)(q[l] >> 4) * ds;
                    float w = t + dm;
                    acc[l] = fmaf(w, xs[32 * j + 16 + l], acc[l]);
                }
            }
        }
        y[mm] = faddv16(acc); /* :11129 */
    }
}

/* 0x76  bytecode_interpreter.s:11146-11222: 84-byte super-blocks
 * [scales 16][qs 64][d][dmin]; 16 sub-blocks of 16 values; element 16j+l
 * = bits 2l..2l+1 of the little-endian word qs[4j..4j+3];
 * w = fl(fl(q * fl(d*(sc&15))) + fl(-dmin*(sc>>4))). */
void oracle_q2_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y) {
    size_t nsb = K >> 8;
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long mm = 0; mm < (long)M; mm++) {
        const uint8_t* row = W + (size_t)mm * nsb * 84;
        float acc[16];
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = row + sb * 84;
            const float* xs = x + 256 * sb;
            float d = h2f(blk + 80), nmin = -h2f(blk + 82); /* :11169-11174 */
            for (int j = 0; j < 16; j++) {
                uint32_t sc = blk[j] & 15u, m = (uint32_t)(blk[j] >> 4); /* :11180-11182 */
                float ds = d * (float)sc, dm = nmin * (float)m;
                uint32_t q32 = ld32(blk + 16 + 4 * j); /* :11193 */
                for (int l = 0; l < 16; l++) { /* :11203-11212 */
                    float t = (float)((q32 >> (2 * l)) & 3u) * ds;
                    float w = t + dm;
                    acc[l] = fmaf(w, xs[16 * j + l], acc[l]);
                }
            }
        }
        y[mm] = faddv16(acc); /* :11220 */
    }
}

/* 0x77  bytecode_interpreter.s:11236-11358: 110-byte super-blocks
 * [hmask 32][qs 64][scales 12][d]; sub-block j (32 values): signed scale
 * sc-32 (sc 6 bits, low four sub-blocks scales[j]&63, high four rebuilt as
 * for Q4_K); element 32j+l: 2 bits from the word qs[8j..], high bit l of the
 * halfword hmask[4j..]; element 32j+16+l: the word qs[8j+4..] and halfword
 * hmask[4j+2..], w = fl((q - 4) * fl(d*(sc-32))).
 * The second half reproduces the handler as it runs: its first shift
 * (:11329, lsr z0, z0, z1) uses z1 after :11323 reloaded it with the first
 * half's inputs, so the word is first shifted right by the bit pattern of
 * x[32j+l] (0 for +0.0, small for tiny denormals, everything else >= 32 and
 * so a zero field) before the 2l shift. */
void oracle_q3_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y) {
    size_t nsb = K >> 8;
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long mm = 0; mm < (long)M; mm++) {
        const uint8_t* row = W + (size_t)mm * nsb * 110;
        float acc[16];
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = row + sb * 110;
            const uint8_t *hm = blk, *qs = blk + 32, *s = blk + 96;
            const float* xs = x + 256 * sb;
            float d = h2f(blk + 108); /* :11260-11261 */
            for (int j = 0; j < 8; j++) {
                uint32_t sc = j < 4 ? (s[j] & 63u) : ((s[j + 4] & 15u) | ((uint32_t)(s[j - 4] >> 6) << 4));
                float ds = d * (float)((int)sc - 32); /* :11288-11290 */
                uint32_t qa = ld32(qs + 8 * j), ha = ld16(hm + 4 * j);
                for (int l = 0; l < 16; l++) { /* :11297-11325 */
                    int q = (int)(((qa >> (2 * l)) & 3u) | (((ha >> l) & 1u) << 2));
                    float w = (float)(q - 4) * ds;
                    acc[l] = fmaf(w, xs[32 * j + l], acc[l]);
                }
                uint32_t qb = ld32(qs + 8 * j + 4), hb = ld16(hm + 4 * j + 2);
                for (int l = 0; l < 16; l++) { /* :11327-11348 */
                    uint32_t v = lsr_sve(qb, fbits(xs[32 * j + l]));
                    int q = (int)(((v >> (2 * l)) & 3u) | (((hb >> l) & 1u) << 2));
                    float w = (float)(q - 4) * ds;
                    acc[l] = fmaf(w, xs[32 * j + 16 + l], acc[l]);
                }
            }
        }
        y[mm] = faddv16(acc); /* :11356 */
    }
}

/* 0x78  bytecode_interpreter.s:11372-11483: 176-byte super-blocks
 * [d][dmin][scales 12][qh 32][qs 128]; sub-block j: qs[16j+l] low nibble |
 * bit l of qh word j << 4 -> element 32j+l, high nibble | bit 16+l << 4 ->
 * element 32j+16+l; w = fl(fl(q * fl(d*sc)) + fl(-dmin*m)). */
void oracle_q5_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y) {
    size_t nsb = K >> 8;
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long mm = 0; mm < (long)M; mm++) {
        const uint8_t* row = W + (size_t)mm * nsb * 176;
        float acc[16];
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = row + sb * 176;
            const float* xs = x + 256 * sb;
            float d = h2f(blk), nmin = -h2f(blk + 2); /* :11393-11398 */
            for (int j = 0; j < 8; j++) {
                uint32_t sc, m;
                kq_scale_min(blk + 4, j, &sc, &m);
                float ds = d * (float)sc, dm = nmin * (float)m; /* :11428-11433 */
                const uint8_t* q = blk + 48 + 16 * j;
                uint32_t h = ld32(blk + 16 + 4 * j); /* :11444 */
                for (int l = 0; l < 16; l++) { /* :11436-11458 */
                    uint32_t qv = (q[l] & 15u) | ((((h & 0xffffu) >> l) & 1u) << 4);
                    float t = (float)qv * ds;
                    float w = t + dm;
                    acc[l] = fmaf(w, xs[32 * j + l], acc[l]);
                }
                for (int l = 0; l < 16; l++) { /* :11460-11476 */
                    uint32_t qv = (uint32_t)(q[l] >> 4) | ((((h >> 16) >> l) & 1u) << 4);
                    float t = (float)qv * ds;
                    float w = t + dm;
                    acc[l] = fmaf(w, xs[32 * j + 16 + l], acc[l]);
                }
            }
        }
        y[mm] = faddv16(acc); /* :11481 */
    }
}

/* 0x79  bytecode_interpreter.s:11498-11626: 210-byte super-blocks
 * [ql 128][qh 64][scales 16 int8][d]; 16 sub-blocks of 16 values; element
 * 16j+n = nibble n of ql[8j..8j+7] (low nibble of byte n/2 for even n, high
 * for odd) | bits 2n..2n+1 of the word qh[4j..] << 4, centred by 32;
 * w = fl((q - 32) * fl(d*sc)); the even and odd lanes are zipped back into
 * element order before the fmla (:11609-11613). */
void oracle_q6_k_gemv(uint32_t M, uint32_t K, const float* x, const uint8_t* W, float* y) {
    size_t nsb = K >> 8;
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long mm = 0; mm < (long)M; mm++) {
        const uint8_t* row = W + (size_t)mm * nsb * 210;
        float acc[16];
        for (int l = 0; l < 16; l++) acc[l] = 0.0f;
        for (size_t sb = 0; sb < nsb; sb++) {
            const uint8_t* blk = row + sb * 210;
            const float* xs = x + 256 * sb;
            float d = h2f(blk + 208); /* :11522-11523 */
            for (int j = 0; j < 16; j++) {
                float ds = d * (float)(int8_t)blk[192 + j]; /* :11530-11532 */
                uint32_t h = ld32(blk + 128 + 4 * j); /* :11560 */
                for (int n = 0; n < 16; n++) {
                    uint8_t byte = blk[8 * j + (n >> 1)];
                    uint32_t nib = (n & 1) ? (uint32_t)(byte >> 4) : (uint32_t)(byte & 15);
                    int q = (int)(nib | (((h >> (2 * n)) & 3u) << 4));
                    float w = (float)(q - 32) * ds;
                    acc[n] = fmaf(w, xs[16 * j + n], acc[n]);
                }
            }
        }
        y[mm] = faddv16(acc); /* :11622 */
    }
}

/* 0x7C  bytecode_interpreter.s:12363-12408: out row r = dequantized Q8_0 row
 * indices[r] (u32), dim/32 blocks of 34 bytes: out = fl((float)q * d). */
void oracle_get_rows_q8_0(uint32_t n_rows, uint32_t dim, const uint8_t* table, const uint32_t* indices,
                          float* out) {
    size_t nb = dim >> 5, rb = nb * 34;
    for (size_t r = 0; r < n_rows; r++) {
        const uint8_t* row = table + (size_t)indices[r] * rb;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t* blk = row + b * 34;
            float d = h2f(blk);
            for (int q = 0; q < 32; q++) out[r * nb * 32 + b * 32 + q] = (float)(int8_t)blk[2 + q] * d;
        }
    }
}

/* 0x7D  bytecode_interpreter.s:12419-12469: Q4_0 rows of 18-byte blocks;
 * element i = (qs[i] & 15) - 8, element 16+i = (qs[i] >> 4) - 8, times d. */
void oracle_get_rows_q4_0(uint32_t n_rows, uint32_t dim, const uint8_t* table, const uint32_t* indices,
                          float* out) {
    size_t nb = dim >> 5, rb = nb * 18;
    for (size_t r = 0; r < n_rows; r++) {
        const uint8_t* row = table + (size_t)indices[r] * rb;
        for (size_t b = 0; b < nb; b++) {
            const uint8_t* blk = row + b * 18;
            float d = h2f(blk);
            float* o = out + r * nb * 32 + b * 32;
            for (int i = 0; i < 16; i++) {
                o[i] = (float)((int)(blk[2 + i] & 15) - 8) * d;
                o[16 + i] = (float)((int)(blk[2 + i] >> 4) - 8) * d;
            }
        }
    }
}

/* 0x61 cblas_igemm / 0x62 cblas_ugemm / 0x63 cblas_usgemm: the
 * CBLAS_INTEGER_GEMM macro, bytecode_interpreter.s:8328-9135, instantiated
 * at :9137-9139 with smopa / umopa / usmopa.  variant 0: s8 x s8, 1: u8 x u8,
 * 2: u8 x s8.  Only rows < M and columns < N of C are written (the store
 * predicates, :8946-8960 and the w15 row count).
 *   k blocks      : K / 64 (:8375), a remainder of K is never read;
 *   A, transA = 0 : row i at A + i*lda (:8504-8509, :8521-8560);
 *   A, transA = 1 : the handler adds the k offset to A + ti and steps rows by
 *                   lda (:8513-8514, :8562-8575), so output row i reads
 *                   A[(i % 16)*lda + (i - i % 16) + k] -- not A^T;
 *   B, transB = 0 : B[k*ldb + j], one byte per ld1b lane (:8604-8680);
 *   B, transB = 1 : B[j*ldb + k], rows of B transposed through za3
 *                   (:8768-8872);
 *   accumulator   : zero when the bits of beta are zero, otherwise seeded
 *                   with the BIT PATTERN of fl(beta * C[i][j]) (:8402-8488:
 *                   fmul, then mova into the int32 za tiles), then the
 *                   products are added as wrapping int32 (smopa);
 *   store         : C = fl(fl32(acc) * alpha) (scvtf, fmul: :8962-8980).
 * semantics 1 instead computes what the header comment (:8330) describes:
 * op(A) = A^T for transA, and C = fl(fl(fl32(acc) * alpha) + fl(beta * C))
 * with C not read when beta == 0. */
static inline int32_t igemm_elem(const uint8_t* p, int is_unsigned) {
    return is_unsigned ? (int32_t)*p : (int32_t)(int8_t)*p;
}

void oracle_cblas_igemm(int variant, int semantics, uint8_t flags, uint32_t M, uint32_t N, uint32_t K,
                        uint32_t lda, uint32_t ldb, uint32_t ldc, float alpha, float beta, const void* A,
                        const void* B, float* C) {
    const uint8_t* a8 = (const uint8_t*)A;
    const uint8_t* b8 = (const uint8_t*)B;
    const int au = variant == 1 || variant == 2, bu = variant == 1;
    const int ta = flags & 1, tb = (flags >> 1) & 1;
    const size_t Ke = (size_t)(K / 64) * 64;
    uint32_t beta_bits;
    memcpy(&beta_bits, &beta, 4);
    int nt = g_threads;
#pragma omp parallel for num_threads(nt) schedule(static)
    for (long ii = 0; ii < (long)M; ii++) {
        const size_t i = (size_t)ii;
        size_t arow, astep;
        if (!ta) {
            arow = i * lda;
            astep = 1;
        } else if (semantics == 0) {
            arow = (i % 16) * (size_t)lda + (i - i % 16);
            astep = 1;
        } else {
            arow = i;
            astep = lda;
        }
        for (size_t j = 0; j < N; j++) {
            float* c = C + i * ldc + j;
            uint32_t acc = 0;
            if (semantics == 0 && beta_bits != 0) {
                float seed = beta * *c; /* fmul (:8449-8450) */
                memcpy(&acc, &seed, 4);
            }
            for (size_t k = 0; k < Ke; k++) {
                const int32_t a = igemm_elem(a8 + arow + k * astep, au);
                const int32_t b = igemm_elem(b8 + (tb ? j * (size_t)ldb + k : k * (size_t)ldb + j), bu);
                acc += (uint32_t)(a * b);
            }
            float v = (float)(int32_t)acc * alpha;
            if (semantics == 1 && beta != 0.0f) {
                float cb = beta * *c;
                v = v + cb;
            }
            *c = v;
        }
    }
}

/* ------------------------------------------------------------------------
 * The decode-step handlers: rms_norm_fp32 (0x51), silu_fp32 (0x54),
 * rope_fp32 (0x55) and softmax_fp32 (0x56), bytecode_interpreter.s:6508-7009,
 * in their exact fp32 operation sequence.  fmla/fmls/fmad are fused (fmaf),
 * every other operation rounds once.  The estimate instructions follow the
 * Arm ARM pseudocode (FPRSqrtEstimate / RecipSqrtEstimate, FPRecipEstimate /
 * RecipEstimate, FPCR.AH = 0, no increased precision), and the step
 * instructions FRSQRTS / FRECPS are the fused (3 - a*b)/2 and 2 - a*b.
 * ---------------------------------------------------------------------- */
static inline float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* RecipSqrtEstimate(a), a in [128, 512): the Arm ARM's loop, literally. */
static uint32_t recip_sqrt_estimate(uint32_t a) {
    if (a < 256) a = a * 2 + 1;
    else { a = (a >> 1) << 1; a = (a + 1) * 2; }
    uint64_t b = 512;
    while ((uint64_t)a * (b + 1) * (b + 1) < (1ull << 28)) b++;
    return (uint32_t)((b + 1) / 2);
}

float oracle_frsqrte(float x) {
    const uint32_t u = fbits(x), sign = u >> 31, ex = (u >> 23) & 0xff, fr = u & 0x7fffff;
    if (ex == 0xff && fr) return f_of(u | 0x00400000u);          /* quiet the NaN */
    if (ex == 0 && fr == 0) return f_of((sign << 31) | 0x7f800000u); /* +-0 -> +-inf */
    if (sign) return f_of(0x7fc00000u);                           /* default NaN */
    if (ex == 0xff) return 0.0f;                                  /* +inf -> +0 */
    uint64_t f52 = (uint64_t)fr << 29;
    int e = (int)ex;
    if (e == 0) {                                                 /* normalise a denormal */
        while (!(f52 & (1ull << 51))) { f52 <<= 1; e--; }
        f52 = (f52 << 1) & ((1ull << 52) - 1);
    }
    const uint32_t scaled = (e & 1) == 0 ? 256u + (uint32_t)(f52 >> 44) : 128u + (uint32_t)(f52 >> 45);
    const int rexp = (380 - e) / 2;
    const uint32_t est = recip_sqrt_estimate(scaled);
    return f_of(((uint32_t)(rexp & 0xff) << 23) | ((est & 0xff) << 15));
}

float oracle_frecpe(float x) {
    const uint32_t u = fbits(x), sign = u >> 31, ex = (u >> 23) & 0xff, fr = u & 0x7fffff;
    if (ex == 0xff && fr) return f_of(u | 0x00400000u);
    if (ex == 0xff) return f_of(sign << 31);                       /* +-inf -> +-0 */
    if (ex == 0 && fr == 0) return f_of((sign << 31) | 0x7f800000u);
    if (ex == 0 && fr < (1u << 21)) return f_of((sign << 31) | 0x7f800000u); /* |x| < 2^-128: overflow, RNE */
    uint64_t f52 = (uint64_t)fr << 29;
    int e = (int)ex;
    if (e == 0) {
        if (!(f52 & (1ull << 51))) { e = -1; f52 = (f52 << 2) & ((1ull << 52) - 1); }
        else f52 = (f52 << 1) & ((1ull << 52) - 1);
    }
    const uint32_t scaled = 256u + (uint32_t)(f52 >> 44);
    int rexp = 253 - e;
    const uint32_t a = scaled * 2 + 1;
    const uint32_t est = ((1u << 19) / a + 1) / 2;                 /* RecipEstimate */
    uint64_t frac = (uint64_t)(est & 0xff) << 44;
    if (rexp == 0) frac = (1ull << 51) | (frac >> 1);
    else if (rexp == -1) { frac = (1ull << 50) | (frac >> 2); rexp = 0; }
    return f_of((sign << 31) | ((uint32_t)(rexp & 0xff) << 23) | (uint32_t)(frac >> 29));
}

static inline float frsqrts(float a, float b) {
    if ((isinf(a) && b == 0.0f) || (a == 0.0f && isinf(b))) return 1.5f;
    return fmaf(-a, b, 3.0f) * 0.5f;
}
static inline float frecps(float a, float b) {
    if ((isinf(a) && b == 0.0f) || (a == 0.0f && isinf(b))) return 2.0f;
    return fmaf(-a, b, 2.0f);
}
#define K_LOG2E 0x3FB8AA3Bu
#define K_C4 0x3C1D955Au
#define K_C3 0x3D635847u
#define K_C2 0x3E75FDF0u
#define K_LN2 0x3F317218u

/* The exp approximation of silu/softmax (:6627-6665, :6965-6989): range
 * reduction by floor, a degree-4 Horner polynomial of 2^f, and 2^n injected
 * as exponent bits ((n + 127) << 23, n clamped below at -127 when clamp). */
static float exp_poly(float x, int clamp) {
    const float t = x * f_of(K_LOG2E);
    const float n = floorf(t);
    const float f = t - n;
    float p = f_of(K_C4) * f;
    p = p + f_of(K_C3);
    p = p * f;
    p = p + f_of(K_C2);
    p = p * f;
    p = p + f_of(K_LN2);
    p = p * f;
    p = p + 1.0f;
    int32_t ni = cvtzs(n);
    if (clamp && ni < -127) ni = -127;
    return p * f_of(((uint32_t)ni + 127u) << 23);
}

/* 0x54 silu_fp32 (:6617-6713): out = fl(x * r), r = 1/(1 + e^-x) by frecpe
 * and two frecps steps.  count elements. */
void oracle_silu_fp32(uint32_t count, const float* in, float* out) {
    for (uint32_t i = 0; i < count; i++) {
        const float x = in[i];
        const float e = exp_poly(-x, 1);
        const float d = e + 1.0f;
        float r = oracle_frecpe(d);
        r = r * frecps(d, r);
        r = r * frecps(d, r);
        out[i] = x * r;
    }
}

/* 0x51 rms_norm_fp32 (:6508-6565): 16 fmla lanes over x^2, FADDV, fdiv by
 * (float)dim, fadd eps, frsqrte + two frsqrts steps, out = fl(fl(x*r)*w).
 * dim a multiple of 16 (the handler's loops step 16 lanes to zero). */
void oracle_rms_norm_fp32(uint32_t dim, float eps, const float* in, const float* w, float* out) {
    float acc[16];
    for (int l = 0; l < 16; l++) acc[l] = 0.0f;
    for (uint32_t i = 0; i < dim; i++) acc[i % 16] = fmaf(in[i], in[i], acc[i % 16]);
    const float ss = faddv16(acc);
    const float mean = ss / (float)dim;
    const float t = mean + eps;
    float r = oracle_frsqrte(t);
    float s = r * r;
    s = frsqrts(t, s);
    r = r * s;
    s = r * r;
    s = frsqrts(t, s);
    r = r * s;
    for (uint32_t i = 0; i < dim; i++) out[i] = (in[i] * r) * w[i];
}

/* 0x56 softmax_fp32 (:6913-7009): fmax over all, then e = exp_poly(x - max)
 * stored, 16 fadd lanes of e (lane l takes i = l mod 16, increasing i),
 * FADDV, fdiv 1/sum, out = fl(e * inv).  The handler needs dim % 16 == 0;
 * here a lane past dim contributes nothing, which equals it for those. */
void oracle_softmax_fp32(uint32_t dim, const float* in, float* out) {
    if (dim == 0) return;
    float mx = -INFINITY;
    for (uint32_t i = 0; i < dim; i++) mx = fmaxA(mx, in[i]);
    float acc[16];
    for (int l = 0; l < 16; l++) acc[l] = 0.0f;
    for (uint32_t i = 0; i < dim; i++) {
        const float e = exp_poly(in[i] - mx, 1);
        out[i] = e;
        acc[i % 16] = acc[i % 16] + e;
    }
    const float inv = 1.0f / faddv16(acc);
    for (uint32_t i = 0; i < dim; i++) out[i] = out[i] * inv;
}

/* rope_fp32's ratio theta^(2/dim) (:6725-6783): ln(theta) from the exponent
 * and a cubic in the mantissa, then the exp polynomial without the clamp. */
static float rope_ratio(uint32_t dim, float theta) {
    const uint32_t tb = fbits(theta);
    const int32_t e = (int32_t)((tb >> 23) & 0xff) - 127;
    const float fe = (float)e;
    const float m = f_of((tb & ~(0xffu << 23)) | (127u << 23));
    const float t = m - 1.0f;
    float l = f_of(0x3E943014u) * t;
    l = l + f_of(0xBEFBD464u);
    l = l * t;
    l = l + f_of(0x3F7FF972u);
    l = l * t;
    float lt = fe * f_of(K_LN2);
    lt = lt + l;
    float step = 2.0f / (float)dim;
    step = step * lt;
    return exp_poly(step, 0);
}

/* 0x55 rope_fp32 (:6714-6912): pair k of 16-pair chunk c uses power =
 * ratio^(k mod 16) (sequential products) times ratio^16 applied c times;
 * freq = pos / power; r = freq - rint(freq / pi) * pi (fused); sin and cos
 * by fmad Horner polynomials, both negated for odd rint; then
 * out_even = fmls(a*cos, b, sin), out_odd = fmla(b*cos, a, sin). */
void oracle_rope_fp32(uint32_t dim, uint32_t pos, float theta, const float* in, float* out) {
    const uint32_t pairs = dim / 2;
    if (!pairs) return;
    const float ratio = rope_ratio(dim, theta);
    float pw[16], s2 = 1.0f;
    for (int k = 0; k < 16; k++) { pw[k] = s2; s2 = s2 * ratio; }
    const float r16 = s2, posf = (float)pos;
    for (uint32_t c = 0; c * 16 < pairs; c++) {
        for (uint32_t l = 0; l < 16 && c * 16 + l < pairs; l++) {
            const uint32_t p = c * 16 + l;
            float power = pw[l];
            for (uint32_t i = 0; i < c; i++) power = power * r16;
            const float freq = posf / power;
            const float nq = rintf(freq * f_of(0x3EA2F983u));
            const uint32_t odd = ((uint32_t)cvtzs(nq) & 1u) << 31;
            const float r = fmaf(-nq, f_of(0x40490FDBu), freq);
            const float r2 = r * r;
            float sn = f_of(0xB9500D01u);
            sn = fmaf(sn, r2, f_of(0x3C088889u));
            sn = fmaf(sn, r2, f_of(0xBE2AAAABu));
            sn = fmaf(sn, r2, 1.0f);
            sn = sn * r;
            float cs = f_of(0xBAB60B61u);
            cs = fmaf(cs, r2, f_of(0x3D2AAAABu));
            cs = fmaf(cs, r2, -0.5f);
            cs = fmaf(cs, r2, 1.0f);
            sn = f_of(fbits(sn) ^ odd);
            cs = f_of(fbits(cs) ^ odd);
            const float a = in[2 * p], b = in[2 * p + 1];
            float oe = a * cs;
            oe = fmaf(-b, sn, oe);
            float oo = b * cs;
            oo = fmaf(a, sn, oo);
            out[2 * p] = oe;
            out[2 * p + 1] = oo;
        }
    }
}

/* The build's RMSNorm (the fused decode kernels and ane_hip_rms_norm): the
 * canonical fp64 sum of squares (per 32-block part sums, block sums, 64
 * strided lane sums, adjacent-pairs tree), ms = (float)(ss / K), inv =
 * 1 / sqrtf(ms + eps), out = fl(fl(x * inv) * w).  K % 32 == 0. */
void oracle_rms_norm_build(uint32_t K, float eps, const float* x, const float* w, float* out) {
    const uint32_t nb = K / 32;
    double c[64];
    for (int l = 0; l < 64; l++) c[l] = 0.0;
    for (uint32_t b = 0; b < nb; b++) {
        double q[8];
        for (int p = 0; p < 8; p++) {
            const float* v = x + 32 * b + 4 * p;
            q[p] = ((double)v[0] * v[0] + (double)v[1] * v[1]) + ((double)v[2] * v[2] + (double)v[3] * v[3]);
        }
        const double sb = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
        c[b % 64] = c[b % 64] + sb;
    }
    for (int off = 1; off < 64; off <<= 1) {
        double n[64];
        for (int l = 0; l < 64; l++) n[l] = c[l] + c[l ^ off];
        memcpy(c, n, sizeof c);
    }
    const float ms = (float)(c[0] / (double)K);
    const float inv = 1.0f / sqrtf(ms + eps);
    for (uint32_t i = 0; i < K; i++) out[i] = (x[i] * inv) * w[i];
}

/* 16-lane dot product in the handlers' style: lane l accumulates
 * fma(a[i], b[i], acc) for i = l mod 16 in increasing i, then FADDV. */
static float dot16(const float* a, const float* b, uint32_t n) {
    float acc[16];
    for (int l = 0; l < 16; l++) acc[l] = 0.0f;
    for (uint32_t i = 0; i < n; i++) acc[i % 16] = fmaf(a[i], b[i], acc[i % 16]);
    return faddv16(acc);
}

/* Decode attention in the reference-arithmetic mode (the build's
 * composition of the handlers' arithmetic: the reference has no single-query
 * attention over a cache): for query head h and positions j < len of kv head
 * g = h / (n_heads / n_kv):  s_j = fl(dot16(q_h, k_j) * c), c = fl(1/sqrt(128)),
 * p = softmax_fp32(s), out_h[d] = FADDV of 16 lanes, lane l accumulating
 * fma(p_j, v_j[d], acc) for j = l mod 16 in increasing j.  k and v are fp16
 * [n_kv][ctx][128], widened exactly. */
void oracle_attention_ref(uint32_t n_heads, uint32_t n_kv, uint32_t len, uint32_t ctx, const float* q,
                          const uint16_t* kc, const uint16_t* vc, float* out) {
    const uint32_t G = n_heads / n_kv;
    const float c = f_of(0x3DB504F3u);
    float* s = (float*)malloc(sizeof(float) * (len ? len : 1));
    float* p = (float*)malloc(sizeof(float) * (len ? len : 1));
    float kj[128];
    for (uint32_t h = 0; h < n_heads; h++) {
        const uint32_t g = h / G;
        for (uint32_t j = 0; j < len; j++) {
            for (int d = 0; d < 128; d++) kj[d] = oracle_f16_to_f32(kc[((size_t)g * ctx + j) * 128 + d]);
            s[j] = dot16(q + (size_t)h * 128, kj, 128) * c;
        }
        oracle_softmax_fp32(len, s, p);
        for (int d = 0; d < 128; d++) {
            float acc[16];
            for (int l = 0; l < 16; l++) acc[l] = 0.0f;
            for (uint32_t j = 0; j < len; j++)
                acc[j % 16] = fmaf(p[j], oracle_f16_to_f32(vc[((size_t)g * ctx + j) * 128 + d]), acc[j % 16]);
            out[(size_t)h * 128 + d] = faddv16(acc);
        }
    }
    free(s);
    free(p);
}
