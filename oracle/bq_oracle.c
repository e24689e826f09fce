/*
 * bq_oracle.c -- CPU restatement of the reference's quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for libbq.so, never part of it.
 * Built with -O2 -ffp-contract=off (no fast-math) so every fp32 expression is
 * evaluated exactly as written.  See bq_oracle.h for how each function is pinned.
 */
#include "bq_oracle.h"

#include <math.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* synthetic data: splitmix64 + Box-Muller (double precision, then rounded)   */
/* ------------------------------------------------------------------------- */
static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void orc_gaussian(uint64_t seed, float mean, float std, float* out, size_t n) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        /* 53-bit uniforms in (0,1] and [0,1) */
        double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(mean + std * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(mean + std * r * sin(two_pi * u2));
    }
}

/* ------------------------------------------------------------------------- */
/* fp16                                                                       */
/* ------------------------------------------------------------------------- */
/* bruce.cu:4768-4781: a zero exponent is a denormal m * 2^-24, not zero. */
float orc_h2f(uint16_t h) {
    const uint32_t sg = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        const float f = (float)m * 5.9604644775390625e-8f;
        return (h & 0x8000u) ? -f : f;
    }
    uint32_t x = (e == 31) ? (sg | 0x7F800000u | (m << 13)) : (sg | ((e + 112u) << 23) | (m << 13));
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* IEEE binary32 -> binary16, round to nearest even (what __float2half does). */
uint16_t orc_f2h_rn(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) /* inf / nan */
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) /* rounds to >= 65520 -> inf */
        return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) { /* result is a half denormal or zero: value / 2^-24 */
        if (ax < 0x33000000u) return sign; /* < 2^-25 rounds to 0 (2^-25 exactly ties to 0) */
        const uint32_t e = ax >> 23;                 /* 102..112 */
        const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t shift = 126u - e;             /* 14..24 */
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t halfw = 1u << (shift - 1u);
        if (rem > halfw || (rem == halfw && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    /* normal half */
    uint32_t e = (ax >> 23) - 112u;
    uint32_t mant = ax & 0x7FFFFFu;
    uint32_t q = (e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------------------- */
/* activation quantizer: bruce.cu:518-539 (k_q8_quant), :1081-1108 (k_q8_rows) */
/* ------------------------------------------------------------------------- */
/* __float2int_rn as the PTX ISA defines cvt.rni.s32.f32: round to nearest
 * even, NaN -> 0, out-of-range values (infinities included) saturate to
 * INT_MIN / INT_MAX.  The quantizer needs it when 0 < amax < 127 * 2^-128:
 * d is then denormal and id = 1/d = inf, so v * id is NaN for v = 0 and
 * +-inf otherwise. */
static int cvt_rni(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.f) return 2147483647;
    if (f <= -2147483648.f) return -2147483647 - 1;
    return (int)rintf(f);
}

void orc_q8_rows(const float* x, int M, int K, int8_t* xq, float* xd, int32_t* xsum) {
    const int nb = K / 32;
    for (int r = 0; r < M; ++r) {
        for (int b = 0; b < nb; ++b) {
            const float* p = x + (size_t)r * K + (size_t)b * 32;
            float amax = 0.f;
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(p[i]));
            const float d = amax * (1.f / 127.f);
            const float id = d > 0.f ? 1.f / d : 0.f;
            int s = 0;
            for (int i = 0; i < 32; ++i) {
                int v = cvt_rni(p[i] * id);
                v = v < -127 ? -127 : (v > 127 ? 127 : v);
                xq[(size_t)r * K + (size_t)b * 32 + i] = (int8_t)v;
                s += v;
            }
            xd[(size_t)r * nb + b] = d;
            xsum[(size_t)r * nb + b] = s;
        }
    }
}

void orc_fill_xdh(const float* xd, const int32_t* xsum, size_t n, uint16_t* xdh) {
    for (size_t i = 0; i < n; ++i) xdh[i] = orc_f2h_rn(xd[i] * (float)xsum[i]);
}

/* ------------------------------------------------------------------------- */
/* format decode (GGUF k-quant layouts, restated from bruce.cu / ref_np.py)   */
/* ------------------------------------------------------------------------- */
void orc_q5k_scale(const uint8_t* s, int js, int* sc, int* m) {
    if (js < 4) {
        *sc = s[js] & 63;
        *m = s[js + 4] & 63;
    } else {
        const int lo = s[js + 4];
        *sc = (lo & 0xF) | ((s[js - 4] >> 6) << 4);
        *m = (lo >> 4) | ((s[js] >> 6) << 4);
    }
}

int orc_q5k_code(const uint8_t* blk, int k) {
    const int j = k >> 5, l = k & 31;
    const int lo = (blk[48 + 32 * (j >> 1) + l] >> (4 * (j & 1))) & 0xF;
    const int hi = (blk[16 + l] >> j) & 1;
    return lo | (hi << 4);
}

int orc_q6k_code(const uint8_t* blk, int k) {
    const int h = k >> 7, u = (k >> 5) & 3, l = k & 31;
    const uint8_t qlb = blk[64 * h + 32 * (u & 1) + l];
    const int lo = (u < 2) ? (qlb & 0xF) : (qlb >> 4);
    const int hi = (blk[128 + 32 * h + l] >> (2 * u)) & 3;
    return lo | (hi << 4);
}

int orc_q6k_sc(const uint8_t* blk, int k) { return (int)(int8_t)blk[192 + (k >> 4)]; }

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

void orc_dequant_q5k(const uint8_t* raw, int N, int K, float* out) {
    const int nsb = K / 256;
    for (int n = 0; n < N; ++n)
        for (int sb = 0; sb < nsb; ++sb) {
            const uint8_t* b = raw + ((size_t)n * nsb + sb) * 176;
            const float d = orc_h2f(rd16(b)), dmin = orc_h2f(rd16(b + 2));
            for (int j = 0; j < 8; ++j) {
                int sc, m;
                orc_q5k_scale(b + 4, j, &sc, &m);
                const float d1 = d * (float)sc, m1 = dmin * (float)m;
                for (int l = 0; l < 32; ++l)
                    out[(size_t)n * K + sb * 256 + 32 * j + l] = d1 * (float)orc_q5k_code(b, 32 * j + l) - m1;
            }
        }
}

void orc_dequant_q6k(const uint8_t* raw, int N, int K, float* out) {
    const int nsb = K / 256;
    for (int n = 0; n < N; ++n)
        for (int sb = 0; sb < nsb; ++sb) {
            const uint8_t* b = raw + ((size_t)n * nsb + sb) * 210;
            const float d = orc_h2f(rd16(b + 208));
            for (int k = 0; k < 256; ++k)
                out[(size_t)n * K + sb * 256 + k] =
                    d * (float)orc_q6k_sc(b, k) * (float)(orc_q6k_code(b, k) - 32);
        }
}

/* ------------------------------------------------------------------------- */
/* encoders (own design).  Deterministic; both the GPU path and the oracle    */
/* consume the same bytes, so only validity and determinism matter.           */
/* ------------------------------------------------------------------------- */
static int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

void orc_quantize_q5k(const float* w, int N, int K, uint8_t* out) {
    const int nsb = K / 256;
    for (int n = 0; n < N; ++n)
        for (int sb = 0; sb < nsb; ++sb) {
            const float* v = w + (size_t)n * K + (size_t)sb * 256;
            uint8_t* b = out + ((size_t)n * nsb + sb) * 176;
            memset(b, 0, 176);
            float scf[8], mnf[8], maxs = 0.f, maxm = 0.f;
            for (int j = 0; j < 8; ++j) {
                float lo = v[32 * j], hi = v[32 * j];
                for (int l = 1; l < 32; ++l) {
                    lo = fminf(lo, v[32 * j + l]);
                    hi = fmaxf(hi, v[32 * j + l]);
                }
                mnf[j] = lo < 0.f ? -lo : 0.f;
                scf[j] = (hi + mnf[j]) / 31.f;
                maxs = fmaxf(maxs, scf[j]);
                maxm = fmaxf(maxm, mnf[j]);
            }
            const uint16_t dh = orc_f2h_rn(maxs / 63.f), mh = orc_f2h_rn(maxm / 63.f);
            const float d = orc_h2f(dh), dmin = orc_h2f(mh);
            int sc[8], m[8];
            for (int j = 0; j < 8; ++j) {
                sc[j] = d > 0.f ? clampi((int)ceilf(scf[j] / d), 0, 63) : 0;
                m[j] = dmin > 0.f ? clampi((int)ceilf(mnf[j] / dmin), 0, 63) : 0;
            }
            b[0] = (uint8_t)(dh & 0xFF); b[1] = (uint8_t)(dh >> 8);
            b[2] = (uint8_t)(mh & 0xFF); b[3] = (uint8_t)(mh >> 8);
            uint8_t* s = b + 4;
            for (int j = 0; j < 4; ++j) {
                s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
                s[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
                s[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
            }
            for (int j = 0; j < 8; ++j) {
                const float ds = d * (float)sc[j], dm = dmin * (float)m[j];
                for (int l = 0; l < 32; ++l) {
                    int u = ds > 0.f ? (int)rintf((v[32 * j + l] + dm) / ds) : 0;
                    u = clampi(u, 0, 31);
                    b[48 + 32 * (j >> 1) + l] |= (uint8_t)((u & 0xF) << (4 * (j & 1)));
                    b[16 + l] |= (uint8_t)(((u >> 4) & 1) << j);
                }
            }
        }
}

void orc_quantize_q6k(const float* w, int N, int K, uint8_t* out) {
    const int nsb = K / 256;
    for (int n = 0; n < N; ++n)
        for (int sb = 0; sb < nsb; ++sb) {
            const float* v = w + (size_t)n * K + (size_t)sb * 256;
            uint8_t* b = out + ((size_t)n * nsb + sb) * 210;
            memset(b, 0, 210);
            float sf[16], maxs = 0.f;
            for (int g = 0; g < 16; ++g) {
                float amax = 0.f, vmax = 0.f;
                for (int l = 0; l < 16; ++l) {
                    const float a = fabsf(v[16 * g + l]);
                    if (a > amax) { amax = a; vmax = v[16 * g + l]; }
                }
                /* signed group scale: the largest-magnitude value maps to code +31 */
                sf[g] = (vmax < 0.f ? -amax : amax) / 31.f;
                maxs = fmaxf(maxs, amax / 31.f);
            }
            const uint16_t dh = orc_f2h_rn(maxs / 127.f);
            const float d = orc_h2f(dh);
            b[208] = (uint8_t)(dh & 0xFF); b[209] = (uint8_t)(dh >> 8);
            for (int g = 0; g < 16; ++g) {
                int sc = 0;
                if (d > 0.f) {
                    const float r = sf[g] / d;
                    sc = clampi((int)(r < 0.f ? floorf(r) : ceilf(r)), -127, 127);
                }
                b[192 + g] = (uint8_t)(int8_t)sc;
                const float scale = d * (float)sc;
                for (int l = 0; l < 16; ++l) {
                    const int k = 16 * g + l;
                    int q = scale != 0.f ? (int)rintf(v[k] / scale) : 0;
                    q = clampi(q, -32, 31) + 32;
                    const int h = k >> 7, u = (k >> 5) & 3, ll = k & 31;
                    b[64 * h + 32 * (u & 1) + ll] |= (uint8_t)((q & 0xF) << (u < 2 ? 0 : 4));
                    b[128 + 32 * h + ll] |= (uint8_t)(((q >> 4) & 3) << (2 * u));
                }
            }
        }
}

/* ------------------------------------------------------------------------- */
/* integer dots (gemvbench.cu:405-430 sub_stats)                              */
/* ------------------------------------------------------------------------- */
void orc_dots_q5k(const uint8_t* raw, const int8_t* xq, int M, int N, int K, int32_t* dots) {
    const int nsb = K / 256, nb = K / 32;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n)
            for (int g = 0; g < nb; ++g) {
                const uint8_t* b = raw + ((size_t)n * nsb + g / 8) * 176;
                int32_t acc = 0;
                for (int l = 0; l < 32; ++l)
                    acc += orc_q5k_code(b, 32 * (g % 8) + l) * (int32_t)xq[(size_t)m * K + 32 * g + l];
                dots[((size_t)m * N + n) * nb + g] = acc;
            }
}

void orc_dots16_q6k(const uint8_t* raw, const int8_t* xq, int M, int N, int K, int32_t* dots) {
    const int nsb = K / 256, nb = K / 16;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n)
            for (int g = 0; g < nb; ++g) {
                const uint8_t* b = raw + ((size_t)n * nsb + g / 16) * 210;
                int32_t acc = 0;
                for (int l = 0; l < 16; ++l)
                    acc += (orc_q6k_code(b, 16 * (g % 16) + l) - 32) * (int32_t)xq[(size_t)m * K + 16 * g + l];
                dots[((size_t)m * N + n) * nb + g] = acc;
            }
}

/* ------------------------------------------------------------------------- */
/* GEMM references                                                            */
/* ------------------------------------------------------------------------- */
/* mmq_test.cu:269-294, evaluated in double from the exact fp32 ds / dm. */
void orc_gemm_q5k(const uint8_t* raw, const int8_t* xq, const float* xd, const int32_t* xsum,
                  int M, int N, int K, double* y) {
    const int nsb = K / 256, nb = K / 32;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int sb = 0; sb < nsb; ++sb) {
                const uint8_t* b = raw + ((size_t)n * nsb + sb) * 176;
                const float d = orc_h2f(rd16(b)), dmin = orc_h2f(rd16(b + 2));
                for (int j = 0; j < 8; ++j) {
                    int sc, mm;
                    orc_q5k_scale(b + 4, j, &sc, &mm);
                    const float ds = d * (float)sc, dm = dmin * (float)mm; /* exact in fp32 */
                    const int g = sb * 8 + j;
                    int32_t dot = 0;
                    for (int l = 0; l < 32; ++l)
                        dot += orc_q5k_code(b, 32 * j + l) * (int32_t)xq[(size_t)m * K + 32 * g + l];
                    acc += (double)xd[(size_t)m * nb + g] *
                           ((double)ds * (double)dot - (double)dm * (double)xsum[(size_t)m * nb + g]);
                }
            }
            y[(size_t)m * N + n] = acc;
        }
}

/* The reference's scalar host loop, fp32 and serial (mmq_test.cu:269-294).
 * This is the CPU baseline that bench.py times. */
void orc_gemm_q5k_f32(const uint8_t* raw, const int8_t* xq, const float* xd, const int32_t* xsum,
                      int M, int N, int K, float* y) {
    const int nsb = K / 256, nb = K / 32;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float acc = 0.f;
            for (int sb = 0; sb < nsb; ++sb) {
                const uint8_t* wb = raw + ((size_t)n * nsb + sb) * 176;
                const float d = orc_h2f(rd16(wb)), dmin = orc_h2f(rd16(wb + 2));
                for (int j = 0; j < 8; ++j) {
                    int sc, mm;
                    orc_q5k_scale(wb + 4, j, &sc, &mm);
                    const float ds = d * (float)sc, dm = dmin * (float)mm;
                    const int kb = sb * 8 + j;
                    int dot = 0;
                    for (int o = 0; o < 32; ++o) {
                        const int u = ((wb[48 + 32 * (j >> 1) + o] >> (4 * (j & 1))) & 0xF) |
                                      (((wb[16 + o] >> j) & 1) << 4);
                        dot += u * (int)xq[(size_t)m * K + kb * 32 + o];
                    }
                    acc += xd[(size_t)m * nb + kb] * (ds * (float)dot - dm * (float)xsum[(size_t)m * nb + kb]);
                }
            }
            y[(size_t)m * N + n] = acc;
        }
}

/* Q6_K: bruce.cu:4330-4345 (per 16-value group scale d*sc, per 32-group xd). */
void orc_gemm_q6k(const uint8_t* raw, const int8_t* xq, const float* xd,
                  int M, int N, int K, double* y) {
    const int nsb = K / 256, nb = K / 32;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int sb = 0; sb < nsb; ++sb) {
                const uint8_t* b = raw + ((size_t)n * nsb + sb) * 210;
                const float d = orc_h2f(rd16(b + 208));
                for (int g16 = 0; g16 < 16; ++g16) {
                    const float scl = d * (float)orc_q6k_sc(b, 16 * g16); /* exact */
                    int32_t dot = 0;
                    for (int l = 0; l < 16; ++l) {
                        const int k = 16 * g16 + l;
                        dot += (orc_q6k_code(b, k) - 32) * (int32_t)xq[(size_t)m * K + sb * 256 + k];
                    }
                    acc += (double)xd[(size_t)m * nb + sb * 8 + g16 / 2] * (double)scl * (double)dot;
                }
            }
            y[(size_t)m * N + n] = acc;
        }
}

void orc_gemm_q6k_f32(const uint8_t* raw, const int8_t* xq, const float* xd,
                      int M, int N, int K, float* y) {
    const int nsb = K / 256, nb = K / 32;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            float acc = 0.f;
            for (int sb = 0; sb < nsb; ++sb) {
                const uint8_t* b = raw + ((size_t)n * nsb + sb) * 210;
                const float d = orc_h2f(rd16(b + 208));
                for (int g16 = 0; g16 < 16; ++g16) {
                    const float scl = d * (float)(int8_t)b[192 + g16];
                    int dot = 0;
                    for (int l = 0; l < 16; ++l) {
                        const int k = 16 * g16 + l, h = k >> 7, u = (k >> 5) & 3, ll = k & 31;
                        const uint8_t qlb = b[64 * h + 32 * (u & 1) + ll];
                        const int q = ((u < 2) ? (qlb & 0xF) : (qlb >> 4)) | (((b[128 + 32 * h + ll] >> (2 * u)) & 3) << 4);
                        dot += (q - 32) * (int)xq[(size_t)m * K + sb * 256 + k];
                    }
                    acc += xd[(size_t)m * nb + sb * 8 + g16 / 2] * scl * (float)dot;
                }
            }
            y[(size_t)m * N + n] = acc;
        }
}

/* bruce.cu:6615-6790: main term from the 144 B stages, min term from fp16 Dm x fp16 xdh. */
void orc_gemm_q5k_144(const uint8_t* w144, const uint16_t* dm, const int8_t* xq, const float* xd,
                      const uint16_t* xdh, int M, int N, int K, double* y) {
    const int nb = K / 32, nst = K / 128;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int s = 0; s < nst; ++s) {
                const uint8_t* st = w144 + ((size_t)s * N + n) * 144;
                float ds4[4];
                memcpy(ds4, st + 128, 16);
                for (int q = 0; q < 4; ++q) {
                    int32_t dot = 0;
                    for (int l = 0; l < 32; ++l)
                        dot += (int32_t)(int8_t)st[32 * q + l] * (int32_t)xq[(size_t)m * K + 128 * s + 32 * q + l];
                    acc += (double)ds4[q] * (double)xd[(size_t)m * nb + 4 * s + q] * (double)dot;
                }
            }
            for (int g = 0; g < nb; ++g)
                acc += (double)orc_h2f(dm[(size_t)n * nb + g]) * (double)orc_h2f(xdh[(size_t)m * nb + g]);
            y[(size_t)m * N + n] = acc;
        }
}

/* ------------------------------------------------------------------------- */
/* load-time repacks                                                          */
/* ------------------------------------------------------------------------- */
/* bruce.cu:5756-5789 index map: stage-major [K/128][N][144]. */
void orc_repack_q5k_144(const uint8_t* raw, int K, int N, uint8_t* w144, uint16_t* dmo) {
    const int nsb = K / 256, nb = K / 32;
    for (int n = 0; n < N; ++n)
        for (int sb = 0; sb < nsb; ++sb) {
            const uint8_t* b = raw + ((size_t)n * nsb + sb) * 176;
            const float d = orc_h2f(rd16(b)), dmin = orc_h2f(rd16(b + 2));
            for (int hh = 0; hh < 2; ++hh) {
                uint8_t* o = w144 + ((size_t)(sb * 2 + hh) * N + n) * 144;
                for (int i = 0; i < 128; ++i) o[i] = (uint8_t)orc_q5k_code(b, 128 * hh + i);
                for (int q = 0; q < 4; ++q) {
                    int sc, mm;
                    const int j = 4 * hh + q;
                    orc_q5k_scale(b + 4, j, &sc, &mm);
                    const float ds = d * (float)sc, dm = dmin * (float)mm;
                    memcpy(o + 128 + 4 * q, &ds, 4);
                    dmo[(size_t)n * nb + sb * 8 + j] = orc_f2h_rn(-dm);
                }
            }
        }
}

/* bruce.cu:4783-4811: row-major [N][K/128][160]. */
void orc_repack_q6k_160(const uint8_t* raw, int K, int N, uint8_t* dst) {
    const int nsb = K / 256, nst = K / 128;
    for (int n = 0; n < N; ++n)
        for (int h = 0; h < nst; ++h) {
            const uint8_t* b = raw + ((size_t)n * nsb + h / 2) * 210;
            uint8_t* o = dst + ((size_t)n * nst + h) * 160;
            const float d = orc_h2f(rd16(b + 208));
            for (int i = 0; i < 128; ++i)
                o[i] = (uint8_t)(int8_t)(orc_q6k_code(b, 128 * (h & 1) + i) - 32);
            for (int g = 0; g < 8; ++g) {
                const float s = d * (float)(int8_t)b[192 + 8 * (h & 1) + g];
                memcpy(o + 128 + 4 * g, &s, 4);
            }
        }
}

/* ------------------------------------------------------------------------- */
/* Q8_0 logits head                                                           */
/* ------------------------------------------------------------------------- */
static float bf16_to_f32(uint16_t b) {
    const uint32_t x = (uint32_t)b << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* bruce.cu:4843-4867 (q8k_quant_host) and :5162-5184 (k_bf16_to_q8, its device
 * twin and the load path in use): per 32 values d = amax*(1/127),
 * id = d>0 ? 1/d : 0, q = clamp(rint(v*id), -127, 127); the scale is stored as
 * half_rn(d). */
void orc_quantize_q8s(const uint16_t* bf16, int K, int N, uint8_t* dst) {
    const int nsb = K / 256;
    for (int r = 0; r < N; ++r)
        for (int s = 0; s < nsb; ++s) {
            uint8_t* blk = dst + ((size_t)r * nsb + s) * 272;
            for (int g = 0; g < 8; ++g) {
                const uint16_t* p = bf16 + (size_t)r * K + (size_t)s * 256 + (size_t)g * 32;
                float amax = 0.f;
                for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(bf16_to_f32(p[i])));
                const float d = amax * (1.f / 127.f);
                const float id = d > 0.f ? 1.f / d : 0.f;
                const uint16_t h = orc_f2h_rn(d);
                memcpy(blk + 2 * g, &h, 2);
                for (int i = 0; i < 32; ++i) {
                    /* the device kernel's __float2int_rn, then the clamp (the host
                     * loop's lrintf(v*id) is undefined when id overflows to inf:
                     * the device result is kept) */
                    int v = cvt_rni(bf16_to_f32(p[i]) * id);
                    v = v < -127 ? -127 : (v > 127 ? 127 : v);
                    blk[16 + 32 * g + i] = (uint8_t)(int8_t)v;
                }
            }
        }
}

/* bruce.cu:4409-4449: acc += ws * xd * dot per 32-value group, then * rs[row]. */
void orc_gemv_q8s(const uint8_t* w, int K, int N, int M, const int8_t* xq, const float* xd,
                  const float* rs, double* y) {
    const int nsb = K / 256, nb = K / 32;
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double acc = 0.0;
            for (int s = 0; s < nsb; ++s) {
                const uint8_t* blk = w + ((size_t)n * nsb + s) * 272;
                for (int g = 0; g < 8; ++g) {
                    uint16_t h;
                    memcpy(&h, blk + 2 * g, 2);
                    int32_t dot = 0;
                    for (int i = 0; i < 32; ++i)
                        dot += (int32_t)(int8_t)blk[16 + 32 * g + i] *
                               (int32_t)xq[(size_t)m * K + (size_t)s * 256 + 32 * g + i];
                    acc += (double)orc_h2f(h) * (double)xd[(size_t)m * nb + s * 8 + g] * (double)dot;
                }
            }
            y[(size_t)m * N + n] = rs ? acc * (double)rs[n] : acc;
        }
}

/* ------------------------------------------------------------------------- */
/* q8 producers: elementwise op -> L2 norm (bruce.cu:541-641, 1110-1228)      */
/* ------------------------------------------------------------------------- */
/* l2_scale (bruce.cu:305-307) with eps = 1e-6f (:73), in double */
static double l2_scale_d(double ss, int n) {
    const double eps = (double)1e-6f;
    return (1.0 / sqrt(ss / n + eps / n)) * (1.0 / sqrt((double)n));
}

void orc_norm_rows(int op, const float* a, const float* b, const float* c, const float* d, int rows, int n,
                   double* out) {
    for (int m = 0; m < rows; ++m) {
        const float* ar = a + (size_t)m * n;
        const float* br = b ? b + (size_t)m * n : 0;
        double* o = out + (size_t)m * n;
        if (op == 2) { /* k_resid :571-600 */
            double sa = 0.0, sb = 0.0;
            for (int i = 0; i < n; ++i) { sa += (double)ar[i] * ar[i]; sb += (double)br[i] * br[i]; }
            const double ka = l2_scale_d(sa, n), kb = l2_scale_d(sb, n);
            for (int i = 0; i < n; ++i) {
                const double an = ar[i] * ka, bn = br[i] * kb;
                o[i] = an + (bn - an) * c[i];
            }
        } else {
            for (int i = 0; i < n; ++i) {
                double t;
                if (op == 0) t = ar[i];                         /* k_norm :541-554 */
                else if (op == 1) t = (double)ar[i] + br[i];     /* k_add_norm :556-569 */
                else if (op == 3) t = ar[i] / (1.0 + exp(-((double)br[i] * c[i])));  /* k_gate_norm :602-620 */
                else {                                           /* k_silu_mul_norm :622-641 */
                    const double gv = (double)ar[i] * c[i];
                    t = gv / (1.0 + exp(-gv)) * br[i] * d[i];
                }
                o[i] = t;
            }
        }
        double ss = 0.0;
        for (int i = 0; i < n; ++i) ss += o[i] * o[i];
        const double k = l2_scale_d(ss, n);
        for (int i = 0; i < n; ++i) o[i] *= k;
    }
}
