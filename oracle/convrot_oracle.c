/*
 * CPU restatement of the ConvRot W4A4 / W4A16 eager contract.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels are
 * compared against; it is never linked into the product library and nothing on
 * the product path may call it.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it.
 *
 * Every function restates one eager MLX function of the reference
 * (/root/reference/src/convrot_mlx/core.py) with the reference's per-operation
 * rounding: MLX evaluates each elementwise op on a bf16/f16 array by widening
 * to float32, computing, and rounding the result back to the array dtype with
 * round-to-nearest-even.  `rb()` below is that rounding.
 *
 * Build: gcc -O2 -std=c11 -fPIC -shared -ffp-contract=off -fno-fast-math
 * (contraction off so that a*b+c is two roundings, as in the eager graph).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* dtype codes shared with include/convrot_amd.h */
enum { CR_F32 = 0, CR_F16 = 1, CR_BF16 = 2 };

/* ---------------------------------------------------------------- rounding */

static inline uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* float32 -> bfloat16, round to nearest even; NaN stays a quiet NaN. */
uint16_t cr_f32_to_bf16(float x) {
    uint32_t u = f32_bits(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float cr_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* float32 -> IEEE binary16, round to nearest even, with subnormals and
 * overflow to infinity (the behaviour of a hardware RNE conversion). */
uint16_t cr_f32_to_f16(float x) {
    uint32_t u = f32_bits(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);           /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* rounds to inf */
    if (a >= 0x38800000u) {                                            /* normal f16 */
        uint32_t mant = a + 0xfffu + ((a >> 13) & 1u);                 /* RNE at bit 13 */
        return (uint16_t)(sign | ((mant - 0x38000000u) >> 13));
    }
    /* subnormal f16 (or zero): value = a * 2^24 in units of 2^-24 */
    if (a < 0x33000000u) return sign;                                  /* < 2^-25: rounds to 0 */
    {
        uint32_t e = a >> 23;                                          /* biased f32 exponent */
        uint32_t m = (a & 0x7fffffu) | 0x800000u;                      /* 24-bit significand */
        uint32_t shift = 126u - e;                                     /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
}

float cr_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1fu) return bits_f32(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f;                  /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* rb(): round a float32 result to the array dtype (core.py per-op semantics). */
static inline float rb(int dt, float x) {
    if (dt == CR_BF16) return cr_bf16_to_f32(cr_f32_to_bf16(x));
    if (dt == CR_F16) return cr_f16_to_f32(cr_f32_to_f16(x));
    return x;
}

static inline float load_elem(int dt, const void* p, int64_t i) {
    if (dt == CR_BF16) return cr_bf16_to_f32(((const uint16_t*)p)[i]);
    if (dt == CR_F16) return cr_f16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

static inline void store_elem(int dt, void* p, int64_t i, float v) {
    if (dt == CR_BF16) ((uint16_t*)p)[i] = cr_f32_to_bf16(v);
    else if (dt == CR_F16) ((uint16_t*)p)[i] = cr_f32_to_f16(v);
    else ((float*)p)[i] = v;
}

/* core.py:50-61 */
static int power_of_four(int g) {
    if (g < 4) return 0;
    while (g > 1 && g % 4 == 0) g /= 4;
    return g == 1;
}

/* ---------------------------------------------------------------- rotation */

/*
 * regular_hadamard (core.py:64-94).  Per feature group of G values, log4(G)
 * radix-4 stages with stride 1, 4, 16, ...; each stage maps (a, b, c, d) at
 * offsets {0,1,2,3}*stride to
 *     a + b + c - d,  a + b - c + d,  a - b + c + d,  -a + b + c + d
 * evaluated left to right with a dtype rounding after every add/subtract
 * (core.py:89-91), then divides by sqrt(G) and rounds (core.py:94).
 * `work` is the row buffer: K floats.
 */
static void hadamard_row(int dt, float* y, int64_t K, int G) {
    float tmp[4];
    for (int64_t g0 = 0; g0 < K; g0 += G) {
        float* v = y + g0;
        for (int stride = 1; stride < G; stride *= 4) {
            for (int blk = 0; blk < G; blk += 4 * stride) {
                for (int o = 0; o < stride; ++o) {
                    float a = v[blk + o], b = v[blk + o + stride];
                    float c = v[blk + o + 2 * stride], d = v[blk + o + 3 * stride];
                    tmp[0] = rb(dt, rb(dt, rb(dt, a + b) + c) - d);
                    tmp[1] = rb(dt, rb(dt, rb(dt, a + b) - c) + d);
                    tmp[2] = rb(dt, rb(dt, rb(dt, a - b) + c) + d);
                    tmp[3] = rb(dt, rb(dt, rb(dt, -a + b) + c) + d);
                    for (int j = 0; j < 4; ++j) v[blk + o + j * stride] = tmp[j];
                }
            }
        }
        /* y / math.sqrt(G): sqrt of a power of four is an exact power of two */
        float root = (float)sqrt((double)G);
        for (int i = 0; i < G; ++i) v[i] = rb(dt, v[i] / root);
    }
}

/* Returns 0, or -1 for an invalid group size / feature count. */
int cr_oracle_regular_hadamard(const void* x, int dt, int64_t rows, int64_t K, int G,
                               void* out, float* work) {
    if (!power_of_four(G) || K % G) return -1;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t k = 0; k < K; ++k) work[k] = load_elem(dt, x, r * K + k);
        hadamard_row(dt, work, K, G);
        for (int64_t k = 0; k < K; ++k) store_elem(dt, out, r * K + k, work[k]);
    }
    return 0;
}

/* ---------------------------------------------------------------- quantize */

/*
 * quantize_signed_int4_rowwise (core.py:149-158) on one row already in float
 * form (values exactly representable in dtype):
 *   absmax = max |x|                         (exact)
 *   absmax = max(absmax, dtype(1e-10))        (core.py:155)
 *   scale  = dtype(absmax / 7)                (core.py:156, INT4_MAX = 7)
 *   q      = clip(rint(dtype(x / scale)), -7, 7)   (core.py:157, round half even)
 * Writes one int8 code per feature and returns the scale as float32 (:158).
 */
static float quantize_row(int dt, const float* v, int64_t K, int8_t* codes) {
    float absmax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
        float a = fabsf(v[k]);
        if (a > absmax) absmax = a;
    }
    float floor_v = rb(dt, 1e-10f);
    if (floor_v > absmax) absmax = floor_v;
    float scale = rb(dt, absmax / 7.0f);
    for (int64_t k = 0; k < K; ++k) {
        float ratio = rb(dt, v[k] / scale);
        float q = rintf(ratio);
        if (q > 7.0f) q = 7.0f;
        if (q < -7.0f) q = -7.0f;
        if (q != q) q = 0.0f; /* 0/0 on an all-zero f16 row: outside the contract */
        codes[k] = (int8_t)q;
    }
    return scale;
}

int cr_oracle_quantize_rowwise(const void* x, int dt, int64_t rows, int64_t K,
                               int8_t* codes, float* scales, float* work) {
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t k = 0; k < K; ++k) work[k] = load_elem(dt, x, r * K + k);
        scales[r] = quantize_row(dt, work, K, codes + r * K);
    }
    return 0;
}

/* prepare_convrot_activation (core.py:161-167) and quantize_convrot_weight
 * (core.py:514-527): quantize_signed_int4_rowwise(regular_hadamard(x, G)). */
int cr_oracle_prepare(const void* x, int dt, int64_t rows, int64_t K, int G,
                      int8_t* codes, float* scales, float* work) {
    if (!power_of_four(G) || K % G) return -1;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t k = 0; k < K; ++k) work[k] = load_elem(dt, x, r * K + k);
        hadamard_row(dt, work, K, G);
        scales[r] = quantize_row(dt, work, K, codes + r * K);
    }
    return 0;
}

/* ---------------------------------------------------------------- matmuls */

/*
 * reference_w4a4_matmul (core.py:1155-1171): integer codes widened to float32,
 * an exact float32 matmul (every partial sum is an integer below 2^24 for the
 * supported K), then
 *     ((dot * xscales[m]) * wscales[n]) + bias[n]
 * as three separate float32 ops (core.py:1168-1170), then .astype(out dtype).
 * Takes unpacked codes: a_codes [M, K] and w_codes [N, K] (NK orientation).
 * Also writes the exact int32 dots when `dots` is non-null.
 */
int cr_oracle_w4a4_matmul(const int8_t* a_codes, const int8_t* w_codes,
                          const float* xscales, const float* wscales, const float* bias,
                          int64_t M, int64_t N, int64_t K, int out_dt, void* out,
                          int32_t* dots) {
    for (int64_t m = 0; m < M; ++m) {
        const int8_t* a = a_codes + m * K;
        for (int64_t n = 0; n < N; ++n) {
            const int8_t* w = w_codes + n * K;
            int64_t acc = 0;
            for (int64_t k = 0; k < K; ++k) acc += (int64_t)a[k] * (int64_t)w[k];
            if (dots) dots[m * N + n] = (int32_t)acc;
            float v = (float)acc;
            v = v * xscales[m];
            v = v * wscales[n];
            v = v + bias[n];
            store_elem(out_dt, out, m * N + n, v);
        }
    }
    return 0;
}

/*
 * The epilogue of reference_w4a4_matmul (core.py:1168-1171) applied to exact
 * integer dots computed elsewhere: ((dot * xscales[m]) * wscales[n]) + bias[n]
 * as three float32 ops, then .astype(out dtype).  cr_oracle_w4a4_matmul is
 * this loop fused with its int64 dot; the split form lets a caller compute the
 * dots of a large product by another exact method.
 */
int cr_oracle_w4a4_epilogue(const int32_t* dots, const float* xscales, const float* wscales,
                            const float* bias, int64_t M, int64_t N, int out_dt, void* out) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            float v = (float)dots[m * N + n];
            v = v * xscales[m];
            v = v * wscales[n];
            v = v + bias[n];
            store_elem(out_dt, out, m * N + n, v);
        }
    }
    return 0;
}

/*
 * mpp_w4a16_matmul (core.py:1123-1152): dots = act(float) . codes in float32
 * with an unspecified summation order (the Metal TensorOp), then
 * (dots * wscales[n]) + bias[n] as two float32 ops (core.py:1151) and
 * .astype(out dtype) (core.py:1152).  The oracle accumulates in double and
 * rounds the dot once to float32 (the most accurate member of the family of
 * valid orders); comparisons against it are tolerance-based.  `dots_out`, if
 * non-null, receives the float32 dots and `abs_out` the float32 value of
 * sum_k |act*code| (used to size the tolerance).
 */
int cr_oracle_w4a16_matmul(const void* act, int act_dt, const int8_t* w_codes,
                           const float* wscales, const float* bias,
                           int64_t M, int64_t N, int64_t K, int out_dt, void* out,
                           float* dots_out, float* abs_out) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            const int8_t* w = w_codes + n * K;
            double acc = 0.0, mag = 0.0;
            for (int64_t k = 0; k < K; ++k) {
                double t = (double)load_elem(act_dt, act, m * K + k) * (double)w[k];
                acc += t;
                mag += fabs(t);
            }
            float d = (float)acc;
            if (dots_out) dots_out[m * N + n] = d;
            if (abs_out) abs_out[m * N + n] = (float)mag;
            float v = d * wscales[n];
            v = v + bias[n];
            store_elem(out_dt, out, m * N + n, v);
        }
    }
    return 0;
}

/* Elementwise dtype conversions exposed for the test helpers. */
void cr_oracle_f32_to_dtype(const float* x, int64_t n, int dt, void* out) {
    for (int64_t i = 0; i < n; ++i) store_elem(dt, out, i, x[i]);
}

void cr_oracle_dtype_to_f32(const void* x, int64_t n, int dt, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = load_elem(dt, x, i);
}

/* ------------------------------------------------------ modulated producer */

/*
 * The fused producer's input transform (no reference counterpart: it is the
 * adaLN pattern `(1 + scale) * layer_norm(x) + shift` of a diffusion
 * transformer, evaluated as a bf16/f16 eager graph would):
 *   mean  = (float)(s1 / K)
 *   rstd  = (float)(1 / sqrt(max(s2 / K - (s1 / K)^2, 0) + eps))   (float64)
 *   ln    = rb((x - mean) * rstd)                                  (float32 ops)
 *   y     = rb(rb(rb(1 + scale) * ln) + shift)
 * with shift / scale row v = row / rows_per_vector.  s1 = sum x and
 * s2 = sum x*x are float64 sums in this fixed order: for each 1024-feature
 * block b, lane l (0..63) adds features b*1024 + 16l .. +15 in order
 * (features past K count as 0), the 64 lane sums are combined by the xor
 * butterfly  s[l] <- s[l] + s[l ^ m]  for m = 32, 16, 8, 4, 2, 1 (every lane
 * then holds the block sum), and the block sums are added in block order.
 */
static void block_moments(int dt, const void* x, int64_t r, int64_t K, int64_t b, double* b1, double* b2) {
    double s[64], q[64], t[64], u[64];
    for (int l = 0; l < 64; ++l) {
        double a1 = 0.0, a2 = 0.0;
        for (int j = 0; j < 16; ++j) {
            int64_t k = b * 1024 + 16 * l + j;
            double d = k < K ? (double)load_elem(dt, x, r * K + k) : 0.0;
            a1 += d;
            a2 += d * d;
        }
        s[l] = a1;
        q[l] = a2;
    }
    for (int m = 32; m >= 1; m >>= 1) {
        for (int l = 0; l < 64; ++l) {
            t[l] = s[l] + s[l ^ m];
            u[l] = q[l] + q[l ^ m];
        }
        for (int l = 0; l < 64; ++l) {
            s[l] = t[l];
            q[l] = u[l];
        }
    }
    *b1 = s[0];
    *b2 = q[0];
}

int cr_oracle_modulate(const void* x, int dt, int64_t rows, int64_t K, const void* shift, const void* scale,
                       int64_t rows_per_vector, float eps, void* out) {
    if (rows_per_vector <= 0) return -1;
    const int64_t blocks = (K + 1023) / 1024;
    for (int64_t r = 0; r < rows; ++r) {
        double s1 = 0.0, s2 = 0.0;
        for (int64_t b = 0; b < blocks; ++b) {
            double b1, b2;
            block_moments(dt, x, r, K, b, &b1, &b2);
            s1 += b1;
            s2 += b2;
        }
        double m64 = s1 / (double)K;
        double var = s2 / (double)K - m64 * m64;
        if (var < 0.0) var = 0.0;
        float mean = (float)m64;
        float rstd = (float)(1.0 / sqrt(var + (double)eps));
        int64_t vrow = r / rows_per_vector;
        for (int64_t k = 0; k < K; ++k) {
            float ln = rb(dt, (load_elem(dt, x, r * K + k) - mean) * rstd);
            float one_plus = rb(dt, 1.0f + load_elem(dt, scale, vrow * K + k));
            float y = rb(dt, rb(dt, one_plus * ln) + load_elem(dt, shift, vrow * K + k));
            store_elem(dt, out, r * K + k, y);
        }
    }
    return 0;
}

/* ------------------------------------------------- tanh GELU (producer input)
 *
 * Input transform of the fused GELU producer; it has no reference counterpart.
 * The FLUX MLP activation nn.GELU(approximate="tanh"),
 *   gelu(x) = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))),
 * evaluated in float32 in this fixed sequence, rounded once to the dtype:
 *   x3    = (x * x) * x
 *   u     = kBeta * fma(kKappa, x3, x)
 *   q     = 2 / (exp(2|u|) + 1)            (q = 0 where 2|u| > 88 or u is NaN)
 *   onept = u >= 0 ? 2 - q : q             (= 1 + tanh(u), without cancellation)
 *   y     = (0.5 * x) * onept
 * exp(z), 0 <= z <= 88, is Cody-Waite reduced, z = n ln2 + r with
 * n = rint(z log2 e), r = fma(-n, ln2_lo, fma(-n, ln2_hi, z)), |r| <= ln2/2, then
 * 2^n times the degree-7 Taylor polynomial of e^r (Horner, fma), whose
 * truncation error r^8/8! < 6e-9 is below float32 resolution.  Every step is an
 * IEEE float32 operation (+ - * /, fma, rint, ldexp), so any IEEE machine that
 * runs the same sequence (the HIP producer kernel does) gets the same bits.
 */
#define GELU_BETA 0x1.988454p-1f   /* float32(sqrt(2/pi)) */
#define GELU_KAPPA 0x1.6e4e26p-5f  /* float32(0.044715) */
#define EXP_LOG2E 0x1.715476p+0f
#define EXP_LN2_HI 0x1.62e4p-1f
#define EXP_LN2_LO 0x1.7f7d1cp-20f

static float gelu_tanh32(float x) {
    const float x3 = (x * x) * x;
    const float u = GELU_BETA * fmaf(GELU_KAPPA, x3, x);
    const float z = fabsf(u) + fabsf(u);
    float q = 0.0f;
    if (z <= 88.0f) {
        const float n = rintf(z * EXP_LOG2E);
        float r = fmaf(-n, EXP_LN2_HI, z);
        r = fmaf(-n, EXP_LN2_LO, r);
        float p = 0x1.a01a02p-13f;         /* 1/7! */
        p = fmaf(p, r, 0x1.6c16c2p-10f);   /* 1/6! */
        p = fmaf(p, r, 0x1.111112p-7f);    /* 1/5! */
        p = fmaf(p, r, 0x1.555556p-5f);    /* 1/4! */
        p = fmaf(p, r, 0x1.555556p-3f);    /* 1/3! */
        p = fmaf(p, r, 0x1p-1f);           /* 1/2! */
        p = fmaf(p, r, 1.0f);
        p = fmaf(p, r, 1.0f);
        q = 2.0f / (ldexpf(p, (int)n) + 1.0f);
    }
    const float onept = u >= 0.0f ? 2.0f - q : q;
    return (0.5f * x) * onept;
}

int cr_oracle_gelu(const void* x, int dt, int64_t n, void* out) {
    for (int64_t i = 0; i < n; ++i) store_elem(dt, out, i, rb(dt, gelu_tanh32(load_elem(dt, x, i))));
    return 0;
}
