/*
 * mt_oracle.c -- CPU oracle for the MingTTS linear hot path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or as the timed CPU baseline).  The HIP library never links it and
 * has no CPU fallback.
 *
 * What it restates (paths relative to the reference checkout):
 *   - the known-answer-test RNG, a 64-bit LCG giving uniforms in [-1, 1)
 *       Tests/MingTTSTests/KernelTests.swift:21-28
 *   - bf16 round-to-nearest-even of an fp32 value
 *       Tests/MingTTSTests/KernelTests.swift:30-36
 *   - the seeded standard normals, SplitMix64 + Box-Muller
 *       Sources/MingTTS/Engine/Engine.swift:432-453
 *   - the CPU reference loop of one linear: per output element an fp32
 *     accumulate over K in natural order, then the epilogue
 *       Tests/MingTTSTests/KernelTests.swift:86-101
 *     with the epilogue order of the kernels (bias, SiLU-gate, GELU, SiLU,
 *     accumulate) and the clamped tanh-GELU
 *       Sources/MingTTS/Engine/Shaders.swift:21-29, 92-103
 *   - an fp64 recomputation of the same linear on the same rounded inputs,
 *     the precision gate for every configuration.
 *
 * fp16 encode/decode are written from the IEEE 754 binary16 definition (gcc 11
 * has no _Float16 on x86-64); they are pinned against numpy's float16 over all
 * 65536 bit patterns by the CPU tests.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#if defined(__F16C__) && defined(__AVX2__) && defined(__FMA__)
#include <immintrin.h>
#define MTO_HAVE_F16C 1
#endif

enum { MTO_F32 = 0, MTO_F16 = 1, MTO_BF16 = 2 };
enum { MTO_BIAS = 1, MTO_ACCUM = 2, MTO_GELU = 4, MTO_SILU_GATE = 8, MTO_SILU = 16 };

/* ---------------------------------------------------------------- RNGs -- */

/* KernelTests.swift:21-28: state = state * 6364136223846793005 + 1442695040888963407
 * (wrapping), value = (state >> 40) / 2^24 * 2 - 1, then * scale, all in fp32. */
uint64_t mto_lcg_fill(uint64_t state, float *out, int64_t n, float scale) {
    for (int64_t i = 0; i < n; i++) {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        float v = (float)(state >> 40) / 16777216.0f * 2.0f - 1.0f;
        out[i] = v * scale;
    }
    return state;
}

/* Engine.swift:432-453.  The stream's t-th draw (t = 1, 2, ...) is SplitMix64's
 * output for the state seed + golden + t * golden (the reference starts its state
 * at seed + golden), so pair j (draws 2j+1, 2j+2) is independent of the others and
 * the fill parallelises without changing a single bit. */
uint64_t mto_splitmix64(uint64_t seed, uint64_t t) {
    const uint64_t golden = 0x9E3779B97F4A7C15ULL;
    uint64_t z = seed + golden + t * golden;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static double mto_splitmix_u01(uint64_t seed, uint64_t t) {
    return (double)(mto_splitmix64(seed, t) >> 11) / 9007199254740992.0; /* 2^53 */
}

void mto_gaussian_fill(uint64_t seed, float *out, int64_t n, float scale) {
    const int64_t pairs = (n + 1) / 2;
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < pairs; j++) {
        double u1 = mto_splitmix_u01(seed, (uint64_t)(2 * j + 1));
        double u2 = mto_splitmix_u01(seed, (uint64_t)(2 * j + 2));
        if (u1 < 1e-300) u1 = 1e-300;
        double r = sqrt(-2.0 * log(u1));
        double a = 2.0 * 3.14159265358979323846 * u2;
        out[2 * j] = (float)(r * cos(a)) * scale;
        if (2 * j + 1 < n) out[2 * j + 1] = (float)(r * sin(a)) * scale;
    }
}

/* ------------------------------------------------------------ rounding -- */

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* KernelTests.swift:30-36: bits + 0x7FFF + ((bits >> 16) & 1), keep the top 16. */
uint16_t mto_bf16_bits(float x) {
    uint32_t u = f2u(x);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

float mto_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16, round to nearest even, overflow to infinity, NaN kept quiet. */
uint16_t mto_f16_bits(float x) {
    uint32_t u = f2u(x);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t exp = (u >> 23) & 0xFFu;
    uint32_t man = u & 0x7FFFFFu;
    if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u | (man >> 13) : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        /* subnormal half (or zero): value = m * 2^-24 with m < 1024 */
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;          /* 24-bit significand */
        int shift = 14 - e;                    /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);           /* q may carry into the exponent: still correct */
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;  /* carry may reach inf: correct */
    return (uint16_t)(sign | q);
}

float mto_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    if (exp == 0x1Fu) return u2f(sign | 0x7F800000u | (man << 13));
    if (exp == 0) {
        float v = (float)man * 5.9604644775390625e-08f; /* 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* Round an fp32 array to a 16-bit type: bits out, and the rounded values back in fp32. */
void mto_round16(const float *in, int64_t n, int dtype, uint16_t *bits, float *rounded) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; i++) {
        uint16_t b = dtype == MTO_BF16 ? mto_bf16_bits(in[i]) : mto_f16_bits(in[i]);
        if (bits) bits[i] = b;
        if (rounded) rounded[i] = dtype == MTO_BF16 ? mto_bf16_to_f32(b) : mto_f16_to_f32(b);
    }
}

/* Decode 16-bit storage to fp32. */
void mto_decode16(const uint16_t *bits, int64_t n, int dtype, float *out) {
#pragma omp parallel for schedule(static) if (n > 65536)
    for (int64_t i = 0; i < n; i++)
        out[i] = dtype == MTO_BF16 ? mto_bf16_to_f32(bits[i]) : mto_f16_to_f32(bits[i]);
}

/* ------------------------------------------------------------- epilogue -- */

/* Shaders.swift:21-27 (clamped tanh-GELU) and :29 (SiLU), in fp32. */
static inline float gelu_f(float v) {
    float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
    if (u > 15.0f) u = 15.0f;
    if (u < -15.0f) u = -15.0f;
    return 0.5f * v * (1.0f + tanhf(u));
}
static inline float silu_f(float v) { return v / (1.0f + expf(-v)); }

static inline double gelu_d(double v) {
    double u = 0.7978845608028654 * (v + 0.044715 * v * v * v);
    if (u > 15.0) u = 15.0;
    if (u < -15.0) u = -15.0;
    return 0.5 * v * (1.0 + tanh(u));
}
static inline double silu_d(double v) { return v / (1.0 + exp(-v)); }

static inline float wdec(const void *w, int wt, int64_t i) {
    uint16_t h = ((const uint16_t *)w)[i];
    return wt == MTO_BF16 ? mto_bf16_to_f32(h) : mto_f16_to_f32(h);
}

/* ---------------------------------------------------------------- linear -- */

/*
 * The reference CPU loop (KernelTests.swift:86-101) in fp32:
 *   acc = sum_k x[m,k] w[n,k] (natural k order), acc2 likewise with w2;
 *   v = acc + bias[n]; v = silu(v) * acc2 (SiLU-gate); v = gelu(v); v = silu(v);
 *   v += y0[m,n] (accumulate); y[m,n] = v.
 * x is fp32 (callers pass already-rounded fp16/bf16 values when the kernel reads
 * 16-bit activations); w, w2, bias are 16-bit storage of type wt.  y0 is read
 * only with MTO_ACCUM and may equal y.  threads <= 0 means the OpenMP default.
 */
int mto_linear_f32(const float *x, int64_t ldx, const void *w, const void *w2, int wt,
                   const void *bias, const float *y0, float *y, int64_t ldy,
                   int M, int N, int K, uint32_t flags, int threads) {
    if (M < 0 || N < 0 || K < 0) return -22;
    if ((flags & MTO_SILU_GATE) && !w2) return -22;
    if ((flags & MTO_BIAS) && !bias) return -22;
    const int gated = (flags & MTO_SILU_GATE) != 0;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nt) collapse(2)
#endif
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            const float *xr = x + (int64_t)m * ldx;
            float acc = 0.0f, acc2 = 0.0f;
            for (int k = 0; k < K; k++) {
                acc += xr[k] * wdec(w, wt, (int64_t)n * K + k);
                if (gated) acc2 += xr[k] * wdec(w2, wt, (int64_t)n * K + k);
            }
            float v = acc + ((flags & MTO_BIAS) ? wdec(bias, wt, n) : 0.0f);
            if (gated) v = silu_f(v) * acc2;
            if (flags & MTO_GELU) v = gelu_f(v);
            if (flags & MTO_SILU) v = silu_f(v);
            if (flags & MTO_ACCUM) v += y0[(int64_t)m * ldy + n];
            y[(int64_t)m * ldy + n] = v;
        }
    }
    return 0;
}

/*
 * fp64 recomputation on the same inputs: every product and sum in double, the
 * epilogue in double, y0 read as fp32.  This is the precision oracle; the
 * result is written as double.
 */
int mto_linear_f64(const float *x, int64_t ldx, const void *w, const void *w2, int wt,
                   const void *bias, const float *y0, int64_t ldy0, double *y, int64_t ldy,
                   int M, int N, int K, uint32_t flags, int threads) {
    if (M < 0 || N < 0 || K < 0) return -22;
    if ((flags & MTO_SILU_GATE) && !w2) return -22;
    if ((flags & MTO_BIAS) && !bias) return -22;
    const int gated = (flags & MTO_SILU_GATE) != 0;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
    for (int n = 0; n < N; n++) {
        for (int m = 0; m < M; m++) {
            const float *xr = x + (int64_t)m * ldx;
            double acc = 0.0, acc2 = 0.0;
            for (int k = 0; k < K; k++) {
                acc += (double)xr[k] * (double)wdec(w, wt, (int64_t)n * K + k);
                if (gated) acc2 += (double)xr[k] * (double)wdec(w2, wt, (int64_t)n * K + k);
            }
            double v = acc + ((flags & MTO_BIAS) ? (double)wdec(bias, wt, n) : 0.0);
            if (gated) v = silu_d(v) * acc2;
            if (flags & MTO_GELU) v = gelu_d(v);
            if (flags & MTO_SILU) v = silu_d(v);
            if (flags & MTO_ACCUM) v += (double)y0[(int64_t)m * ldy0 + n];
            y[(int64_t)m * ldy + n] = v;
        }
    }
    return 0;
}

/*
 * CPU baseline: the same linear with the K sum split over 16 interleaved fp32
 * partial sums (k mod 16), so the compiler can vectorise it.  Same epilogue.
 * It differs from mto_linear_f32 only by the reassociation of the K sum; the
 * CPU tests hold it to the fp32 error bound against the fp64 recomputation.
 * With F16C/AVX2/FMA the fp16 weights are widened eight at a time.
 */
__attribute__((optimize("fp-contract=fast")))
int mto_linear_fast(const float *x, int64_t ldx, const void *w, const void *w2, int wt,
                    const void *bias, const float *y0, float *y, int64_t ldy,
                    int M, int N, int K, uint32_t flags, int threads) {
    if (M < 0 || N < 0 || K < 0 || (K % 16) != 0 || M > 16) return -22;
    if ((flags & MTO_SILU_GATE) && !w2) return -22;
    if ((flags & MTO_BIAS) && !bias) return -22;
    const int gated = (flags & MTO_SILU_GATE) != 0;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nt)
#endif
    for (int n = 0; n < N; n++) {
        float acc[16][16], acc2[16][16];
        for (int m = 0; m < M; m++)
            for (int j = 0; j < 16; j++) { acc[m][j] = 0.0f; acc2[m][j] = 0.0f; }
        const uint16_t *wr = (const uint16_t *)w + (int64_t)n * K;
        const uint16_t *w2r = gated ? (const uint16_t *)w2 + (int64_t)n * K : wr;
        for (int k = 0; k < K; k += 16) {
            float wf[16], wg[16];
#ifdef MTO_HAVE_F16C
            if (wt == MTO_F16) {
                _mm256_storeu_ps(wf, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(wr + k))));
                _mm256_storeu_ps(wf + 8, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(wr + k + 8))));
                if (gated) {
                    _mm256_storeu_ps(wg, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(w2r + k))));
                    _mm256_storeu_ps(wg + 8, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(w2r + k + 8))));
                }
            } else
#endif
            {
                for (int j = 0; j < 16; j++) {
                    wf[j] = wt == MTO_BF16 ? mto_bf16_to_f32(wr[k + j]) : mto_f16_to_f32(wr[k + j]);
                    wg[j] = gated ? (wt == MTO_BF16 ? mto_bf16_to_f32(w2r[k + j]) : mto_f16_to_f32(w2r[k + j])) : 0.0f;
                }
            }
            for (int m = 0; m < M; m++) {
                const float *xr = x + (int64_t)m * ldx + k;
                for (int j = 0; j < 16; j++) acc[m][j] += xr[j] * wf[j];
                if (gated)
                    for (int j = 0; j < 16; j++) acc2[m][j] += xr[j] * wg[j];
            }
        }
        for (int m = 0; m < M; m++) {
            float a = 0.0f, a2 = 0.0f;
            for (int j = 0; j < 16; j++) { a += acc[m][j]; a2 += acc2[m][j]; }
            float v = a + ((flags & MTO_BIAS) ? wdec(bias, wt, n) : 0.0f);
            if (gated) v = silu_f(v) * a2;
            if (flags & MTO_GELU) v = gelu_f(v);
            if (flags & MTO_SILU) v = silu_f(v);
            if (flags & MTO_ACCUM) v += y0[(int64_t)m * ldy + n];
            y[(int64_t)m * ldy + n] = v;
        }
    }
    return 0;
}

int mto_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
