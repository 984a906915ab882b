/* CPU restatement of the W4A8 MLP chain, the same arithmetic as oracle/ref.py's rmsnorm + mono_mlp
 * (rotation "none"), in C with a thread per share of output channels. Test infrastructure and the CPU
 * baseline of the MLP bench line only: nothing in the library calls it.
 *
 * Reference semantics restated (comfy-mono-decode-xpu):
 *   decode       csrc/w4a8_decode.sycl:35-45   w8 = clamp(rint(cb[code] * s_rel), -127, 127), NaN -> 0
 *   dot          csrc/w4a8_decode.sycl:8-9     int32 sum of int8 x * int8 w8 (wrapping)
 *   scaleback    csrc/w4a8_decode.sycl:155-157 f = (float(acc) * xs) * sch
 *   quantisation csrc/act_prep.sycl:70-91      s = max(amax / 127, 1e-30), codes rint(bf16(x / bf16(s)))
 *   SiLU * up    csrc/mono_mlp.sycl:130-138    h = bf16(lut[bf16(g)] * bf16(u))
 *   RMSNorm      the library's canonical order (ref.rmsnorm_factor): per 256-group, 64 runs of four
 *                ((sq0 + sq1) + sq2) + sq3, a halving tree over the runs, the groups added in order
 * Weights: packed int4 codes row-major [N, K / 2] (low nibble: even k), float32 relative group scales
 * [N, K / G] (G a multiple of 64), float32 channel scales [N]; the default codebook (code - 8). AVX2:
 * the decode by byte shuffles through each group's 16-entry table, the dots by int16 pair sums.
 * Build: oracle/Makefile (gcc -O3 -mavx2 -mfma -ffp-contract=off -fPIC -shared -pthread). */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint16_t f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

static float bfround(float f) { return bf2f(f2bf(f)); }

/* r = 1 / sqrt(ss / K + eps) in the canonical order (K a multiple of 256) */
static float rms_factor(const float* x, int K, float eps) {
    float ss = 0.f;
    for (int g = 0; g < K / 256; ++g) {
        float p[64];
        for (int l = 0; l < 64; ++l) {
            const float* v = x + 256 * g + 4 * l;
            float q = v[0] * v[0];
            q = q + v[1] * v[1];
            q = q + v[2] * v[2];
            q = q + v[3] * v[3];
            p[l] = q;
        }
        for (int n = 32; n >= 1; n /= 2)
            for (int l = 0; l < n; ++l) p[l] = p[l] + p[l + n];
        ss = g == 0 ? p[0] : ss + p[0];
    }
    const float mean = ss / (float)K;
    return 1.f / sqrtf(mean + eps);
}

/* quantise one row of float values: codes and the f32 scale */
static float quant_row(const float* v, int K, int8_t* q) {
    float amax = 0.f;
    for (int k = 0; k < K; ++k) {
        const float a = fabsf(v[k]);
        if (a > amax) amax = a; /* (NaN never wins) */
    }
    float s = amax / 127.0f;
    if (!(s >= 1e-30f)) s = 1e-30f;
    uint16_t sb = f2bf(s);
    if ((sb & 0x7FFFu) == 0) sb = 0x0080u;
    const float sbf = bf2f(sb);
    for (int k = 0; k < K; ++k) {
        const float d = bfround(v[k] / sbf);
        float r = nearbyintf(d);
        if (r != r) r = 0.f;
        r = r < -128.f ? -128.f : (r > 127.f ? 127.f : r);
        q[k] = (int8_t)r;
    }
    return s;
}

/* a group's 16 decoded values clamp(rint((c - 8) * s), -127, 127), NaN -> 0: the fp32 products, rounding
 * to nearest even, the NaN lanes zeroed, the clamp, then exact conversions */
static void group_table(float s, int8_t tab[16]) {
    const __m256 sv = _mm256_set1_ps(s);
    const __m256 c0 = _mm256_setr_ps(-8.f, -7.f, -6.f, -5.f, -4.f, -3.f, -2.f, -1.f);
    const __m256 c1 = _mm256_setr_ps(0.f, 1.f, 2.f, 3.f, 4.f, 5.f, 6.f, 7.f);
    __m256 r0 = _mm256_round_ps(_mm256_mul_ps(c0, sv), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 r1 = _mm256_round_ps(_mm256_mul_ps(c1, sv), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    r0 = _mm256_and_ps(r0, _mm256_cmp_ps(r0, r0, _CMP_ORD_Q));
    r1 = _mm256_and_ps(r1, _mm256_cmp_ps(r1, r1, _CMP_ORD_Q));
    const __m256 lo = _mm256_set1_ps(-127.f), hi = _mm256_set1_ps(127.f);
    r0 = _mm256_min_ps(_mm256_max_ps(r0, lo), hi);
    r1 = _mm256_min_ps(_mm256_max_ps(r1, lo), hi);
    int32_t v[16];
    _mm256_storeu_si256((__m256i*)v, _mm256_cvttps_epi32(r0));
    _mm256_storeu_si256((__m256i*)(v + 8), _mm256_cvttps_epi32(r1));
    for (int c = 0; c < 16; ++c) tab[c] = (int8_t)v[c];
}

/* codes of G weights (G / 2 bytes, G a multiple of 64) -> int8 through the group's 16-entry table: one
 * byte shuffle per 32 codes of a nibble position, the two positions interleaved back into k order */
static void decode_group(const uint8_t* qb, int G, const int8_t tab[16], int8_t* w8) {
    const __m256i t = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i*)tab));
    const __m256i m = _mm256_set1_epi8(0x0F);
    for (int i = 0; i < G / 2; i += 32) {
        const __m256i b = _mm256_loadu_si256((const __m256i*)(qb + i));
        const __m256i lo = _mm256_shuffle_epi8(t, _mm256_and_si256(b, m));                      /* k = 2 j */
        const __m256i hi = _mm256_shuffle_epi8(t, _mm256_and_si256(_mm256_srli_epi16(b, 4), m)); /* k = 2 j + 1 */
        const __m256i a0 = _mm256_unpacklo_epi8(lo, hi); /* bytes 0-7 | 16-23 of each half, interleaved */
        const __m256i a1 = _mm256_unpackhi_epi8(lo, hi); /* bytes 8-15 | 24-31 */
        _mm256_storeu_si256((__m256i*)(w8 + 2 * i), _mm256_permute2x128_si256(a0, a1, 0x20));
        _mm256_storeu_si256((__m256i*)(w8 + 2 * i + 32), _mm256_permute2x128_si256(a0, a1, 0x31));
    }
}

/* sum of a[k] * b[k] over K int8 (K a multiple of 32): int16 products added in pairs into int32 lanes
 * (exact: |a b| <= 16384), then the lanes */
static int32_t dot_i8(const int8_t* a, const int8_t* b, int K) {
    __m256i acc = _mm256_setzero_si256();
    for (int k = 0; k < K; k += 32) {
        const __m256i va = _mm256_loadu_si256((const __m256i*)(a + k));
        const __m256i vb = _mm256_loadu_si256((const __m256i*)(b + k));
        const __m256i a0 = _mm256_cvtepi8_epi16(_mm256_castsi256_si128(va));
        const __m256i a1 = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(va, 1));
        const __m256i b0 = _mm256_cvtepi8_epi16(_mm256_castsi256_si128(vb));
        const __m256i b1 = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(vb, 1));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(a0, b0));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(a1, b1));
    }
    int32_t l[8];
    _mm256_storeu_si256((__m256i*)l, acc);
    return ((l[0] + l[1]) + (l[2] + l[3])) + ((l[4] + l[5]) + (l[6] + l[7]));
}

typedef struct {
    const int8_t* x;  /* [rows, K] */
    const float* xs;  /* [rows] */
    int rows, K, N, G;
    const uint8_t* wq;
    const float* ws;
    const float* wsch;
    float* out;       /* [rows, N] */
    int n0, n1;
} GemvJob;

/* output channels [n0, n1): each row of weights decoded through its groups' 16-entry tables into an
 * int8 row, then its dot with every activation row */
static void* gemv_worker(void* arg) {
    GemvJob* j = (GemvJob*)arg;
    const int K = j->K, G = j->G, ng = K / G;
    int8_t* w8 = (int8_t*)malloc((size_t)K);
    for (int n = j->n0; n < j->n1; ++n) {
        const uint8_t* qb = j->wq + (size_t)n * (K / 2);
        for (int g = 0; g < ng; ++g) {
            int8_t tab[16];
            group_table(j->ws[(size_t)n * ng + g], tab);
            decode_group(qb + g * (G / 2), G, tab, w8 + g * G);
        }
        for (int r = 0; r < j->rows; ++r) {
            const int32_t acc = dot_i8(j->x + (size_t)r * K, w8, K);
            const float f = ((float)acc * j->xs[r]) * j->wsch[n];
            j->out[(size_t)r * j->N + n] = f;
        }
    }
    free(w8);
    return NULL;
}

static void gemv(const int8_t* x, const float* xs, int rows, int K, int N, int G, const uint8_t* wq, const float* ws,
                 const float* wsch, float* out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t tid[256];
    GemvJob job[256];
    for (int t = 0; t < threads; ++t) {
        job[t] = (GemvJob){x, xs, rows, K, N, G, wq, ws, wsch, out, (int)((int64_t)N * t / threads),
                           (int)((int64_t)N * (t + 1) / threads)};
        if (t > 0) pthread_create(&tid[t], NULL, gemv_worker, &job[t]);
    }
    gemv_worker(&job[0]);
    for (int t = 1; t < threads; ++t) pthread_join(tid[t], NULL);
}

/* out (bf16 [rows, H]) = mono_mlp(rmsnorm(x, nw, eps)) with gate/up [I, H] and down [H, I]; returns 0 */
int cpu_mlp(const uint16_t* x, const uint16_t* nw, float eps, int rows, int H, int I, int G, const uint8_t* gq,
            const float* gs, const float* gsch, const uint8_t* uq, const float* us, const float* usch,
            const uint8_t* dq, const float* ds, const float* dsch, const uint16_t* lut, uint16_t* out, int threads) {
    if (rows < 1 || H % 256 || I % 256 || G < 64 || G % 64 || H % G || I % G) return 1;
    float* v = (float*)malloc(sizeof(float) * (size_t)rows * (H > I ? H : I));
    int8_t* q = (int8_t*)malloc((size_t)rows * (H > I ? H : I));
    float* xs = (float*)malloc(sizeof(float) * rows);
    float* g = (float*)malloc(sizeof(float) * (size_t)rows * I);
    float* u = (float*)malloc(sizeof(float) * (size_t)rows * I);
    float* d = (float*)malloc(sizeof(float) * (size_t)rows * H);
    /* RMSNorm (bf16 out) and the activation quantisation */
    for (int r = 0; r < rows; ++r) {
        float* vr = v + (size_t)r * H;
        for (int k = 0; k < H; ++k) vr[k] = bf2f(x[(size_t)r * H + k]);
        const float rf = rms_factor(vr, H, eps);
        for (int k = 0; k < H; ++k) vr[k] = bfround((vr[k] * rf) * bf2f(nw[k]));
        xs[r] = quant_row(vr, H, q + (size_t)r * H);
    }
    gemv(q, xs, rows, H, I, G, gq, gs, gsch, g, threads);
    gemv(q, xs, rows, H, I, G, uq, us, usch, u, threads);
    /* h = bf16(lut[bf16(g)] * bf16(u)), quantised */
    for (int r = 0; r < rows; ++r) {
        float* vr = v + (size_t)r * I;
        for (int i = 0; i < I; ++i) {
            const size_t o = (size_t)r * I + i;
            vr[i] = bfround(bf2f(lut[f2bf(g[o])]) * bfround(u[o]));
        }
        xs[r] = quant_row(vr, I, q + (size_t)r * I);
    }
    gemv(q, xs, rows, I, H, G, dq, ds, dsch, d, threads);
    for (size_t o = 0; o < (size_t)rows * H; ++o) out[o] = f2bf(d[o]);
    free(v);
    free(q);
    free(xs);
    free(g);
    free(u);
    free(d);
    return 0;
}
