/* synth.c — deterministic synthetic GGUF blocks and activations.
 *
 * Every value is a pure function of (key, element index): draw i of a stream
 * is output i of a splitmix64 generator seeded at `key`, so any thread count
 * and any chunking produce the same bytes on any IEEE-754 machine.  Normal
 * deviates use Marsaglia's polar method with a logarithm built only from
 * +, -, *, / and frexp (all exact or correctly rounded), so no libm
 * transcendental whose last bit may vary between CPUs or glibc ifunc variants
 * enters the data.  Build with -ffp-contract=off.
 *
 * Distributions (the benchmark configurations):
 *   Q4_K block: d = f16(|N(0, d_sigma)|), dmin = f16(|N(0, dmin_sigma)|),
 *               16 six-bit scales/mins uniform 0..63 packed into scales[12],
 *               128 bytes of nibbles uniform 0..15.
 *   Q8_0 block: d = f16(|N(0, d_sigma)|), 32 int8 uniform in [-127, 127].
 *   activations: fp32 N(0, sigma).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#define GOLDEN 0x9E3779B97F4A7C15ull

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Output i of a splitmix64 generator whose state starts at `key`. */
static inline uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * GOLDEN); }

uint64_t bpdq_synth_key(uint64_t seed, uint64_t stream) {
    return mix64(seed * GOLDEN ^ mix64(stream + 0x5851F42D4C957F2Dull));
}

/* ln(s) for s in (0, 1]: s = m 2^e, ln m = 2 atanh((m-1)/(m+1)) by its odd series. */
static double det_log(double s) {
    int e;
    double m = frexp(s, &e);
    if (m < 0.70710678118654752440) { m = m * 2.0; e -= 1; }
    double f = (m - 1.0) / (m + 1.0);
    double f2 = f * f;
    double p = 1.0 / 25.0;
    for (int k = 23; k >= 1; k -= 2) p = p * f2 + 1.0 / (double)k;
    return (double)e * 0.69314718055994530941723212145818 + 2.0 * f * p;
}

/* Standard normal deviate for `slot`; slot s owns draws [32 s, 32 s + 32). */
static double normal_at(uint64_t key, uint64_t slot) {
    for (uint64_t a = 0; a < 16; a++) {
        uint64_t r1 = draw(key, slot * 32 + 2 * a);
        uint64_t r2 = draw(key, slot * 32 + 2 * a + 1);
        double u = (double)(r1 >> 11) * 0x1p-52 - 1.0;
        double v = (double)(r2 >> 11) * 0x1p-52 - 1.0;
        double s = u * u + v * v;
        if (s > 0.0 && s < 1.0) return u * sqrt(-2.0 * det_log(s) / s);
    }
    return 0.0;
}

/* IEEE binary32 -> binary16, round to nearest even, overflow to Inf. */
static uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return sign | 0x7E00u;
    if (ax >= 0x477FF000u) return sign | 0x7C00u;
    if (ax >= 0x38800000u) {
        uint32_t r = ax - 0x38000000u;
        uint32_t h = r >> 13, rem = r & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return sign | (uint16_t)h;
    }
    if (ax < 0x33000000u) return sign;
    uint32_t E = ax >> 23, m = (ax & 0x7FFFFFu) | 0x800000u;
    uint32_t shift = 126u - E;
    uint32_t h = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return sign | (uint16_t)h;
}

static uint16_t abs_normal_f16(uint64_t key, uint64_t slot, double sigma) {
    double z = normal_at(key, slot);
    return f32_to_f16_rne((float)(fabs(z) * sigma));
}

/* ---- per-range workers ------------------------------------------------- */

typedef struct {
    int kind;
    void* out;
    int64_t begin, end;
    uint64_t key;
    double s0, s1;
} job_t;

enum { JOB_Q4K, JOB_Q80, JOB_NORMAL, JOB_BYTES };

static void q4k_range(uint8_t* out, int64_t b0, int64_t b1, uint64_t key, double ds, double ms) {
    const uint64_t kn = key ^ 0x1ull, ki = key ^ 0x2ull;
    for (int64_t b = b0; b < b1; b++) {
        uint8_t* blk = out + b * 144;
        uint16_t d = abs_normal_f16(kn, (uint64_t)b * 2, ds);
        uint16_t dm = abs_normal_f16(kn, (uint64_t)b * 2 + 1, ms);
        blk[0] = (uint8_t)(d & 0xFF); blk[1] = (uint8_t)(d >> 8);
        blk[2] = (uint8_t)(dm & 0xFF); blk[3] = (uint8_t)(dm >> 8);
        uint64_t r0 = draw(ki, (uint64_t)b * 18), r1 = draw(ki, (uint64_t)b * 18 + 1);
        uint8_t six[16];
        for (int k = 0; k < 10; k++) six[k] = (uint8_t)((r0 >> (6 * k)) & 63u);
        for (int k = 0; k < 6; k++) six[10 + k] = (uint8_t)((r1 >> (6 * k)) & 63u);
        const uint8_t* sc = six;      /* sub-block scales 0..7 */
        const uint8_t* mn = six + 8;  /* sub-block mins   0..7 */
        uint8_t* s = blk + 4;
        for (int j = 0; j < 4; j++) {
            s[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
        }
        for (int k = 0; k < 16; k++) {
            uint64_t r = draw(ki, (uint64_t)b * 18 + 2 + (uint64_t)k);
            for (int t = 0; t < 8; t++) blk[16 + 8 * k + t] = (uint8_t)(r >> (8 * t));
        }
    }
}

static void q80_range(uint8_t* out, int64_t b0, int64_t b1, uint64_t key, double ds) {
    const uint64_t kn = key ^ 0x1ull, ki = key ^ 0x2ull;
    for (int64_t b = b0; b < b1; b++) {
        uint8_t* blk = out + b * 34;
        uint16_t d = abs_normal_f16(kn, (uint64_t)b, ds);
        blk[0] = (uint8_t)(d & 0xFF); blk[1] = (uint8_t)(d >> 8);
        for (int k = 0; k < 16; k++) {
            uint64_t r = draw(ki, (uint64_t)b * 16 + (uint64_t)k);
            for (int h = 0; h < 2; h++) {
                uint64_t half = (r >> (32 * h)) & 0xFFFFFFFFull;
                int v = (int)((half * 255u) >> 32) - 127;
                blk[2 + 2 * k + h] = (uint8_t)(int8_t)v;
            }
        }
    }
}

static void normal_range(float* out, int64_t i0, int64_t i1, uint64_t key, double sigma) {
    for (int64_t i = i0; i < i1; i++) out[i] = (float)(normal_at(key, (uint64_t)i) * sigma);
}

static void bytes_range(uint8_t* out, int64_t i0, int64_t i1, uint64_t key) {
    for (int64_t i = i0; i < i1; i++) out[i] = (uint8_t)(draw(key, (uint64_t)i >> 3) >> (8 * (i & 7)));
}

static void* run_job(void* p) {
    job_t* j = (job_t*)p;
    switch (j->kind) {
    case JOB_Q4K: q4k_range((uint8_t*)j->out, j->begin, j->end, j->key, j->s0, j->s1); break;
    case JOB_Q80: q80_range((uint8_t*)j->out, j->begin, j->end, j->key, j->s0); break;
    case JOB_NORMAL: normal_range((float*)j->out, j->begin, j->end, j->key, j->s0); break;
    default: bytes_range((uint8_t*)j->out, j->begin, j->end, j->key); break;
    }
    return NULL;
}

static void run_parallel(int kind, void* out, int64_t n, uint64_t key, double s0, double s1, int nthreads) {
    enum { MAXT = 64 };
    if (n <= 0) return;
    if (nthreads < 1) nthreads = 1;
    if (nthreads > MAXT) nthreads = MAXT;
    if ((int64_t)nthreads > n) nthreads = (int)n;
    job_t jobs[MAXT];
    pthread_t th[MAXT];
    int started[MAXT];
    for (int t = 0; t < nthreads; t++) {
        jobs[t].kind = kind; jobs[t].out = out; jobs[t].key = key; jobs[t].s0 = s0; jobs[t].s1 = s1;
        jobs[t].begin = n * t / nthreads;
        jobs[t].end = n * (t + 1) / nthreads;
        started[t] = (t > 0) && pthread_create(&th[t], NULL, run_job, &jobs[t]) == 0;
        if (t > 0 && !started[t]) run_job(&jobs[t]);
    }
    run_job(&jobs[0]);
    for (int t = 1; t < nthreads; t++)
        if (started[t]) pthread_join(th[t], NULL);
}

void bpdq_synth_q4k(uint8_t* out, int64_t n_blocks, uint64_t key, double d_sigma, double dmin_sigma, int nthreads) {
    run_parallel(JOB_Q4K, out, n_blocks, key, d_sigma, dmin_sigma, nthreads);
}

void bpdq_synth_q8_0(uint8_t* out, int64_t n_blocks, uint64_t key, double d_sigma, int nthreads) {
    run_parallel(JOB_Q80, out, n_blocks, key, d_sigma, 0.0, nthreads);
}

void bpdq_synth_normal_f32(float* out, int64_t n, uint64_t key, double sigma, int nthreads) {
    run_parallel(JOB_NORMAL, out, n, key, sigma, 0.0, nthreads);
}

void bpdq_synth_bytes(uint8_t* out, int64_t n, uint64_t key, int nthreads) {
    run_parallel(JOB_BYTES, out, n, key, 0.0, 0.0, nthreads);
}
