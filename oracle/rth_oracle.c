/*
 * CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain C restatement of the reference engine's attention and KV-quantization
 * arithmetic, used as the checker for the HIP kernels. It is loaded only by
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py. The
 * product library (runtherder_amd/lib/libruntherder_attn.so) never links it.
 *
 * Reference citations are path:line in the reference repository.
 *
 * Parity pins (what checks each function against something other than itself):
 *   rth_ref_e4m3_encode       OCP FP8 E4M3FN spec, RNE + satfinite. Pinned by an
 *                             exact-rational Python encoder (tests), by
 *                             torch.float8_e4m3fn on in-range values, and by an
 *                             exhaustive nearest-value sweep over all 2^32 fp32
 *                             bit patterns (rth_ref_e4m3_sweep_check).
 *   rth_ref_quantize_kv_fp8   closed form scale = amax/448 (bit-exact, as the
 *                             reference test requires), zero-row and NaN cases,
 *                             round-trip bounds from the reference test.
 *   rth_ref_quantize_kv_fp8_scaled  parity unpinned by the reference: the
 *                             reference has no given-scale quantize; pinned only
 *                             by the same encoder and the closed form.
 *   rth_ref_attention_f32     fp64 brute force (numpy, tests), single-key and
 *                             uniform-score invariants, chunked == tail rows.
 *   rth_ref_decode_split_f32  equal to rth_ref_attention_f32 up to
 *                             reassociation for every split count, including
 *                             empty splits.
 *   rth_ref_rope_*            closed forms (position 0 is identity, rotation
 *                             preserves pair norms, plain table is
 *                             theta^(-2i/D)); rope_apply against an
 *                             independent numpy restatement and the
 *                             reference's own bound (max-abs 5e-2 vs double).
 *   rth_ref_rmsnorm_bf16      the reference test's own CPU formula (double sum
 *                             of squares, tests/kernels/test_rmsnorm.cpp:39-60)
 *                             within one bf16 ulp, closed forms (constant rows,
 *                             scale invariance, unit gain).
 */
#include "rth_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* scalar formats                                                            */
/* ------------------------------------------------------------------------ */

static inline uint32_t f32_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, sizeof u);
    return u;
}

static inline float bits_f32(uint32_t u) {
    float x;
    memcpy(&x, &u, sizeof x);
    return x;
}

/* bf16 round-to-nearest-even, as __float2bfloat16 in the reference
 * (attention.cu:89, flash_decode.cu:246). NaN maps to a quiet NaN. */
uint16_t rth_ref_f32_to_bf16(float x) {
    uint32_t u = f32_bits(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t)((u >> 16) | 0x0040u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float rth_ref_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* OCP FP8 E4M3 ("E4M3FN": bias 7, no infinities, S.1111.111 is NaN, max
 * finite 448) with round-to-nearest-even and saturation to +-448, the
 * conversion the reference relies on at quantization.cu:248-250 ("E4M3 ctor
 * saturates out of range"). Written from the OCP 8-bit floating point
 * specification. NaN encodes as 0x7F. */
uint8_t rth_ref_e4m3_encode(float x) {
    const uint32_t u    = f32_bits(x);
    const uint8_t  sign = (uint8_t)((u >> 24) & 0x80u);
    const uint32_t a    = u & 0x7fffffffu;
    if (a > 0x7f800000u) {
        return 0x7f;                      /* NaN */
    }
    if (a >= 0x43e00000u) {               /* |x| >= 448 (incl. inf): saturate */
        return (uint8_t)(sign | 0x7e);
    }
    if (a < 0x3c800000u) {                /* |x| < 2^-6: subnormal grid 2^-9 */
        const float r = nearbyintf(bits_f32(a) * 512.0f); /* exact scale, RNE */
        return (uint8_t)(sign | (uint8_t)r); /* r == 8 is the min normal code */
    }
    const int      e    = (int)(a >> 23) - 127;   /* -6 .. 8 */
    uint32_t       keep = (a >> 20) & 0x7u;       /* 3 mantissa bits */
    const uint32_t rest = a & 0xfffffu;           /* 20 dropped bits */
    if (rest > 0x80000u || (rest == 0x80000u && (keep & 1u))) {
        ++keep;                                   /* carry may bump exponent */
    }
    return (uint8_t)(sign | (uint8_t)((((uint32_t)(e + 7)) << 3) + keep));
}

float rth_ref_e4m3_decode(uint8_t b) {
    const int e = (b >> 3) & 0xf;
    const int m = b & 0x7;
    float     v;
    if (e == 0xf && m == 0x7) {
        return NAN;
    }
    if (e == 0) {
        v = ldexpf((float)m, -9);
    } else {
        v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    }
    return (b & 0x80) ? -v : v;
}

void rth_ref_e4m3_encode_array(const float* x, uint8_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        out[i] = rth_ref_e4m3_encode(x[i]);
    }
}

void rth_ref_e4m3_encode_bits_range(uint32_t first_bits, uint64_t count,
                                    uint8_t* out) {
    for (uint64_t i = 0; i < count; ++i) {
        out[i] = rth_ref_e4m3_encode(bits_f32((uint32_t)(first_bits + i)));
    }
}

/* A second, structurally different encoder for the exhaustive sweep: nearest
 * entry of the sorted table of finite E4M3 magnitudes, computed in double,
 * ties to the even code, saturating at 448. */
static double g_e4m3_mag[127];

static void e4m3_table_init(void) {
    for (int c = 0; c < 127; ++c) {
        g_e4m3_mag[c] = (double)rth_ref_e4m3_decode((uint8_t)c);
    }
}

static uint8_t e4m3_encode_by_search(float x) {
    if (isnan(x)) {
        return 0x7f;
    }
    const uint8_t sign = signbit(x) ? 0x80 : 0x00;
    const double  a    = fabs((double)x);
    if (a >= 448.0) {
        return (uint8_t)(sign | 0x7e);
    }
    int lo = 0, hi = 126; /* g_e4m3_mag[lo] <= a < g_e4m3_mag[hi] */
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (g_e4m3_mag[mid] <= a) {
            lo = mid;
        } else {
            hi = mid;
        }
    }
    const double dlo = a - g_e4m3_mag[lo];
    const double dhi = g_e4m3_mag[hi] - a;
    int          c;
    if (dlo < dhi) {
        c = lo;
    } else if (dhi < dlo) {
        c = hi;
    } else {
        c = (lo & 1) ? hi : lo;
    }
    return (uint8_t)(sign | c);
}

typedef struct {
    uint32_t stride;
    uint64_t begin, end; /* index range over patterns 0, stride, 2*stride ... */
    int64_t  mismatches;
} sweep_job_t;

static void* sweep_worker(void* p) {
    sweep_job_t* job = (sweep_job_t*)p;
    int64_t      bad = 0;
    for (uint64_t i = job->begin; i < job->end; ++i) {
        const uint32_t bits = (uint32_t)(i * job->stride);
        const float    x    = bits_f32(bits);
        if (rth_ref_e4m3_encode(x) != e4m3_encode_by_search(x)) {
            ++bad;
        }
    }
    job->mismatches = bad;
    return NULL;
}

/* Number of fp32 bit patterns (every stride-th one) on which the bit-level
 * encoder and the nearest-value search disagree. stride 1 covers all 2^32. */
int64_t rth_ref_e4m3_sweep_check(uint32_t stride, int nthreads) {
    if (stride == 0) {
        stride = 1;
    }
    if (nthreads < 1) {
        nthreads = 1;
    }
    if (nthreads > 64) {
        nthreads = 64;
    }
    e4m3_table_init();
    const uint64_t total = ((1ull << 32) + stride - 1) / stride;
    pthread_t      th[64];
    sweep_job_t    jobs[64];
    for (int t = 0; t < nthreads; ++t) {
        jobs[t].stride     = stride;
        jobs[t].begin      = total * (uint64_t)t / (uint64_t)nthreads;
        jobs[t].end        = total * (uint64_t)(t + 1) / (uint64_t)nthreads;
        jobs[t].mismatches = 0;
        pthread_create(&th[t], NULL, sweep_worker, &jobs[t]);
    }
    int64_t bad = 0;
    for (int t = 0; t < nthreads; ++t) {
        pthread_join(th[t], NULL);
        bad += jobs[t].mismatches;
    }
    return bad;
}

/* ------------------------------------------------------------------------ */
/* seeded inputs                                                             */
/* ------------------------------------------------------------------------ */

static inline uint64_t mix64(uint64_t z) { /* splitmix64 finalizer */
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* uniform double in (0, 1], counter based so any element is reproducible */
static inline double unit_open0(uint64_t seed, uint64_t ctr) {
    const uint64_t r = mix64(seed ^ mix64(ctr));
    return ((double)(r >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

static inline float normal_at(uint64_t seed, int64_t i) {
    const uint64_t pair = (uint64_t)i >> 1;
    const double   u1   = unit_open0(seed, 2 * pair);
    const double   u2   = unit_open0(seed, 2 * pair + 1);
    const double   r    = sqrt(-2.0 * log(u1));
    const double   t    = 6.283185307179586476925 * u2;
    return (float)((i & 1) ? r * sin(t) : r * cos(t));
}

typedef struct {
    void*    out;
    int64_t  begin, end;
    uint64_t seed;
    int      kind; /* 0 = bf16 normal, 1 = f32 normal */
} fill_job_t;

static void* fill_worker(void* p) {
    fill_job_t* j = (fill_job_t*)p;
    for (int64_t i = j->begin; i < j->end; ++i) {
        const float z = normal_at(j->seed, i);
        if (j->kind == 0) {
            ((uint16_t*)j->out)[i] = rth_ref_f32_to_bf16(z);
        } else {
            ((float*)j->out)[i] = z;
        }
    }
    return NULL;
}

static void fill_parallel(void* out, int64_t n, uint64_t seed, int kind) {
    const int   nt = (n > (1 << 20)) ? 8 : 1;
    pthread_t   th[8];
    fill_job_t  jobs[8];
    for (int t = 0; t < nt; ++t) {
        jobs[t].out   = out;
        jobs[t].begin = n * t / nt;
        jobs[t].end   = n * (t + 1) / nt;
        jobs[t].seed  = seed;
        jobs[t].kind  = kind;
        if (nt == 1) {
            fill_worker(&jobs[t]);
        } else {
            pthread_create(&th[t], NULL, fill_worker, &jobs[t]);
        }
    }
    if (nt > 1) {
        for (int t = 0; t < nt; ++t) {
            pthread_join(th[t], NULL);
        }
    }
}

/* N(0,1) via Box-Muller on a counter-based splitmix64 stream, rounded to bf16
 * with RNE. Element i depends only on (seed, i). */
void rth_ref_fill_normal_bf16(uint16_t* out, int64_t n, uint64_t seed) {
    fill_parallel(out, n, seed, 0);
}

void rth_ref_fill_normal_f32(float* out, int64_t n, uint64_t seed) {
    fill_parallel(out, n, seed, 1);
}

void rth_ref_fill_uniform_f32(float* out, int64_t n, float lo, float hi,
                              uint64_t seed) {
    for (int64_t i = 0; i < n; ++i) {
        const double u = unit_open0(seed, (uint64_t)i) - 0x1p-53; /* [0, 1) */
        out[i]         = (float)(lo + (hi - lo) * u);
    }
}

/* std::mt19937 (Matsumoto & Nishimura 1998 parameters) feeding
 * std::uniform_real_distribution<float>(-scale, scale) as libstdc++ evaluates
 * it (one 32-bit draw, float(draw) / 2^32, then u * (b - a) + a without
 * contraction), then __float2bfloat16. Reproduces the inputs of the
 * reference's kernel tests (tests/kernels/test_attention.cpp:65-75,
 * tests/kernels/test_quantization.cpp:25-35) built with GCC on x86-64. */
typedef struct {
    uint32_t mt[624];
    int      idx;
} mt19937_t;

static void mt_seed(mt19937_t* g, uint32_t seed) {
    g->mt[0] = seed;
    for (int i = 1; i < 624; ++i) {
        g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
    }
    g->idx = 624;
}

static uint32_t mt_next(mt19937_t* g) {
    if (g->idx >= 624) {
        for (int i = 0; i < 624; ++i) {
            const uint32_t y = (g->mt[i] & 0x80000000u) | (g->mt[(i + 1) % 624] & 0x7fffffffu);
            g->mt[i] = g->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
        }
        g->idx = 0;
    }
    uint32_t y = g->mt[g->idx++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

/* Raw 32-bit std::mt19937 output stream (pinned by the C++ standard's
 * requirement that the 10000th draw of the default seed 5489 is 4123659995). */
void rth_ref_mt19937_raw(uint32_t seed, int64_t n, uint32_t* out) {
    mt19937_t g;
    mt_seed(&g, seed);
    for (int64_t k = 0; k < n; ++k) {
        out[k] = mt_next(&g);
    }
}

void rth_ref_fill_mt19937_uniform_bf16(uint16_t* out, int64_t n, float scale,
                                       uint32_t seed) {
    mt19937_t g;
    mt_seed(&g, seed);
    const float a = -scale;
    const float b = scale;
    for (int64_t k = 0; k < n; ++k) {
        const uint32_t y   = mt_next(&g);
        volatile float sum = (float)y;
        float          u   = sum / 4294967296.0f;
        if (u >= 1.0f) {
            u = nextafterf(1.0f, 0.0f);
        }
        volatile float prod = u * (b - a);
        const float    val  = prod + a;
        out[k]              = rth_ref_f32_to_bf16(val);
    }
}

/* ------------------------------------------------------------------------ */
/* KV quantization                                                           */
/* ------------------------------------------------------------------------ */

static const float kE4M3Max = 448.0f;

/* Follows quantize_kv_fp8_kernel (src/kernels/quantization.cu:200-254): per row
 * amax = fmaxf over |x| (NaN ignored by fmaxf, :226), scale = amax / 448
 * (:236), inv = amax > 0 ? 448 / amax : 0 (:237, a separate division, not
 * 1/scale), q = E4M3_satfinite(x * inv) (:248-250). Row r lands at
 * destination row r + at_pos * rows_per_pos (:210-211). */
void rth_ref_quantize_kv_fp8(uint8_t* q, float* scale, const uint16_t* x,
                             int at_pos, int rows_per_pos, int num_rows,
                             int head_dim) {
    for (int r = 0; r < num_rows; ++r) {
        const int64_t   dst  = (int64_t)r + (int64_t)at_pos * rows_per_pos;
        const uint16_t* xr   = x + (int64_t)r * head_dim;
        float           amax = 0.0f;
        for (int d = 0; d < head_dim; ++d) {
            amax = fmaxf(amax, fabsf(rth_ref_bf16_to_f32(xr[d])));
        }
        volatile float s   = amax / kE4M3Max;
        volatile float inv = (amax > 0.0f) ? (kE4M3Max / amax) : 0.0f;
        scale[dst]         = s;
        uint8_t* qr        = q + dst * head_dim;
        for (int d = 0; d < head_dim; ++d) {
            volatile float p = rth_ref_bf16_to_f32(xr[d]) * inv;
            qr[d]            = rth_ref_e4m3_encode(p);
        }
    }
}

/* Given-scale variant (no reference counterpart; parity unpinned by the
 * reference): the destination row's scale s is an input and
 * q = E4M3_satfinite(x * (s > 0 ? 1/s : 0)). Values beyond 448*s saturate. */
void rth_ref_quantize_kv_fp8_scaled(uint8_t* q, const float* scale,
                                    const uint16_t* x, int at_pos,
                                    int rows_per_pos, int num_rows,
                                    int head_dim) {
    for (int r = 0; r < num_rows; ++r) {
        const int64_t   dst = (int64_t)r + (int64_t)at_pos * rows_per_pos;
        const uint16_t* xr  = x + (int64_t)r * head_dim;
        const float     s   = scale[dst];
        volatile float  inv = (s > 0.0f) ? (1.0f / s) : 0.0f;
        uint8_t*        qr  = q + dst * head_dim;
        for (int d = 0; d < head_dim; ++d) {
            volatile float p = rth_ref_bf16_to_f32(xr[d]) * inv;
            qr[d]            = rth_ref_e4m3_encode(p);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* attention                                                                 */
/* ------------------------------------------------------------------------ */

static float g_e4m3_f32[256];
static int   g_e4m3_f32_ready = 0;

static void e4m3_f32_table_init(void) {
    if (!g_e4m3_f32_ready) {
        for (int c = 0; c < 256; ++c) {
            g_e4m3_f32[c] = rth_ref_e4m3_decode((uint8_t)c);
        }
        g_e4m3_f32_ready = 1;
    }
}

typedef struct {
    uint16_t*       out;
    const uint16_t* q;
    const uint8_t*  k;
    const uint8_t*  v;
    const float*    ks;
    const float*    vs;
    int             n_new, cache_len, hq, hkv, d;
    float           scale;
    int64_t         row_begin, row_end;
} attn_job_t;

/* q.k for one key with the dequantized key value float(k8) * k_scale formed
 * first and accumulated with a fused multiply-add, as qk_dot does
 * (src/kernels/attention.cu:18-28, nvcc contracts s += a * b into an fma). */
static inline float qk_dot_f32(const float* qf, const uint8_t* kr, float ks,
                               int d) {
    float s = 0.0f;
    for (int i = 0; i < d; ++i) {
        s = fmaf(qf[i], g_e4m3_f32[kr[i]] * ks, s);
    }
    return s;
}

/* One output row per (token, q head), two passes over keys 0..cache_len+qt:
 * max of scaled scores, then exp-weighted sum of dequantized values; GQA head
 * kvh = qh / (Hq / Hkv); output bf16 RNE of acc / denom. Follows
 * attention_causal_bf16_kernel, src/kernels/attention.cu:34-91. The reference
 * uses __expf; this uses expf (differences are far below the bf16 output
 * rounding). */
static void* attn_worker(void* p) {
    attn_job_t* j     = (attn_job_t*)p;
    const int   group = j->hq / j->hkv;
    float*      qf    = (float*)malloc(sizeof(float) * (size_t)j->d);
    float*      acc   = (float*)malloc(sizeof(float) * (size_t)j->d);
    for (int64_t idx = j->row_begin; idx < j->row_end; ++idx) {
        const int qt     = (int)(idx / j->hq);
        const int qh     = (int)(idx % j->hq);
        const int kvh    = qh / group;
        const int n_keys = j->cache_len + qt + 1;
        const uint16_t* qr = j->q + ((int64_t)qt * j->hq + qh) * j->d;
        for (int i = 0; i < j->d; ++i) {
            qf[i] = rth_ref_bf16_to_f32(qr[i]);
        }
        float m = -INFINITY;
        for (int t = 0; t < n_keys; ++t) {
            const int64_t row = (int64_t)t * j->hkv + kvh;
            const float   s   = qk_dot_f32(qf, j->k + row * j->d, j->ks[row], j->d);
            m                 = fmaxf(m, s * j->scale);
        }
        for (int i = 0; i < j->d; ++i) {
            acc[i] = 0.0f;
        }
        float denom = 0.0f;
        for (int t = 0; t < n_keys; ++t) {
            const int64_t  row = (int64_t)t * j->hkv + kvh;
            const uint8_t* vr  = j->v + row * j->d;
            const float    vsc = j->vs[row];
            const float    s   = qk_dot_f32(qf, j->k + row * j->d, j->ks[row], j->d);
            const float    w   = expf(fmaf(s, j->scale, -m));
            denom += w;
            for (int i = 0; i < j->d; ++i) {
                acc[i] = fmaf(w, g_e4m3_f32[vr[i]] * vsc, acc[i]);
            }
        }
        uint16_t* orow = j->out + ((int64_t)qt * j->hq + qh) * j->d;
        for (int i = 0; i < j->d; ++i) {
            orow[i] = rth_ref_f32_to_bf16(acc[i] / denom);
        }
    }
    free(qf);
    free(acc);
    return NULL;
}

void rth_ref_attention_f32(uint16_t* out, const uint16_t* q, const uint8_t* k,
                           const uint8_t* v, const float* k_scale,
                           const float* v_scale, int n_new, int cache_len,
                           int num_q_heads, int num_kv_heads, int head_dim,
                           float scale, int nthreads) {
    e4m3_f32_table_init();
    const int64_t rows = (int64_t)n_new * num_q_heads;
    if (nthreads < 1) {
        nthreads = 1;
    }
    if (nthreads > 256) {
        nthreads = 256;
    }
    if (rows < nthreads) {
        nthreads = (int)rows;
    }
    attn_job_t* jobs = (attn_job_t*)calloc((size_t)nthreads, sizeof(attn_job_t));
    pthread_t*  th   = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    for (int t = 0; t < nthreads; ++t) {
        attn_job_t* j = &jobs[t];
        j->out = out; j->q = q; j->k = k; j->v = v; j->ks = k_scale; j->vs = v_scale;
        j->n_new = n_new; j->cache_len = cache_len; j->hq = num_q_heads;
        j->hkv = num_kv_heads; j->d = head_dim; j->scale = scale;
        /* interleave rows so late (longer) tokens spread over all threads */
        j->row_begin = rows * t / nthreads;
        j->row_end   = rows * (t + 1) / nthreads;
    }
    if (nthreads == 1) {
        attn_worker(&jobs[0]);
    } else {
        for (int t = 0; t < nthreads; ++t) {
            pthread_create(&th[t], NULL, attn_worker, &jobs[t]);
        }
        for (int t = 0; t < nthreads; ++t) {
            pthread_join(th[t], NULL);
        }
    }
    free(jobs);
    free(th);
}

/* Double precision attention over the exactly dequantized cache values
 * (double(E4M3) * double(scale)), the tighter reference of
 * tests/kernels/test_attention.cpp:88-145, extended with the cache_len
 * offset of src/kernels/attention.cu:55. Output is unrounded. */
void rth_ref_attention_f64(double* out, const uint16_t* q, const uint8_t* k,
                           const uint8_t* v, const float* k_scale,
                           const float* v_scale, int n_new, int cache_len,
                           int num_q_heads, int num_kv_heads, int head_dim,
                           double scale) {
    e4m3_f32_table_init();
    const int group  = num_q_heads / num_kv_heads;
    double*   scores = (double*)malloc(sizeof(double) * (size_t)(cache_len + n_new));
    for (int qt = 0; qt < n_new; ++qt) {
        for (int qh = 0; qh < num_q_heads; ++qh) {
            const int       kvh    = qh / group;
            const int       n_keys = cache_len + qt + 1;
            const uint16_t* qr     = q + ((int64_t)qt * num_q_heads + qh) * head_dim;
            double          m      = -INFINITY;
            for (int t = 0; t < n_keys; ++t) {
                const int64_t  row = (int64_t)t * num_kv_heads + kvh;
                const uint8_t* kr  = k + row * head_dim;
                double         s   = 0.0;
                for (int i = 0; i < head_dim; ++i) {
                    s += (double)rth_ref_bf16_to_f32(qr[i]) *
                         ((double)g_e4m3_f32[kr[i]] * (double)k_scale[row]);
                }
                s *= scale;
                scores[t] = s;
                if (s > m) {
                    m = s;
                }
            }
            double denom = 0.0;
            for (int t = 0; t < n_keys; ++t) {
                scores[t] = exp(scores[t] - m);
                denom += scores[t];
            }
            double* orow = out + ((int64_t)qt * num_q_heads + qh) * head_dim;
            for (int i = 0; i < head_dim; ++i) {
                double acc = 0.0;
                for (int t = 0; t < n_keys; ++t) {
                    const int64_t row = (int64_t)t * num_kv_heads + kvh;
                    acc += scores[t] *
                           ((double)g_e4m3_f32[v[row * head_dim + i]] * (double)v_scale[row]);
                }
                orow[i] = acc / denom;
            }
        }
    }
    free(scores);
}

/* Split-K decode restated serially: key range of split si is
 * [si*chunk, min(si*chunk+chunk, n_keys)) with chunk = ceil(n_keys / S)
 * (src/kernels/flash_decode.cu:145-148); each split runs an online softmax
 * from m = -FLT_MAX/2, l = 0 (:160-161, :68-87); splits merge by
 * M = max m_i, L = sum e^(m_i-M) l_i, out = sum e^(m_i-M) acc_i / L
 * (:222-247). Decode attends cache_len + 1 keys. */
void rth_ref_decode_split_f32(uint16_t* out, const uint16_t* q,
                              const uint8_t* k, const uint8_t* v,
                              const float* k_scale, const float* v_scale,
                              int num_splits, int cache_len, int num_q_heads,
                              int num_kv_heads, int head_dim, float scale) {
    e4m3_f32_table_init();
    const int group  = num_q_heads / num_kv_heads;
    const int n_keys = cache_len + 1;
    const int chunk  = (n_keys + num_splits - 1) / num_splits;
    float*    qf     = (float*)malloc(sizeof(float) * (size_t)head_dim);
    float*    pm     = (float*)malloc(sizeof(float) * (size_t)num_splits);
    float*    pl     = (float*)malloc(sizeof(float) * (size_t)num_splits);
    float*    pacc   = (float*)malloc(sizeof(float) * (size_t)num_splits * head_dim);
    for (int qh = 0; qh < num_q_heads; ++qh) {
        const int kvh = qh / group;
        for (int i = 0; i < head_dim; ++i) {
            qf[i] = rth_ref_bf16_to_f32(q[(int64_t)qh * head_dim + i]);
        }
        for (int si = 0; si < num_splits; ++si) {
            const int start = si * chunk;
            const int end   = (start + chunk < n_keys) ? start + chunk : n_keys;
            float     m     = -FLT_MAX / 2.0f;
            float     l     = 0.0f;
            float*    acc   = pacc + (int64_t)si * head_dim;
            for (int i = 0; i < head_dim; ++i) {
                acc[i] = 0.0f;
            }
            for (int t = start; t < end; ++t) {
                const int64_t row   = (int64_t)t * num_kv_heads + kvh;
                const float   score = qk_dot_f32(qf, k + row * head_dim, k_scale[row], head_dim) * scale;
                const float   m_new = fmaxf(m, score);
                const float   corr  = expf(m - m_new);
                const float   w     = expf(score - m_new);
                for (int i = 0; i < head_dim; ++i) {
                    acc[i] = acc[i] * corr + w * (g_e4m3_f32[v[row * head_dim + i]] * v_scale[row]);
                }
                l = l * corr + w;
                m = m_new;
            }
            pm[si] = m;
            pl[si] = l;
        }
        float M = -FLT_MAX;
        for (int si = 0; si < num_splits; ++si) {
            M = fmaxf(M, pm[si]);
        }
        for (int i = 0; i < head_dim; ++i) {
            float a = 0.0f, L = 0.0f;
            for (int si = 0; si < num_splits; ++si) {
                const float e = expf(pm[si] - M);
                L += e * pl[si];
                a += e * pacc[(int64_t)si * head_dim + i];
            }
            out[(int64_t)qh * head_dim + i] = rth_ref_f32_to_bf16(a / L);
        }
    }
    free(qf);
    free(pm);
    free(pl);
    free(pacc);
}

/* ------------------------------------------------------------------------ */
/* RoPE input preparation                                                    */
/* ------------------------------------------------------------------------ */

/* inv_freq[i] = theta^(-2i/D) evaluated in double and narrowed to float
 * (src/model/supported/llama/llama.cu:128-143). */
void rth_ref_rope_inv_freq_plain(float* inv_freq, int head_dim,
                                 float theta_base) {
    const int half = head_dim / 2;
    for (int i = 0; i < half; ++i) {
        const double e = -2.0 * (double)i / (double)head_dim;
        inv_freq[i]    = (float)pow((double)theta_base, e);
    }
}

/* Llama-3 band scaling of the plain table, in double
 * (src/model/supported/llama/llama3.cu:26-60): wavelengths longer than
 * orig/low are divided by factor, shorter than orig/high kept, and the band in
 * between blended by smooth = (orig/wavelen - low) / (high - low). */
void rth_ref_rope_inv_freq_llama3(float* inv_freq, int head_dim,
                                  float theta_base, float factor,
                                  float low_freq_factor,
                                  float high_freq_factor,
                                  int original_max_position_embeddings) {
    rth_ref_rope_inv_freq_plain(inv_freq, head_dim, theta_base);
    const double fac     = (double)factor;
    const double lo      = (double)low_freq_factor;
    const double hi      = (double)high_freq_factor;
    const double old_ctx = (double)original_max_position_embeddings;
    const double lo_wl   = old_ctx / lo;
    const double hi_wl   = old_ctx / hi;
    const double two_pi  = 2.0 * 3.14159265358979323846;
    for (int i = 0; i < head_dim / 2; ++i) {
        const double f      = (double)inv_freq[i];
        const double wl     = two_pi / f;
        double       scaled = f;
        if (wl > lo_wl) {
            scaled = f / fac;
        } else if (wl >= hi_wl) {
            const double smooth = (old_ctx / wl - lo) / (hi - lo);
            scaled              = (1.0 - smooth) * (f / fac) + smooth * f;
        }
        inv_freq[i] = (float)scaled;
    }
}

/* Rotate-half RoPE in place on x[n_tokens, num_heads, head_dim] bf16:
 * theta = float(pos) * inv_freq[i], (a, b) -> (a c - b s, a s + b c) for the
 * pair (i, i + D/2), each rounded to bf16 (src/kernels/rope.cu:32-54), with
 * the products grouped as fma(a, c, -(b s)) and fma(a, s, b c). sin and cos
 * are taken in double of the fp32 angle and rounded to fp32 (the reference
 * uses the __sincosf approximation; its test bound is max-abs 5e-2 against
 * double, include/runtherder/kernels/rope.cuh:14). */
void rth_ref_rope_apply_bf16(uint16_t* x, const int* positions,
                             const float* inv_freq, int n_tokens,
                             int num_heads, int head_dim) {
    const int half = head_dim / 2;
    for (int t = 0; t < n_tokens; ++t) {
        for (int h = 0; h < num_heads; ++h) {
            uint16_t* row = x + ((int64_t)t * num_heads + h) * head_dim;
            for (int i = 0; i < half; ++i) {
                const float th = (float)positions[t] * inv_freq[i];
                const float s  = (float)sin((double)th);
                const float c  = (float)cos((double)th);
                const float a  = rth_ref_bf16_to_f32(row[i]);
                const float b  = rth_ref_bf16_to_f32(row[i + half]);
                row[i]         = rth_ref_f32_to_bf16(fmaf(a, c, -(b * s)));
                row[i + half]  = rth_ref_f32_to_bf16(fmaf(a, s, b * c));
            }
        }
    }
}

/* RMSNorm of each row of x[rows, dim] bf16 with gain g[dim] bf16
 * (src/kernels/rmsnorm.cu:45-136, rmsnorm_bf16_forward): y = bf16((x * rrms) * g)
 * with rrms = 1 / sqrt(ss / dim + eps) (the reference kernel uses rsqrtf; its
 * test oracle, tests/kernels/test_rmsnorm.cpp:39-60, 1.0f / std::sqrt). The sum
 * of squares is taken in the order of the GPU kernel: `lanes` (a power of
 * two) partial sums, lane l accumulating fmaf(x, x, s) over the 8-element
 * vectors l, l + lanes, ... (elements in order), then a butterfly over the
 * lanes (s_l + s_(l^1), then ^2, ^4, ...), which every lane ends with. */
void rth_ref_rmsnorm_bf16(uint16_t* y, const uint16_t* x, const uint16_t* g,
                          int rows, int dim, float eps, int lanes) {
    float part[64];
    for (int r = 0; r < rows; ++r) {
        const uint16_t* xr = x + (int64_t)r * dim;
        for (int l = 0; l < lanes; ++l) {
            float s = 0.0f;
            for (int v = l; v < dim / 8; v += lanes) {
                for (int j = 0; j < 8; ++j) {
                    const float h = rth_ref_bf16_to_f32(xr[8 * v + j]);
                    s             = fmaf(h, h, s);
                }
            }
            part[l] = s;
        }
        for (int m = 1; m < lanes; m <<= 1) {
            float nxt[64];
            for (int l = 0; l < lanes; ++l) {
                nxt[l] = part[l] + part[l ^ m];
            }
            memcpy(part, nxt, sizeof(float) * (size_t)lanes);
        }
        const float t    = part[0] / (float)dim + eps;
        const float rrms = 1.0f / sqrtf(t);
        uint16_t*   yr   = y + (int64_t)r * dim;
        for (int d = 0; d < dim; ++d) {
            const float h = rth_ref_bf16_to_f32(xr[d]);
            yr[d]         = rth_ref_f32_to_bf16((h * rrms) * rth_ref_bf16_to_f32(g[d]));
        }
    }
}
