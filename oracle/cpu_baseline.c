/* cpu_baseline.c - the CPU restatement of the decode attention and the RoPE
 * append written for speed, timed by bench.py as the reported CPU baseline
 * (test infrastructure: nothing on the product path links it). Built at run
 * time with -O3 -march=native for the host it runs on (bench.py), or
 * portably by oracle/Makefile for the CPU tests.
 *
 * Semantics (fp32 throughout, within the attention tolerance of the double
 * oracle, tests/test_cpu_oracle.py):
 *   decode  - native/tests/kernel_ops.cpp:434-476 attn_ref restated as a
 *             blocked online softmax: score = (q . k) * 1/sqrt(128), p =
 *             exp(score - running max), out = sum p v / sum p, bf16 RNE.
 *             Work items are (session, kv head, position segment); every K
 *             and V row is loaded once and used by the 8 query heads of its
 *             group; segment states are merged at the end.
 *   append  - native/kernels/sm120/rope_kv.cu:30-96: pos = base + t, angle
 *             (float)pos * inv_freq[d mod 64], rotate_half on q (in place,
 *             16 heads) and k (to the pool, kv = 0), v copied (kv = 1); cos
 *             and sin from libm in double precision, rounded to float.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#define HQ 16u
#define HKV 2u
#define GROUP 8u
#define D 128u
#define ROW 2560u
#define BLK 32u

static inline float bf2f(uint16_t b) {
    union { uint32_t u; float f; } c;
    c.u = (uint32_t)b << 16;
    return c.f;
}
static inline uint16_t f2bf(float f) {
    union { uint32_t u; float f; } c;
    c.f = f;
    const uint32_t u = c.u;
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u)
        return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
static inline const uint16_t* token_row(const uint16_t* pool, uint32_t P, uint32_t maxp,
                                        uint32_t layer, const uint32_t* pt, uint32_t pos) {
    return pool + ((((uint64_t)layer * maxp + pt[pos / P]) * P + pos % P) * 512u);
}

/* ---------------- decode ---------------- */

typedef struct {
    float m[GROUP], l[GROUP], acc[GROUP][D];
} seg_state_t;

typedef struct {
    const uint16_t* q;      /* [B][2560] */
    const uint32_t* limits; /* [B] */
    const uint32_t* const* pts;
    const uint16_t* pool;
    uint32_t layer, P, maxp, B, nseg;
    seg_state_t* states; /* [B][HKV][nseg] */
    uint32_t job0, job1, njobs;
} dec_ctx_t;

static void decode_segment(const dec_ctx_t* X, uint32_t b, uint32_t h, uint32_t seg,
                           seg_state_t* st) {
    const uint32_t limit = X->limits[b];
    const uint32_t n = limit + 1u;
    const uint32_t p0 = (uint32_t)((uint64_t)n * seg / X->nseg);
    const uint32_t p1 = (uint32_t)((uint64_t)n * (seg + 1u) / X->nseg);
    const float scale = 0.08838834764831845f;
    float qf[GROUP][D];
    for (uint32_t g = 0; g < GROUP; ++g)
        for (uint32_t d = 0; d < D; ++d)
            qf[g][d] = bf2f(X->q[(size_t)b * ROW + (h * GROUP + g) * D + d]);
    for (uint32_t g = 0; g < GROUP; ++g) {
        st->m[g] = -INFINITY;
        st->l[g] = 0.f;
        for (uint32_t d = 0; d < D; ++d) st->acc[g][d] = 0.f;
    }
    float kf[BLK][D], s[GROUP][BLK];
    for (uint32_t j0 = p0; j0 < p1; j0 += BLK) {
        const uint32_t nb = (p1 - j0 < BLK) ? p1 - j0 : BLK;
        const uint16_t* rows[BLK];
        for (uint32_t j = 0; j < nb; ++j) {
            rows[j] = token_row(X->pool, X->P, X->maxp, X->layer, X->pts[b], j0 + j);
            const uint16_t* k = rows[j] + h * D;
            for (uint32_t d = 0; d < D; ++d) kf[j][d] = bf2f(k[d]);
        }
        for (uint32_t g = 0; g < GROUP; ++g) {
            float mx = st->m[g];
            for (uint32_t j = 0; j < nb; ++j) {
                float dot = 0.f;
                for (uint32_t d = 0; d < D; ++d) dot += qf[g][d] * kf[j][d];
                s[g][j] = dot * scale;
                if (s[g][j] > mx) mx = s[g][j];
            }
            const float renew = (st->m[g] == -INFINITY) ? 0.f : expf(st->m[g] - mx);
            float ls = st->l[g] * renew;
            for (uint32_t j = 0; j < nb; ++j) {
                s[g][j] = expf(s[g][j] - mx);
                ls += s[g][j];
            }
            st->l[g] = ls;
            st->m[g] = mx;
            for (uint32_t d = 0; d < D; ++d) st->acc[g][d] *= renew;
        }
        for (uint32_t j = 0; j < nb; ++j) {
            const uint16_t* v = rows[j] + 256u + h * D;
            float vf[D];
            for (uint32_t d = 0; d < D; ++d) vf[d] = bf2f(v[d]);
            for (uint32_t g = 0; g < GROUP; ++g) {
                const float p = s[g][j];
                for (uint32_t d = 0; d < D; ++d) st->acc[g][d] += p * vf[d];
            }
        }
    }
}

static void* decode_worker(void* arg) {
    const dec_ctx_t* X = (const dec_ctx_t*)arg;
    for (uint32_t job = X->job0; job < X->job1; ++job) {
        const uint32_t seg = job % X->nseg, bh = job / X->nseg;
        const uint32_t b = bh / HKV, h = bh % HKV;
        decode_segment(X, b, h, seg, &X->states[((size_t)b * HKV + h) * X->nseg + seg]);
    }
    return NULL;
}

/* Decode attention of B sessions on `threads` threads; states is scratch of
 * B * 2 * nseg seg_state_t (cpb_decode_state_bytes). out [B][2048] bf16. */
size_t cpb_decode_state_bytes(uint32_t B, uint32_t nseg) {
    return (size_t)B * HKV * nseg * sizeof(seg_state_t);
}

void cpb_decode(const uint16_t* q, const uint32_t* limits, const uint32_t* const* pts,
                const uint16_t* pool, uint32_t layer, uint32_t P, uint32_t maxp, uint32_t B,
                uint32_t nseg, void* states, uint16_t* out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t th[256];
    dec_ctx_t ctx[256];
    const uint32_t njobs = B * HKV * nseg;
    for (int i = 0; i < threads; ++i) {
        dec_ctx_t c = {q, limits, pts, pool, layer, P, maxp, B, nseg, (seg_state_t*)states,
                       (uint32_t)((uint64_t)njobs * i / threads),
                       (uint32_t)((uint64_t)njobs * (i + 1) / threads), njobs};
        ctx[i] = c;
        pthread_create(&th[i], NULL, decode_worker, &ctx[i]);
    }
    for (int i = 0; i < threads; ++i) pthread_join(th[i], NULL);
    const seg_state_t* S = (const seg_state_t*)states;
    for (uint32_t b = 0; b < B; ++b)
        for (uint32_t h = 0; h < HKV; ++h)
            for (uint32_t g = 0; g < GROUP; ++g) {
                float M = -INFINITY;
                for (uint32_t k = 0; k < nseg; ++k) {
                    const seg_state_t* s = &S[((size_t)b * HKV + h) * nseg + k];
                    if (s->l[g] != 0.f && s->m[g] > M) M = s->m[g];
                }
                float L = 0.f, A[D];
                for (uint32_t d = 0; d < D; ++d) A[d] = 0.f;
                for (uint32_t k = 0; k < nseg; ++k) {
                    const seg_state_t* s = &S[((size_t)b * HKV + h) * nseg + k];
                    if (s->l[g] == 0.f) continue;
                    const float f = expf(s->m[g] - M);
                    L += s->l[g] * f;
                    for (uint32_t d = 0; d < D; ++d) A[d] += s->acc[g][d] * f;
                }
                uint16_t* o = out + (size_t)b * 2048u + (h * GROUP + g) * D;
                for (uint32_t d = 0; d < D; ++d) o[d] = f2bf(L > 0.f ? A[d] / L : 0.f);
            }
}

/* ---------------- RoPE + append ---------------- */

typedef struct {
    uint16_t* qkv;
    uint32_t base_pos, layer, P, maxp;
    const uint32_t* pt;
    const float* inv_freq; /* [64] */
    uint16_t* pool;
    uint32_t t0, t1;
} app_ctx_t;

static void rotate_row(const uint16_t* src, uint16_t* dst, const float* c, const float* s) {
    float x[D];
    for (uint32_t d = 0; d < D; ++d) x[d] = bf2f(src[d]);
    for (uint32_t d = 0; d < 64u; ++d) {
        dst[d] = f2bf(c[d] * x[d] - s[d] * x[d + 64u]);
        dst[d + 64u] = f2bf(c[d] * x[d + 64u] + s[d] * x[d]);
    }
}

static void* append_worker(void* arg) {
    const app_ctx_t* X = (const app_ctx_t*)arg;
    float c[64], s[64];
    for (uint32_t t = X->t0; t < X->t1; ++t) {
        const uint32_t pos = X->base_pos + t;
        for (uint32_t p = 0; p < 64u; ++p) {
            const double a = (double)((float)pos * X->inv_freq[p]);
            c[p] = (float)cos(a);
            s[p] = (float)sin(a);
        }
        uint16_t* row = X->qkv + (size_t)t * ROW;
        for (uint32_t h = 0; h < HQ; ++h) rotate_row(row + h * D, row + h * D, c, s);
        uint16_t* dst = X->pool + ((((uint64_t)X->layer * X->maxp + X->pt[pos / X->P]) * X->P +
                                    pos % X->P) * 512u);
        for (uint32_t h = 0; h < HKV; ++h) rotate_row(row + 2048u + h * D, dst + h * D, c, s);
        memcpy(dst + 256u, row + 2304u, 256u * sizeof(uint16_t));
    }
    return NULL;
}

void cpb_rope_append(uint16_t* qkv, uint32_t tokens, uint32_t base_pos, uint32_t layer,
                     const uint32_t* pt, uint32_t P, uint32_t maxp, const float* inv_freq,
                     uint16_t* pool, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    pthread_t th[256];
    app_ctx_t ctx[256];
    for (int i = 0; i < threads; ++i) {
        app_ctx_t c = {qkv, base_pos, layer, P, maxp, pt, inv_freq, pool,
                       (uint32_t)((uint64_t)tokens * i / threads),
                       (uint32_t)((uint64_t)tokens * (i + 1) / threads)};
        ctx[i] = c;
        pthread_create(&th[i], NULL, append_worker, &ctx[i]);
    }
    for (int i = 0; i < threads; ++i) pthread_join(th[i], NULL);
}
