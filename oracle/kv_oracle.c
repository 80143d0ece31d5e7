/* kv_oracle.c - CPU oracle of the paged KV-cache hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file restates, on the CPU, the algorithms of
 * the reference's KV path so the HIP kernels can be checked against them. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it;
 * the product library never links or calls it.
 *
 * Every function names the reference file:line it follows (paths relative to
 * the reference repository). Built with -ffp-contract=off so that each
 * floating-point operation is rounded exactly as written.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HQ 16u
#define HKV 2u
#define GROUP 8u
#define HD 128u
#define ROW 2560u
#define PSTRIDE 130u
#define SPLIT2 32u

/* ---- bf16 (native/tests/kernel_ops.cpp:180-204 f2bf RNE, bf2f) ---- */
float orc_bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
uint16_t orc_f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x7FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    uint32_t t = u >> 16;
    const uint32_t rem = u & 0xFFFFu;
    if (rem > 0x8000u) ++t;
    else if (rem == 0x8000u) t += (t & 1u);
    return (uint16_t)t;
}

/* ---- pool addressing (native/runtime/kv_cache.h:40-45 with P a parameter;
 * test twin kv_off at native/tests/kernel_ops.cpp:339-343) ---- */
uint64_t orc_kv_off(uint32_t P, uint32_t maxp, uint32_t layer, uint32_t page,
                    uint32_t slot, uint32_t kv, uint32_t head, uint32_t d) {
    return (((uint64_t)layer * maxp + page) * P + slot) * 512u + (uint64_t)kv * 256u +
           (uint64_t)head * 128u + d;
}

/* ---- RoPE cos/sin of an fp32 angle: Cody-Waite reduction by pi/2 with the
 * three-part split of fdlibm __ieee754_rem_pio2, Taylor series of sin/cos on
 * [-pi/4, pi/4] through degree 17/18 (Horner), quadrant select, rounded to
 * fp32. Stated independently of the product; tests pin it against libm. ---- */
void orc_rope_sincos(float angle, float* c_out, float* s_out) {
    const double x = (double)angle;
    const double k = rint(x * 0.6366197723675814);
    double r = fma(-k, 1.57079632673412561417e+00, x);
    r = fma(-k, 6.07710050630396597660e-11, r);
    r = fma(-k, 2.02226624879595063154e-21, r);
    const double r2 = r * r;
    static const double S[8] = {2.8114572543455206e-15, -7.647163731819816e-13,
                                1.6059043836821613e-10, -2.505210838544172e-08,
                                2.7557319223985893e-06, -0.0001984126984126984,
                                0.008333333333333333,   -0.16666666666666666};
    static const double C[9] = {-1.5619206968586225e-16, 4.779477332387385e-14,
                                -1.1470745597729725e-11, 2.08767569878681e-09,
                                -2.755731922398589e-07,  2.48015873015873e-05,
                                -0.001388888888888889,   0.041666666666666664, -0.5};
    double ps = S[0];
    for (int i = 1; i < 8; ++i) ps = fma(ps, r2, S[i]);
    const double s = fma(ps * r2, r, r);
    double pc = C[0];
    for (int i = 1; i < 9; ++i) pc = fma(pc, r2, C[i]);
    const double c = fma(pc, r2, 1.0);
    const int q = (int)((int64_t)k & 3);
    double cs, sn;
    switch (q) {
        case 0: cs = c; sn = s; break;
        case 1: cs = -s; sn = c; break;
        case 2: cs = -c; sn = -s; break;
        default: cs = s; sn = -c; break;
    }
    *c_out = (float)cs;
    *s_out = (float)sn;
}

void orc_rope_sincos_batch(const float* angles, size_t n, float* c, float* s) {
    for (size_t i = 0; i < n; ++i) orc_rope_sincos(angles[i], &c[i], &s[i]);
}

/* inv_freq table (rope_kv.cu:104-124; tools/reference_forward.py:187):
 * (float)pow((double)(float)theta, -p/64). */
void orc_inv_freq(double theta, float* out64) {
    const double th = (double)(float)theta;
    for (int p = 0; p < 64; ++p) out64[p] = (float)pow(th, -(double)p / 64.0);
}

/* ---- RoPE + K/V append ----
 * mode 0: the reference test oracle rope_ref (native/tests/kernel_ops.cpp:
 *   376-430): double angle pos*theta^(-p/64), double cos/sin and rotation,
 *   one rounding to fp32 then bf16.
 * mode 1: the kernel arithmetic of rope_kv_kernel (rope_kv.cu:30-96) with the
 *   store order of attention_decode.cu:104-113: angle = (float)pos*inv_freq[p]
 *   (fp32), cos/sin from orc_rope_sincos, t = sn*x2 rounded, fma(cs, x, -/+t),
 *   bf16 RNE. This is the bit-exact twin of the HIP kernels.
 * q is rotated in qkv (in place), k is rotated into pool kv=0, v copied to
 * kv=1. `written` (may be NULL) receives 1 at every pool element written. */
void orc_rope_append(uint16_t* qkv, uint32_t tokens, uint32_t base_pos, uint32_t layer,
                     const uint32_t* pt, uint32_t P, uint32_t maxp, double theta,
                     int mode, uint16_t* pool, uint8_t* written) {
    float invf[64];
    orc_inv_freq(theta, invf);
    for (uint32_t t = 0; t < tokens; ++t) {
        const uint32_t pos = base_pos + t;
        const uint32_t page = pt[pos / P], slot = pos % P;
        uint16_t* row = qkv + (size_t)t * ROW;
        float cf[64], sf[64];
        double cd[64], sd[64];
        for (int p = 0; p < 64; ++p) {
            if (mode == 0) {
                const double ang = (double)pos * pow(theta, -(double)p / 64.0);
                cd[p] = cos(ang);
                sd[p] = sin(ang);
            } else {
                orc_rope_sincos((float)pos * invf[p], &cf[p], &sf[p]);
            }
        }
        for (uint32_t h = 0; h < 18u; ++h) {
            uint16_t src[128];
            memcpy(src, row + h * 128u, sizeof(src));
            for (int d = 0; d < 128; ++d) {
                const int pr = d & 63;
                const int lower = d < 64;
                const float x = orc_bf2f(src[d]);
                const float x2 = orc_bf2f(src[d ^ 64]);
                float o;
                if (mode == 0) {
                    const double od = lower ? (double)x * cd[pr] - (double)x2 * sd[pr]
                                            : (double)x * cd[pr] + (double)x2 * sd[pr];
                    o = (float)od;
                } else {
                    const float tt = sf[pr] * x2;
                    o = lower ? fmaf(cf[pr], x, -tt) : fmaf(cf[pr], x, tt);
                }
                const uint16_t b = orc_f2bf(o);
                if (h < 16u) {
                    row[h * 128u + d] = b;
                } else {
                    const uint64_t off = orc_kv_off(P, maxp, layer, page, slot, 0, h - 16u, d);
                    pool[off] = b;
                    if (written) written[off] = 1;
                }
            }
        }
        for (uint32_t h = 0; h < 2u; ++h)
            for (int d = 0; d < 128; ++d) {
                const uint64_t off = orc_kv_off(P, maxp, layer, page, slot, 1, h, d);
                pool[off] = row[2304u + h * 128u + d];
                if (written) written[off] = 1;
            }
    }
}

/* ---- exact attention (native/tests/kernel_ops.cpp:434-476 attn_ref):
 * double scores q.k/sqrt(128), double softmax, out = bf16((float)(a/l)).
 * Query row t is at base_pos + t and sees keys 0..base_pos+t. ---- */
typedef struct {
    const uint16_t* q;
    uint32_t tokens, base_pos, layer, P, maxp;
    const uint16_t* pool;
    const uint32_t* pt;
    uint16_t* out;
    uint32_t job0, job1; /* (t, h) job range */
} attn_job_t;

static void attn_ref_one(const attn_job_t* J, uint32_t t, uint32_t h, double* p) {
    const double scale = 1.0 / sqrt(128.0);
    const uint32_t limit = J->base_pos + t;
    const uint32_t kvh = h / GROUP;
    double m = -1e300, l = 0.0;
    double qd[128];
    for (int d = 0; d < 128; ++d) qd[d] = orc_bf2f(J->q[(size_t)t * ROW + h * 128u + d]);
    for (uint32_t j = 0; j <= limit; ++j) {
        const uint64_t o = orc_kv_off(J->P, J->maxp, J->layer, J->pt[j / J->P], j % J->P, 0, kvh, 0);
        double dot = 0.0;
        for (int d = 0; d < 128; ++d) dot += qd[d] * (double)orc_bf2f(J->pool[o + d]);
        p[j] = dot * scale;
        if (p[j] > m) m = p[j];
    }
    for (uint32_t j = 0; j <= limit; ++j) {
        p[j] = exp(p[j] - m);
        l += p[j];
    }
    double a[128] = {0};
    for (uint32_t j = 0; j <= limit; ++j) {
        const uint64_t o = orc_kv_off(J->P, J->maxp, J->layer, J->pt[j / J->P], j % J->P, 1, kvh, 0);
        for (int d = 0; d < 128; ++d) a[d] += p[j] * (double)orc_bf2f(J->pool[o + d]);
    }
    for (int d = 0; d < 128; ++d)
        J->out[(size_t)t * 2048u + h * 128u + d] = orc_f2bf((float)(a[d] / l));
}

static void* attn_worker(void* arg) {
    const attn_job_t* J = (const attn_job_t*)arg;
    double* p = (double*)malloc(sizeof(double) * (J->base_pos + J->tokens + 1u));
    for (uint32_t job = J->job0; job < J->job1; ++job) attn_ref_one(J, job / HQ, job % HQ, p);
    free(p);
    return NULL;
}

void orc_attn_ref(const uint16_t* q_rows, uint32_t tokens, uint32_t base_pos,
                  uint32_t layer, const uint16_t* pool, const uint32_t* pt, uint32_t P,
                  uint32_t maxp, uint16_t* out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    attn_job_t jobs[64];
    const uint32_t n = tokens * HQ;
    for (int i = 0; i < threads; ++i) {
        attn_job_t J = {q_rows, tokens, base_pos, layer, P, maxp, pool, pt, out,
                        (uint32_t)((uint64_t)n * i / threads),
                        (uint32_t)((uint64_t)n * (i + 1) / threads)};
        jobs[i] = J;
        pthread_create(&th[i], NULL, attn_worker, &jobs[i]);
    }
    for (int i = 0; i < threads; ++i) pthread_join(th[i], NULL);
}

/* ---- chunked decode with bf16 P (native/tests/kernel_ops.cpp:2912-2974
 * h2_cpu_ref, the CPU statement of attn_kv_kernel_h, attention_decode.cu:
 * 966-1368): per (qh, chunk c) a single 16-position-batch online softmax in
 * fp32; l accumulates fp32 p, acc accumulates bf16-rounded p times v
 * (fp32_p != 0: acc accumulates fp32 p times v, the contract of the SIMT
 * kernel attn_kv_kernel_x, attention_decode.cu:506-878).
 * Writes partials [16][NC][130] for every chunk with start <= limit; when
 * limit < C also writes out[qh*128+d] = bf16(acc/l) (the direct path). ---- */
void orc_decode_chunks_p(const uint16_t* q, uint32_t limit, uint32_t layer,
                         const uint16_t* pool, const uint32_t* pt, uint32_t P, uint32_t maxp,
                         uint32_t C, uint32_t NC, float* partials, uint16_t* out, int fp32_p) {
    const float scale = 0.08838834764831845f;
    for (uint32_t qh = 0; qh < HQ; ++qh) {
        const uint32_t kvh = qh / GROUP;
        for (uint32_t c = 0; c < NC; ++c) {
            const uint32_t start = c * C;
            if (start > limit) break;
            const uint32_t end = (start + C - 1u < limit) ? start + C - 1u : limit;
            float m = -INFINITY, l = 0.f, acc[128] = {0};
            for (uint32_t s0 = start; s0 <= end; s0 += 16u) {
                float sc[16], qp[16];
                float mn = m;
                for (uint32_t p = 0; p < 16u; ++p) {
                    const uint32_t j = s0 + p;
                    if (j > end) { sc[p] = -INFINITY; continue; }
                    const uint64_t o = orc_kv_off(P, maxp, layer, pt[j / P], j % P, 0, kvh, 0);
                    float dot = 0.f;
                    for (int d = 0; d < 128; ++d)
                        dot += orc_bf2f(q[qh * 128u + d]) * orc_bf2f(pool[o + d]);
                    sc[p] = dot * scale;
                    mn = fmaxf(mn, sc[p]);
                }
                const float renew = (m == -INFINITY) ? 0.f : expf(m - mn);
                float ls = l * renew;
                for (uint32_t p = 0; p < 16u; ++p) {
                    const float pw = expf(sc[p] - mn);
                    ls += pw;
                    /* bf16-P (HMMA path) rounds P before P.V; fp32-P
                     * (the SIMT fallback, attention_decode.cu:506-878) uses
                     * it as is. */
                    qp[p] = fp32_p ? pw : orc_bf2f(orc_f2bf(pw));
                }
                l = ls;
                m = mn;
                for (int d = 0; d < 128; ++d) acc[d] *= renew;
                for (uint32_t p = 0; p < 16u && s0 + p <= end; ++p) {
                    const uint32_t j = s0 + p;
                    const uint64_t o = orc_kv_off(P, maxp, layer, pt[j / P], j % P, 1, kvh, 0);
                    for (int d = 0; d < 128; ++d) acc[d] += qp[p] * orc_bf2f(pool[o + d]);
                }
            }
            float* pw = partials + ((size_t)qh * NC + c) * PSTRIDE;
            pw[0] = m;
            pw[1] = l;
            for (int d = 0; d < 128; ++d) pw[2 + d] = acc[d];
            if (limit < C && out)
                for (int d = 0; d < 128; ++d)
                    out[qh * 128u + d] = orc_f2bf(l > 0.f ? acc[d] / l : 0.f);
        }
    }
}

void orc_decode_chunks(const uint16_t* q, uint32_t limit, uint32_t layer,
                       const uint16_t* pool, const uint32_t* pt, uint32_t P, uint32_t maxp,
                       uint32_t C, uint32_t NC, float* partials, uint16_t* out) {
    orc_decode_chunks_p(q, limit, layer, pool, pt, P, maxp, C, NC, partials, out, 0);
}

/* ---- two-level merge in double (native/tests/kernel_ops.cpp:2011-2059
 * merge2_cpu_ref, stating attn_merge_a/attn_merge_b of attention_decode.cu:
 * 1494-1578): split s folds chunks c = s mod 32 (ascending, l == 0 skipped),
 * then the 32 splits are folded. level2 (may be NULL) receives [16][32][130]
 * as float; out [16][128] bf16. ---- */
void orc_merge2(const float* parts, uint32_t NC, uint32_t n_valid, float* level2,
                uint16_t* out) {
    for (uint32_t qh = 0; qh < HQ; ++qh) {
        double l2m[SPLIT2], l2l[SPLIT2], l2a[SPLIT2][128];
        for (uint32_t s = 0; s < SPLIT2; ++s) {
            double mloc = -INFINITY, L = 0.0;
            double A[128] = {0};
            for (uint32_t c = s; c < n_valid; c += SPLIT2) {
                const float* p = parts + ((size_t)qh * NC + c) * PSTRIDE;
                if (p[1] != 0.f && (double)p[0] > mloc) mloc = p[0];
            }
            for (uint32_t c = s; c < n_valid; c += SPLIT2) {
                const float* p = parts + ((size_t)qh * NC + c) * PSTRIDE;
                if (p[1] == 0.f) continue;
                const double f = exp((double)p[0] - mloc);
                L += (double)p[1] * f;
                for (int d = 0; d < 128; ++d) A[d] += (double)p[2 + d] * f;
            }
            l2m[s] = mloc;
            l2l[s] = L;
            for (int d = 0; d < 128; ++d) l2a[s][d] = A[d];
            if (level2) {
                float* w = level2 + ((size_t)qh * SPLIT2 + s) * PSTRIDE;
                w[0] = (float)mloc;
                w[1] = (float)L;
                for (int d = 0; d < 128; ++d) w[2 + d] = (float)A[d];
            }
        }
        double M = -INFINITY, L = 0.0, A[128] = {0};
        for (uint32_t s = 0; s < SPLIT2; ++s)
            if (l2l[s] != 0.0 && l2m[s] > M) M = l2m[s];
        for (uint32_t s = 0; s < SPLIT2; ++s) {
            if (l2l[s] == 0.0) continue;
            const double f = exp(l2m[s] - M);
            L += l2l[s] * f;
            for (int d = 0; d < 128; ++d) A[d] += l2a[s][d] * f;
        }
        for (int d = 0; d < 128; ++d)
            out[qh * 128u + d] = orc_f2bf((float)(L > 0.0 ? A[d] / L : 0.0));
    }
}

/* ---- CPU decode baseline: full fp32 decode attention of B sessions
 * (chunk restatement above + fp32 merge), parallel over (session, q head)
 * with pthreads. Used only as bench.py's reported CPU baseline. ---- */
typedef struct {
    const uint16_t* q; /* [B][2560] */
    const uint32_t* limits;
    const uint32_t* const* pts;
    const uint16_t* pool;
    uint32_t layer, P, maxp, B;
    uint16_t* out; /* [B][2048] */
    uint32_t job0, job1;
} cpu_job_t;

static void* cpu_worker(void* arg) {
    const cpu_job_t* J = (const cpu_job_t*)arg;
    const float scale = 0.08838834764831845f;
    for (uint32_t job = J->job0; job < J->job1; ++job) {
        const uint32_t b = job / HQ, qh = job % HQ, kvh = qh / GROUP;
        const uint16_t* q = J->q + (size_t)b * ROW + qh * 128u;
        float qf[128], acc[128] = {0};
        for (int d = 0; d < 128; ++d) qf[d] = orc_bf2f(q[d]);
        float m = -INFINITY, l = 0.f;
        const uint32_t limit = J->limits[b];
        for (uint32_t j = 0; j <= limit; ++j) {
            const uint64_t o = orc_kv_off(J->P, J->maxp, J->layer, J->pts[b][j / J->P], j % J->P, 0, kvh, 0);
            const uint16_t* k = J->pool + o;
            float dot = 0.f;
            for (int d = 0; d < 128; ++d) dot += qf[d] * orc_bf2f(k[d]);
            const float s = dot * scale;
            const float mn = s > m ? s : m;
            const float renew = expf(m - mn), pw = expf(s - mn);
            l = l * renew + pw;
            m = mn;
            const uint16_t* v = k + 256;
            for (int d = 0; d < 128; ++d) acc[d] = acc[d] * renew + pw * orc_bf2f(v[d]);
        }
        for (int d = 0; d < 128; ++d) J->out[(size_t)b * 2048u + qh * 128u + d] = orc_f2bf(acc[d] / l);
    }
    return NULL;
}

void orc_decode_cpu_mt(const uint16_t* q, const uint32_t* limits, const uint32_t* const* pts,
                       const uint16_t* pool, uint32_t layer, uint32_t P, uint32_t maxp,
                       uint32_t B, uint16_t* out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    cpu_job_t jobs[64];
    const uint32_t n = B * HQ;
    for (int i = 0; i < threads; ++i) {
        cpu_job_t J = {q, limits, pts, pool, layer, P, maxp, B, out,
                       (uint32_t)((uint64_t)n * i / threads),
                       (uint32_t)((uint64_t)n * (i + 1) / threads)};
        jobs[i] = J;
        pthread_create(&th[i], NULL, cpu_worker, &jobs[i]);
    }
    for (int i = 0; i < threads; ++i) pthread_join(th[i], NULL);
}
