/*
 * oracle.c -- CPU restatement of NNop's fused-kernel algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  The HIP library's results are checked against this file,
 * which is never part of the library: only tests, the smoke check and bench.py's
 * CPU-baseline leg load it.
 *
 * Every array is column-major exactly like the reference's Julia arrays (first index
 * contiguous) and is passed as double.  Two arithmetic modes:
 *   mode 0 (EXACT):    float64 mathematics of the operation (closed form: full row
 *                      softmax, analytic gradients).  Fully masked attention rows give
 *                      p = 0, o = 0.
 *   mode 1 (FAITHFUL): the reference's own algorithm in float32: the same gsz tiling,
 *                      online-softmax update order, per-thread strided partial sums
 *                      with a @groupreduce tree, and the float16 rounding of Q and K in
 *                      the attention backward.  Fully masked tiles produce NaN exactly
 *                      as the reference does.
 * Each function cites the reference lines it follows.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

typedef int64_t i64;

/* ------------------------------------------------------------------ rounding */

/* Round a float to the nearest IEEE binary16 value (ties to even), returned as float. */
float orc_round_f16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    uint32_t sign = u & 0x80000000u, au = u & 0x7fffffffu;
    float ax;
    memcpy(&ax, &au, 4);
    if (au >= 0x7f800000u) return x;                       /* inf / nan */
    if (ax >= 65520.0f) return sign ? -INFINITY : INFINITY; /* rounds past max half */
    if (ax < 6.103515625e-05f) {                            /* half subnormal: quantum 2^-24 */
        const float qnt = 5.9604644775390625e-08f;
        float r = nearbyintf(ax / qnt) * qnt;
        return sign ? -r : r;
    }
    uint32_t lsb = (au >> 13) & 1u;
    au += 0x0fffu + lsb;
    au &= ~0x1fffu;
    memcpy(&ax, &au, 4);
    return sign ? -ax : ax;
}

/* Round a float to the nearest bfloat16 value (ties to even), returned as float. */
float orc_round_bf16(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return x; /* nan */
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    u &= 0xffff0000u;
    float r;
    memcpy(&r, &u, 4);
    return r;
}

void orc_round_array(int kind, i64 n, const double* in, double* out) {
    for (i64 i = 0; i < n; ++i) {
        float f = (float)in[i];
        out[i] = kind == 1 ? orc_round_f16(f) : kind == 2 ? orc_round_bf16(f) : f;
    }
}

/* @groupreduce(+) over `gsz` per-thread partials: LDS tree, pairs (i, i+s) for
 * s = gsz/2 .. 1 (src/groupreduce.jl:20-43).  Result is thread 1's value. */
static float tree_sum_f(float* part, int gsz) {
    for (int s = gsz / 2; s > 0; s >>= 1)
        for (int i = 0; i < s; ++i) part[i] = part[i] + part[i + s];
    return part[0];
}

/* ------------------------------------------------------------------ softmax */

/* md_reduce (src/softmax.jl:6-16). */
static void md_reduce(float am, float ad, float bm, float bd, float* om, float* od) {
    int a_bigger = am > bm;
    float big_m = a_bigger ? am : bm, big_d = a_bigger ? ad : bd;
    float sml_m = a_bigger ? bm : am, sml_d = a_bigger ? bd : ad;
    float diff = sml_m - big_m;
    if (isnan(diff)) diff = -INFINITY;
    *om = big_m;
    *od = big_d + sml_d * expf(diff);
}

/* Softmax over dim 1 of x (N, M).  FAITHFUL follows online_softmax! with gsz = 256
 * (src/softmax.jl:19-68); EXACT is max-shifted exp over sum in float64. */
void orc_softmax_fwd(int mode, i64 N, i64 M, const double* x, double* y) {
#pragma omp parallel for schedule(static)
    for (i64 j = 0; j < M; ++j) {
        const double* xc = x + j * N;
        double* yc = y + j * N;
        if (mode == 0) {
            double m = -INFINITY, d = 0.0;
            for (i64 i = 0; i < N; ++i) m = fmax(m, xc[i]);
            for (i64 i = 0; i < N; ++i) d += exp(xc[i] - m);
            for (i64 i = 0; i < N; ++i) yc[i] = exp(xc[i] - m) / d;
        } else {
            const int gsz = 256;
            float pm[256], pd[256];
            for (int t = 0; t < gsz; ++t) {
                float m = -INFINITY, d = 0.0f;
                for (i64 i = t; i < N; i += gsz) md_reduce(m, d, (float)xc[i], 1.0f, &m, &d);
                pm[t] = m;
                pd[t] = d;
            }
            for (int s = gsz / 2; s > 0; s >>= 1)
                for (int t = 0; t < s; ++t) md_reduce(pm[t], pd[t], pm[t + s], pd[t + s], &pm[t], &pd[t]);
            float tmax = pm[0], inv = 1.0f / pd[0];
            for (i64 i = 0; i < N; ++i) yc[i] = expf((float)xc[i] - tmax) * inv;
        }
    }
}

/* Pullback of dx = dy .* y - y .* s, s = sum(dy .* y; dims=1) (src/softmax.jl:70-80; the
 * within_gradient branch at :71-74 keeps this second derivative available): for
 * G = dL/d(dx), with u = sum(G .* y; dims=1),
 *   dL/d(dy) = y .* (G - u),   dL/d(y) = G .* (dy - s) - dy .* u.     Float64. */
void orc_softmax_bwd_bwd(i64 N, i64 M, const double* G, const double* dy, const double* y, double* d_dy,
                         double* d_y) {
#pragma omp parallel for schedule(static)
    for (i64 j = 0; j < M; ++j) {
        const double* gc = G + j * N;
        const double* dc = dy + j * N;
        const double* yc = y + j * N;
        double s = 0.0, u = 0.0;
        for (i64 i = 0; i < N; ++i) {
            s += dc[i] * yc[i];
            u += gc[i] * yc[i];
        }
        for (i64 i = 0; i < N; ++i) {
            d_dy[j * N + i] = yc[i] * (gc[i] - u);
            d_y[j * N + i] = gc[i] * (dc[i] - s) - dc[i] * u;
        }
    }
}

/* dx = dy .* y - y .* sum(dy .* y; dims=1)  (src/softmax.jl:70-80). */
void orc_softmax_bwd(int mode, i64 N, i64 M, const double* dy, const double* y, double* dx) {
#pragma omp parallel for schedule(static)
    for (i64 j = 0; j < M; ++j) {
        const double* g = dy + j * N;
        const double* yc = y + j * N;
        double* o = dx + j * N;
        if (mode == 0) {
            double s = 0.0;
            for (i64 i = 0; i < N; ++i) s += g[i] * yc[i];
            for (i64 i = 0; i < N; ++i) o[i] = yc[i] * (g[i] - s);
        } else {
            float s = 0.0f;
            for (i64 i = 0; i < N; ++i) {
                float t = (float)g[i] * (float)yc[i];
                s += t;
            }
            for (i64 i = 0; i < N; ++i) {
                float t = (float)g[i] * (float)yc[i];
                o[i] = t - (float)yc[i] * s;
            }
        }
    }
}

/* ------------------------------------------------------------------ RMS norm */

/* y = (offset + w) x rstd, rstd = 1/sqrt(mean(x^2) + eps).  FAITHFUL follows
 * _rms_norm! (src/rms_norm.jl:3-38): per-thread partial of x^2 scaled by 1/emb, tree. */
void orc_rms_fwd(int mode, i64 emb, i64 n, const double* x, const double* w,
                 double eps, double offset, double* y, double* rstd) {
#pragma omp parallel for schedule(static)
    for (i64 j = 0; j < n; ++j) {
        const double* xc = x + j * emb;
        double* yc = y + j * emb;
        if (mode == 0) {
            double ss = 0.0;
            for (i64 i = 0; i < emb; ++i) ss += xc[i] * xc[i];
            double r = 1.0 / sqrt(ss / (double)emb + eps);
            rstd[j] = r;
            for (i64 i = 0; i < emb; ++i) yc[i] = (offset + w[i]) * xc[i] * r;
        } else {
            const int gsz = 256;
            float part[256];
            float inv_emb = 1.0f / (float)emb;
            for (int t = 0; t < gsz; ++t) {
                float p = 0.0f;
                for (i64 i = t; i < emb; i += gsz) { float xv = (float)xc[i]; p += xv * xv; }
                part[t] = p * inv_emb;
            }
            float avg = tree_sum_f(part, gsz);
            float r = 1.0f / sqrtf(avg + (float)eps);
            rstd[j] = r;
            for (i64 i = 0; i < emb; ++i)
                yc[i] = ((float)offset + (float)w[i]) * (float)xc[i] * r;
        }
    }
}

/* RMS norm backward.  dd = sum(dy (w+off) x); dx = rstd dy (w+off) - rstd^3 dd x / emb;
 * dw = sum_cols dy x rstd.  FAITHFUL follows _∇rms_norm! (src/rms_norm.jl:43-115): dw in
 * float32 partials over groups of 4 columns, then summed (src/rms_norm.jl:162-167). */
void orc_rms_bwd(int mode, i64 emb, i64 n, const double* dy, const double* rstd,
                 const double* x, const double* w, double offset, double* dx, double* dw) {
    if (mode == 0) {
        for (i64 i = 0; i < emb; ++i) dw[i] = 0.0;
        for (i64 j = 0; j < n; ++j) {
            const double *g = dy + j * emb, *xc = x + j * emb;
            double r = rstd[j], dd = 0.0;
            for (i64 i = 0; i < emb; ++i) dd += g[i] * (w[i] + offset) * xc[i];
            for (i64 i = 0; i < emb; ++i) {
                dx[i + j * emb] = r * g[i] * (w[i] + offset) - r * r * r * dd * xc[i] / (double)emb;
                dw[i] += g[i] * xc[i] * r;
            }
        }
        return;
    }
    const int gsz = 256, bpg = 4;
    float inv_emb = 1.0f / (float)emb;
    i64 nblk = (n + bpg - 1) / bpg;
    float* part = (float*)calloc((size_t)(nblk * emb), sizeof(float));
#pragma omp parallel for schedule(static)
    for (i64 blk = 0; blk < nblk; ++blk) {
        float red[256];
        float* dwp = part + blk * emb;
        i64 je = (blk + 1) * bpg < n ? (blk + 1) * bpg : n;
        for (i64 j = blk * bpg; j < je; ++j) {
            const double *g = dy + j * emb, *xc = x + j * emb;
            for (int t = 0; t < gsz; ++t) {
                float dd = 0.0f;
                for (i64 i = t; i < emb; i += gsz)
                    dd += (float)g[i] * ((float)w[i] + (float)offset) * (float)xc[i];
                red[t] = dd;
            }
            float dd = tree_sum_f(red, gsz);
            float r = (float)rstd[j];
            for (i64 i = 0; i < emb; ++i) {
                float d = (float)g[i], wi = (float)w[i], xi = (float)xc[i];
                float m = d * (wi + (float)offset);
                dx[i + j * emb] = r * m + r * (-inv_emb * (r * r) * dd * xi);
                dwp[i] += d * (xi * r);
            }
        }
    }
    for (i64 i = 0; i < emb; ++i) {
        float s = 0.0f;
        for (i64 blk = 0; blk < nblk; ++blk) s += part[blk * emb + i];
        dw[i] = s;
    }
    free(part);
}

/* ----------------------------------------------------------------- layer norm */

/* y = (x - mu) rstd w + b, biased variance.  FAITHFUL follows _layer_norm!
 * (src/layer_norm.jl:8-63): mean, then centred variance, each per-thread * 1/emb + tree. */
void orc_ln_fwd(int mode, i64 emb, i64 n, const double* x, const double* w, const double* b,
                double eps, double* y, double* mu, double* rstd) {
#pragma omp parallel for schedule(static)
    for (i64 j = 0; j < n; ++j) {
        const double* xc = x + j * emb;
        double* yc = y + j * emb;
        if (mode == 0) {
            double m = 0.0, v = 0.0;
            for (i64 i = 0; i < emb; ++i) m += xc[i];
            m /= (double)emb;
            for (i64 i = 0; i < emb; ++i) v += (xc[i] - m) * (xc[i] - m);
            v /= (double)emb;
            double r = 1.0 / sqrt(v + eps);
            mu[j] = m;
            rstd[j] = r;
            for (i64 i = 0; i < emb; ++i) yc[i] = (xc[i] - m) * r * w[i] + b[i];
        } else {
            const int gsz = 256;
            float part[256];
            float inv_emb = 1.0f / (float)emb;
            for (int t = 0; t < gsz; ++t) {
                float p = 0.0f;
                for (i64 i = t; i < emb; i += gsz) p += (float)xc[i];
                part[t] = p * inv_emb;
            }
            float m = tree_sum_f(part, gsz);
            for (int t = 0; t < gsz; ++t) {
                float p = 0.0f;
                for (i64 i = t; i < emb; i += gsz) { float c = (float)xc[i] - m; p += c * c; }
                part[t] = p * inv_emb;
            }
            float v = tree_sum_f(part, gsz);
            float r = 1.0f / sqrtf(v + (float)eps);
            mu[j] = m;
            rstd[j] = r;
            for (i64 i = 0; i < emb; ++i) {
                float c = (float)xc[i] - m;
                yc[i] = c * r * (float)w[i] + (float)b[i];
            }
        }
    }
}

/* Layer norm backward: xn = (x-mu) rstd; c1 = mean(w dy xn); c2 = mean(w dy);
 * dx = (w dy - (xn c1 + c2)) rstd; dw = sum dy xn; db = sum dy.
 * FAITHFUL follows _∇layer_norm! (src/layer_norm.jl:65-148) with float32 partials. */
void orc_ln_bwd(int mode, i64 emb, i64 n, const double* dy, const double* mu, const double* rstd,
                const double* x, const double* w, double* dx, double* dw, double* db) {
    if (mode == 0) {
        for (i64 i = 0; i < emb; ++i) dw[i] = db[i] = 0.0;
        for (i64 j = 0; j < n; ++j) {
            const double *g = dy + j * emb, *xc = x + j * emb;
            double m = mu[j], r = rstd[j], c1 = 0.0, c2 = 0.0;
            for (i64 i = 0; i < emb; ++i) {
                double xn = (xc[i] - m) * r;
                c1 += w[i] * g[i] * xn;
                c2 += w[i] * g[i];
            }
            c1 /= (double)emb;
            c2 /= (double)emb;
            for (i64 i = 0; i < emb; ++i) {
                double xn = (xc[i] - m) * r;
                dx[i + j * emb] = (w[i] * g[i] - (xn * c1 + c2)) * r;
                dw[i] += g[i] * xn;
                db[i] += g[i];
            }
        }
        return;
    }
    const int gsz = 256, bpg = 4;
    float inv_emb = 1.0f / (float)emb;
    i64 nblk = (n + bpg - 1) / bpg;
    float* pw = (float*)calloc((size_t)(nblk * emb), sizeof(float));
    float* pb = (float*)calloc((size_t)(nblk * emb), sizeof(float));
#pragma omp parallel for schedule(static)
    for (i64 blk = 0; blk < nblk; ++blk) {
        float r1[256], r2[256];
        i64 je = (blk + 1) * bpg < n ? (blk + 1) * bpg : n;
        for (i64 j = blk * bpg; j < je; ++j) {
            const double *g = dy + j * emb, *xc = x + j * emb;
            float m = (float)mu[j], r = (float)rstd[j];
            for (int t = 0; t < gsz; ++t) {
                float c1 = 0.0f, c2 = 0.0f;
                for (i64 i = t; i < emb; i += gsz) {
                    float xn = ((float)xc[i] - m) * r, wdy = (float)w[i] * (float)g[i];
                    c1 += wdy * xn;
                    c2 += wdy;
                }
                r1[t] = c1 * inv_emb;
                r2[t] = c2 * inv_emb;
            }
            float c1 = tree_sum_f(r1, gsz), c2 = tree_sum_f(r2, gsz);
            for (i64 i = 0; i < emb; ++i) {
                float d = (float)g[i];
                float xn = ((float)xc[i] - m) * r, wdy = (float)w[i] * d;
                dx[i + j * emb] = (wdy - (xn * c1 + c2)) * r;
                pw[blk * emb + i] += d * xn;
                pb[blk * emb + i] += d;
            }
        }
    }
    for (i64 i = 0; i < emb; ++i) {
        float sw = 0.0f, sb = 0.0f;
        for (i64 blk = 0; blk < nblk; ++blk) { sw += pw[blk * emb + i]; sb += pb[blk * emb + i]; }
        dw[i] = sw;
        db[i] = sb;
    }
    free(pw);
    free(pb);
}

/* ----------------------------------------------------------------------- RoPE */

/* LlamaRotaryEmbedding (src/rope/llama_rope.jl:7-22): inv_freq = 1/base^((0:2:dim-1)/dim),
 * freqs = inv_freq * pos, cos/sin = vcat(freqs, freqs) of shape (dim, L, B).
 * pos is (L, B).  FAITHFUL computes in float32 like the reference; EXACT in float64. */
void orc_rotary_embedding(int mode, i64 dim, double base, i64 L, i64 B, const double* pos,
                          double* cosv, double* sinv) {
    i64 half = dim / 2;
    for (i64 b = 0; b < B; ++b)
        for (i64 l = 0; l < L; ++l)
            for (i64 i = 0; i < half; ++i) {
                double c, s;
                if (mode == 0) {
                    double f = pos[l + L * b] / pow(base, (double)(2 * i) / (double)dim);
                    c = cos(f);
                    s = sin(f);
                } else {
                    float id = (float)(2 * i) / (float)dim;
                    float inv = 1.0f / powf((float)base, id);
                    float f = inv * (float)pos[l + L * b];
                    c = cosf(f);
                    s = sinf(f);
                }
                i64 o = dim * (l + L * b);
                cosv[o + i] = cosv[o + i + half] = c;
                sinv[o + i] = sinv[o + i + half] = s;
            }
}

/* Rotate-half RoPE of q (E, L, QH, B) and k (E, L, KH, B) with cos/sin (E, L, B),
 * rows 1..E/2 read (llama_rope!, src/rope/llama_rope.jl:24-65). */
void orc_rope(int mode, i64 E, i64 L, i64 QH, i64 KH, i64 B, const double* q, const double* k,
              const double* cosv, const double* sinv, double sin_sign, double* qo, double* ko) {
    i64 half = E / 2;
    for (int which = 0; which < 2; ++which) {
        const double* x = which ? k : q;
        double* y = which ? ko : qo;
        i64 H = which ? KH : QH;
        for (i64 b = 0; b < B; ++b)
            for (i64 h = 0; h < H; ++h)
                for (i64 l = 0; l < L; ++l)
                    for (i64 i = 0; i < half; ++i) {
                        i64 cs = i + E * (l + L * b);
                        i64 base = E * (l + L * (h + H * b));
                        if (mode == 0) {
                            double c = cosv[cs], s = sinv[cs] * sin_sign;
                            double x1 = x[base + i], x2 = x[base + i + half];
                            y[base + i] = x1 * c - x2 * s;
                            y[base + i + half] = x2 * c + x1 * s;
                        } else {
                            float c = (float)cosv[cs], s = (float)sinv[cs] * (float)sin_sign;
                            float x1 = (float)x[base + i], x2 = (float)x[base + i + half];
                            y[base + i] = x1 * c - x2 * s;
                            y[base + i + half] = x2 * c + x1 * s;
                        }
                    }
    }
}

/* ------------------------------------------------------------------ attention */

#define QIDX(e, i, h, b) ((e) + E * ((i) + QL * ((h) + QH * (b))))
#define KIDX(e, j, h, b) ((e) + E * ((j) + KL * ((h) + KH * (b))))
#define PIDX(h, i, j, b) ((h) + QH * ((i) + QL * ((j) + KL * (b))))
#define SIDX(i, h, b) ((i) + QL * ((h) + QH * (b)))

static int key_masked(int causal, const uint8_t* kpad, i64 KL, i64 i, i64 j, i64 b) {
    if (causal && j > i) return 1;
    if (kpad && !kpad[j + KL * b]) return 1;
    return 0;
}

/* EXACT forward: o = softmax(scale q.k + pair + masks) v in float64 per row. */
static void attn_fwd_exact(i64 E, i64 QL, i64 KL, i64 QH, i64 KH, i64 B, const double* q,
                           const double* k, const double* v, const double* pair,
                           const uint8_t* kpad, int causal, double scale, double* o,
                           double* ms, double* ls) {
    i64 rep = QH / KH;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (i64 b = 0; b < B; ++b)
        for (i64 h = 0; h < QH; ++h) {
            i64 kh = h / rep;
            double* s = (double*)malloc(sizeof(double) * (size_t)KL);
            for (i64 i = 0; i < QL; ++i) {
                double m = -INFINITY;
                for (i64 j = 0; j < KL; ++j) {
                    if (key_masked(causal, kpad, KL, i, j, b)) { s[j] = -INFINITY; continue; }
                    double d = 0.0;
                    for (i64 e = 0; e < E; ++e) d += q[QIDX(e, i, h, b)] * k[KIDX(e, j, kh, b)];
                    d *= scale;
                    if (pair) d += pair[PIDX(h, i, j, b)];
                    s[j] = d;
                    if (d > m) m = d;
                }
                double l = 0.0;
                for (i64 e = 0; e < E; ++e) o[QIDX(e, i, h, b)] = 0.0;
                if (m == -INFINITY) { ms[SIDX(i, h, b)] = -INFINITY; ls[SIDX(i, h, b)] = 0.0; continue; }
                for (i64 j = 0; j < KL; ++j) {
                    if (s[j] == -INFINITY) continue;
                    double p = exp(s[j] - m);
                    l += p;
                    for (i64 e = 0; e < E; ++e) o[QIDX(e, i, h, b)] += p * v[KIDX(e, j, kh, b)];
                }
                for (i64 e = 0; e < E; ++e) o[QIDX(e, i, h, b)] /= l;
                ms[SIDX(i, h, b)] = m;
                ls[SIDX(i, h, b)] = l;
            }
            free(s);
        }
}

/* FAITHFUL forward: _flash_attention_fwd! (src/attention.jl:8-143) for T = Float32 with
 * group size gsz: per q-tile, K tiles up to the diagonal when causal (:55), scores
 * scaled then biased (:63-74), causal then kpad masks (:77-89), tile max/sum (:92-104),
 * the rescale of P and O by beta/l_new and l_i alpha/l_new (:107-120), O += P V (:125-127). */
static void attn_fwd_faithful(i64 E, i64 QL, i64 KL, i64 QH, i64 KH, i64 B, const double* q,
                              const double* k, const double* v, const double* pair,
                              const uint8_t* kpad, int causal, float scale, int gsz, double* o,
                              double* ms, double* ls) {
    i64 rep = QH / KH;
    i64 qtiles = (QL + gsz - 1) / gsz, ktiles = (KL + gsz - 1) / gsz;
    int in_bounds = (QL % gsz == 0) && (KL % gsz == 0);
    (void)in_bounds;
#pragma omp parallel for collapse(3) schedule(dynamic)
    for (i64 b = 0; b < B; ++b)
        for (i64 h = 0; h < QH; ++h)
            for (i64 qt = 0; qt < qtiles; ++qt) {
                i64 kh = h / rep;
                float* qs = (float*)malloc(sizeof(float) * (size_t)(E * gsz));
                float* ks = (float*)malloc(sizeof(float) * (size_t)(E * gsz));
                float* vs = (float*)malloc(sizeof(float) * (size_t)(E * gsz));
                float* os = (float*)calloc((size_t)(E * gsz), sizeof(float));
                float* ss = (float*)malloc(sizeof(float) * (size_t)gsz);
                float* mi = (float*)malloc(sizeof(float) * (size_t)gsz);
                float* li = (float*)malloc(sizeof(float) * (size_t)gsz);
                i64 q0 = qt * gsz;
                for (int t = 0; t < gsz; ++t) {
                    mi[t] = -INFINITY;
                    li[t] = 0.0f;
                    for (i64 e = 0; e < E; ++e)
                        qs[t * E + e] = (q0 + t < QL) ? (float)q[QIDX(e, q0 + t, h, b)] : 0.0f;
                }
                i64 end_iter = causal ? qt + 1 : ktiles;
                for (i64 it = 0; it < end_iter; ++it) {
                    i64 k0 = it * gsz;
                    for (int t = 0; t < gsz; ++t)
                        for (i64 e = 0; e < E; ++e) {
                            int ok = k0 + t < KL;
                            ks[t * E + e] = ok ? (float)k[KIDX(e, k0 + t, kh, b)] : 0.0f;
                            vs[t * E + e] = ok ? (float)v[KIDX(e, k0 + t, kh, b)] : 0.0f;
                        }
                    for (int t = 0; t < gsz; ++t) {
                        i64 qi = q0 + t;
                        int in_q = qi < QL;
                        for (int c = 0; c < gsz; ++c) {
                            float acc = 0.0f;
                            for (i64 e = 0; e < E; ++e) acc += qs[t * E + e] * ks[c * E + e];
                            ss[c] = acc * scale;
                        }
                        if (pair)
                            for (int c = 0; c < gsz; ++c) {
                                if (!(in_q && k0 + c < KL)) break;
                                ss[c] += (float)pair[PIDX(h, qi, k0 + c, b)];
                            }
                        if (causal)
                            for (int c = 0; c < gsz; ++c) {
                                if (!(k0 + c < KL)) break;
                                ss[c] = (qi >= k0 + c) ? ss[c] : -INFINITY;
                            }
                        if (kpad)
                            for (int c = 0; c < gsz; ++c) {
                                if (!(k0 + c < KL)) break;
                                ss[c] = kpad[k0 + c + KL * b] ? ss[c] : -INFINITY;
                            }
                        float mij = -INFINITY;
                        for (int c = 0; c < gsz; ++c) {
                            if (!(k0 + c < KL)) break;
                            mij = fmaxf(mij, ss[c]);
                        }
                        float lij = 0.0f;
                        for (int c = 0; c < gsz; ++c) {
                            if (!(k0 + c < KL)) break;
                            float tmp = expf(ss[c] - mij);
                            lij += tmp;
                            ss[c] = tmp;
                        }
                        float mnew = fmaxf(mi[t], mij);
                        float alpha = expf(mi[t] - mnew), beta = expf(mij - mnew);
                        float lnew = alpha * li[t] + beta * lij;
                        float pscale = beta / lnew, oscale = li[t] / lnew * alpha;
                        for (int c = 0; c < gsz; ++c) ss[c] *= pscale;
                        for (i64 e = 0; e < E; ++e) {
                            float acc = 0.0f;
                            for (int c = 0; c < gsz; ++c) acc += ss[c] * vs[c * E + e];
                            os[t * E + e] = os[t * E + e] * oscale + acc;
                        }
                        mi[t] = mnew;
                        li[t] = lnew;
                    }
                }
                for (int t = 0; t < gsz; ++t) {
                    i64 qi = q0 + t;
                    if (qi >= QL) continue;
                    for (i64 e = 0; e < E; ++e) o[QIDX(e, qi, h, b)] = os[t * E + e];
                    ms[SIDX(qi, h, b)] = mi[t];
                    ls[SIDX(qi, h, b)] = li[t];
                }
                free(qs); free(ks); free(vs); free(os); free(ss); free(mi); free(li);
            }
}

void orc_attn_fwd(int mode, i64 E, i64 QL, i64 KL, i64 QH, i64 KH, i64 B, const double* q,
                  const double* k, const double* v, const double* pair, const uint8_t* kpad,
                  int causal, double scale, int gsz, double* o, double* ms, double* ls) {
    if (mode == 0)
        attn_fwd_exact(E, QL, KL, QH, KH, B, q, k, v, pair, kpad, causal, scale, o, ms, ls);
    else
        attn_fwd_faithful(E, QL, KL, QH, KH, B, q, k, v, pair, kpad, causal, (float)scale, gsz, o, ms, ls);
}

/* EXACT backward: analytic gradients of o = P v with P = softmax(S), S = scale q.k + pair
 * + masks, in float64; dpair = dS (zero where masked).  With qk_fp16 it is the float64
 * mathematics of the reference's backward: the row statistics (m, l) and o, hence
 * delta = rowsum(dO o), come from the unrounded forward, while the recomputed scores,
 * dK and dQ use Q and K rounded to float16 (src/attention_bwd.jl:20-21,88-92,197-210),
 * so P = exp(S16 - m) / l is not renormalised. */
static void attn_bwd_exact(i64 E, i64 QL, i64 KL, i64 QH, i64 KH, i64 B, const double* dO,
                           const double* q, const double* k, const double* v,
                           const double* pair, const uint8_t* kpad, int causal, double scale,
                           int qk_fp16, double* dq, double* dk, double* dv, double* dpair) {
    i64 rep = QH / KH;
    i64 nq = E * QL * QH * B, nk = E * KL * KH * B;
    double* qq = (double*)malloc(sizeof(double) * (size_t)nq);
    double* kk = (double*)malloc(sizeof(double) * (size_t)nk);
    for (i64 i = 0; i < nq; ++i) qq[i] = qk_fp16 ? orc_round_f16((float)q[i]) : q[i];
    for (i64 i = 0; i < nk; ++i) kk[i] = qk_fp16 ? orc_round_f16((float)k[i]) : k[i];
    memset(dq, 0, sizeof(double) * (size_t)nq);
    memset(dk, 0, sizeof(double) * (size_t)nk);
    memset(dv, 0, sizeof(double) * (size_t)nk);
    if (dpair) memset(dpair, 0, sizeof(double) * (size_t)(QH * QL * KL * B));
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (i64 b = 0; b < B; ++b)
        for (i64 kh = 0; kh < KH; ++kh) {
            double* s = (double*)malloc(sizeof(double) * (size_t)KL);
            double* sf = (double*)malloc(sizeof(double) * (size_t)KL);
            double* dp = (double*)malloc(sizeof(double) * (size_t)KL);
            double* orow = (double*)malloc(sizeof(double) * (size_t)E);
            for (i64 h = kh * rep; h < (kh + 1) * rep; ++h)
                for (i64 i = 0; i < QL; ++i) {
                    double m = -INFINITY;
                    for (i64 j = 0; j < KL; ++j) {
                        if (key_masked(causal, kpad, KL, i, j, b)) { s[j] = sf[j] = -INFINITY; continue; }
                        double d = 0.0, df = 0.0;
                        for (i64 e = 0; e < E; ++e) {
                            d += qq[QIDX(e, i, h, b)] * kk[KIDX(e, j, kh, b)];
                            df += q[QIDX(e, i, h, b)] * k[KIDX(e, j, kh, b)];
                        }
                        d *= scale;
                        df *= scale;
                        if (pair) { d += pair[PIDX(h, i, j, b)]; df += pair[PIDX(h, i, j, b)]; }
                        s[j] = d;
                        sf[j] = df;
                        if (df > m) m = df;
                    }
                    if (m == -INFINITY) continue;
                    /* forward statistics and output from the unrounded scores */
                    double l = 0.0;
                    for (i64 j = 0; j < KL; ++j) if (sf[j] != -INFINITY) l += exp(sf[j] - m);
                    for (i64 e = 0; e < E; ++e) orow[e] = 0.0;
                    for (i64 j = 0; j < KL; ++j) {
                        if (sf[j] == -INFINITY) continue;
                        double p = exp(sf[j] - m) / l;
                        for (i64 e = 0; e < E; ++e) orow[e] += p * v[KIDX(e, j, kh, b)];
                    }
                    double delta = 0.0;
                    for (i64 e = 0; e < E; ++e) delta += dO[QIDX(e, i, h, b)] * orow[e];
                    for (i64 j = 0; j < KL; ++j) {
                        if (s[j] == -INFINITY) { dp[j] = 0.0; s[j] = 0.0; continue; }
                        s[j] = exp(s[j] - m) / l; /* P from the (possibly rounded) scores */
                        double d = 0.0;
                        for (i64 e = 0; e < E; ++e) d += dO[QIDX(e, i, h, b)] * v[KIDX(e, j, kh, b)];
                        dp[j] = d;
                    }
                    for (i64 j = 0; j < KL; ++j) {
                        double p = s[j];
                        if (p == 0.0) continue;
                        double ds = p * (dp[j] - delta);
                        if (dpair) dpair[PIDX(h, i, j, b)] = ds;
                        for (i64 e = 0; e < E; ++e) {
                            dv[KIDX(e, j, kh, b)] += p * dO[QIDX(e, i, h, b)];
                            dk[KIDX(e, j, kh, b)] += scale * ds * qq[QIDX(e, i, h, b)];
                            dq[QIDX(e, i, h, b)] += scale * ds * kk[KIDX(e, j, kh, b)];
                        }
                    }
                }
            free(s);
            free(sf);
            free(dp);
            free(orow);
        }
    free(qq);
    free(kk);
}

/* FAITHFUL backward: _flash_attention_bwd_preprocess! (src/attention_bwd.jl:177-211) and
 * _flash_attention_bwd! (src/attention_bwd.jl:1-175) for T = Float32: Q and K held as
 * Float16 (:20-21) and widened to Float32 in the products (mma! registers are eltype(C),
 * src/mma.jl:19-21); per K tile, per Q tile (from the diagonal when causal, :40-49):
 * P~ = exp(S - m) (:88-92, m = +Inf past QL), dV += dO~^T P~ (:96-109), dP = dO~ V^T
 * (:112-123), dS = P~ (dP - delta) scale (:125-130), dpair = dS/scale (:133-142),
 * dK += dS^T Q (:144-156), dQ = dQ + dS K (:158-170). */
static void attn_bwd_faithful(i64 E, i64 QL, i64 KL, i64 QH, i64 KH, i64 B, const double* dO,
                              const double* o, const double* ms, const double* ls,
                              const double* q, const double* k, const double* v,
                              const double* pair, const uint8_t* kpad, int causal, float scale,
                              int gsz, int qk_fp16, double* dq, double* dk, double* dv,
                              double* dpair) {
    i64 rep = QH / KH;
    i64 qtiles = (QL + gsz - 1) / gsz, ktiles = (KL + gsz - 1) / gsz;
    i64 nq = E * QL * QH * B, nk = E * KL * KH * B;
    float* dts = (float*)malloc(sizeof(float) * (size_t)nq); /* dO / l */
    float* del = (float*)malloc(sizeof(float) * (size_t)(QL * QH * B));
    float* fdq = (float*)calloc((size_t)nq, sizeof(float));
    float* fdk = (float*)calloc((size_t)nk, sizeof(float));
    float* fdv = (float*)calloc((size_t)nk, sizeof(float));
    for (i64 b = 0; b < B; ++b)
        for (i64 h = 0; h < QH; ++h)
            for (i64 i = 0; i < QL; ++i) {
                float inv = 1.0f / (float)ls[SIDX(i, h, b)];
                float d = 0.0f;
                for (i64 e = 0; e < E; ++e) {
                    float t = (float)dO[QIDX(e, i, h, b)] * inv;
                    dts[QIDX(e, i, h, b)] = t;
                    d += t * (float)o[QIDX(e, i, h, b)];
                }
                del[SIDX(i, h, b)] = d;
            }
    if (dpair) memset(dpair, 0, sizeof(double) * (size_t)(QH * QL * KL * B));
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (i64 b = 0; b < B; ++b)
        for (i64 kh = 0; kh < KH; ++kh) {
            float* ks = (float*)malloc(sizeof(float) * (size_t)(E * gsz));
            float* vs = (float*)malloc(sizeof(float) * (size_t)(E * gsz));
            float* qs = (float*)malloc(sizeof(float) * (size_t)(E * gsz));
            float* ds = (float*)malloc(sizeof(float) * (size_t)(E * gsz));
            float* P = (float*)malloc(sizeof(float) * (size_t)(gsz * gsz));
            float* S = (float*)malloc(sizeof(float) * (size_t)(gsz * gsz));
            for (i64 h = kh * rep; h < (kh + 1) * rep; ++h)
                for (i64 kt = 0; kt < ktiles; ++kt) {
                    i64 k0 = kt * gsz;
                    for (int c = 0; c < gsz; ++c)
                        for (i64 e = 0; e < E; ++e) {
                            int ok = k0 + c < KL;
                            float kv = ok ? (float)k[KIDX(e, k0 + c, kh, b)] : 0.0f;
                            ks[c * E + e] = qk_fp16 ? orc_round_f16(kv) : kv;
                            vs[c * E + e] = ok ? (float)v[KIDX(e, k0 + c, kh, b)] : 0.0f;
                        }
                    for (i64 qt = causal ? kt : 0; qt < qtiles; ++qt) {
                        i64 q0 = qt * gsz;
                        for (int t = 0; t < gsz; ++t)
                            for (i64 e = 0; e < E; ++e) {
                                int ok = q0 + t < QL;
                                float qv = ok ? (float)q[QIDX(e, q0 + t, h, b)] : 0.0f;
                                qs[t * E + e] = qk_fp16 ? orc_round_f16(qv) : qv;
                                ds[t * E + e] = ok ? dts[QIDX(e, q0 + t, h, b)] : 0.0f;
                            }
                        for (int t = 0; t < gsz; ++t) {
                            i64 qi = q0 + t;
                            int in_q = qi < QL;
                            float* Sr = S + (i64)t * gsz;
                            for (int c = 0; c < gsz; ++c) {
                                float acc = 0.0f;
                                for (i64 e = 0; e < E; ++e) acc += qs[t * E + e] * ks[c * E + e];
                                Sr[c] = acc * scale;
                            }
                            if (pair)
                                for (int c = 0; c < gsz; ++c) {
                                    if (!(in_q && k0 + c < KL)) break;
                                    Sr[c] += (float)pair[PIDX(h, qi, k0 + c, b)];
                                }
                            if (causal)
                                for (int c = 0; c < gsz; ++c) {
                                    if (!(k0 + c < KL)) break;
                                    Sr[c] = (qi >= k0 + c) ? Sr[c] : -INFINITY;
                                }
                            if (kpad)
                                for (int c = 0; c < gsz; ++c) {
                                    if (!(k0 + c < KL)) break;
                                    Sr[c] = kpad[k0 + c + KL * b] ? Sr[c] : -INFINITY;
                                }
                            float mi = in_q ? (float)ms[SIDX(qi, h, b)] : INFINITY;
                            for (int c = 0; c < gsz; ++c) P[t * gsz + c] = expf(Sr[c] - mi);
                        }
                        /* dV[:, c] += sum_t dts[t] P[t, c] */
                        for (int c = 0; c < gsz; ++c) {
                            if (k0 + c >= KL) continue;
                            for (i64 e = 0; e < E; ++e) {
                                float acc = 0.0f;
                                for (int t = 0; t < gsz; ++t) acc += ds[t * E + e] * P[t * gsz + c];
                                fdv[KIDX(e, k0 + c, kh, b)] += acc;
                            }
                        }
                        /* dS */
                        for (int t = 0; t < gsz; ++t) {
                            i64 qi = q0 + t;
                            float di = qi < QL ? del[SIDX(qi, h, b)] : 0.0f;
                            for (int c = 0; c < gsz; ++c) {
                                float acc = 0.0f;
                                for (i64 e = 0; e < E; ++e) acc += ds[t * E + e] * vs[c * E + e];
                                S[t * gsz + c] = P[t * gsz + c] * (acc - di) * scale;
                            }
                        }
                        if (dpair)
                            for (int t = 0; t < gsz; ++t) {
                                i64 qi = q0 + t;
                                for (int c = 0; c < gsz; ++c) {
                                    if (k0 + c >= KL) break;
                                    if (qi < QL) dpair[PIDX(h, qi, k0 + c, b)] = S[t * gsz + c] / scale;
                                }
                            }
                        /* dK[:, c] += sum_t dS[t, c] Q[t] */
                        for (int c = 0; c < gsz; ++c) {
                            if (k0 + c >= KL) continue;
                            for (i64 e = 0; e < E; ++e) {
                                float acc = 0.0f;
                                for (int t = 0; t < gsz; ++t) acc += S[t * gsz + c] * qs[t * E + e];
                                fdk[KIDX(e, k0 + c, kh, b)] += acc;
                            }
                        }
                        /* dQ[:, t] = dQ + sum_c dS[t, c] K[c] */
                        for (int t = 0; t < gsz; ++t) {
                            i64 qi = q0 + t;
                            if (qi >= QL) continue;
                            for (i64 e = 0; e < E; ++e) {
                                float acc = 0.0f;
                                for (int c = 0; c < gsz; ++c) acc += S[t * gsz + c] * ks[c * E + e];
                                fdq[QIDX(e, qi, h, b)] = fdq[QIDX(e, qi, h, b)] + acc;
                            }
                        }
                    }
                }
            free(ks); free(vs); free(qs); free(ds); free(P); free(S);
        }
    for (i64 i = 0; i < nq; ++i) dq[i] = fdq[i];
    for (i64 i = 0; i < nk; ++i) { dk[i] = fdk[i]; dv[i] = fdv[i]; }
    free(dts); free(del); free(fdq); free(fdk); free(fdv);
}

void orc_attn_bwd(int mode, i64 E, i64 QL, i64 KL, i64 QH, i64 KH, i64 B, const double* dO,
                  const double* o, const double* ms, const double* ls, const double* q,
                  const double* k, const double* v, const double* pair, const uint8_t* kpad,
                  int causal, double scale, int gsz, int qk_fp16, double* dq, double* dk,
                  double* dv, double* dpair) {
    if (mode == 0)
        attn_bwd_exact(E, QL, KL, QH, KH, B, dO, q, k, v, pair, kpad, causal, scale, qk_fp16,
                       dq, dk, dv, dpair);
    else
        attn_bwd_faithful(E, QL, KL, QH, KH, B, dO, o, ms, ls, q, k, v, pair, kpad, causal,
                          (float)scale, gsz, qk_fp16, dq, dk, dv, dpair);
}

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int orc_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
