/*
 * conv_oracle.c - CPU restatement of the reference's 2-D convolution path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path links or calls this
 * file; tests/ and the benchmark's baseline leg use it as the checker.
 *
 * Tensors are contiguous NCHW (the reference makes every operand contiguous
 * first, src/api/ops/conv.cpp:1101-1103,1145-1147). Weights are
 * [Cout][Cin/groups][KH][KW]. Element storage follows gemm_oracle.c (float32,
 * or 16-bit patterns for float16 / bfloat16); accumulation is float32.
 *
 * Restated (reference file:line):
 *   - implicit-GEMM forward: y[n, g*Cy+m, o] = sum over (c, tap) of
 *     W[g*Cy+m, c, tap] * x[n, g*Cx+c, o*s - p + tap*d], zero outside the
 *     input, + bias (src/shaders/helpers/conv.slang:198-207,280-312;
 *     src/api/ops/conv.cpp:1014-1022). k runs over (c, kh, kw) in that order.
 *   - grad input: dx[n, g*Cx+c, i] = sum over (m, tap) of W[g*Cy+m, c, tap] *
 *     dy[n, g*Cy+m, (i + p - tap*d)/s] where the division is exact and in range
 *     (src/shaders/helpers/conv.slang:320-362; conv.cpp:1024-1032).
 *   - grad weight: dW[g*Cy+m, c, tap] = sum over (n, o) of dy[n, g*Cy+m, o] *
 *     x[n, g*Cx+c, o*s - p + tap*d] (conv.slang:447-484; conv.cpp:1034-1060).
 *     The reference splits this sum into chunks of float32 partials; here the
 *     sum is taken in float64 (acc64 = 1) or in float32 in order (acc64 = 0).
 *   - Winograd F(2x2,3x3) forward with U, V and M rounded to the storage type
 *     (src/shaders/helpers/winograd.slang:27-133,
 *     src/shaders/ops/winograd_transform.slang:9-47, conv.cpp:958-988), the
 *     reference's choice for 3x3 / stride 1 / dilation 1 / pad <= 2 / groups 1
 *     / fp16 or fp32 / >= 16 channels (conv.cpp:941-955).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2 };

uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float f);
float oracle_bf16_to_f32(uint16_t b);

static inline float ld(int dt, const void* p, int64_t i) {
    switch (dt) {
    case OR_F32: return ((const float*)p)[i];
    case OR_F16: return oracle_f16_to_f32(((const uint16_t*)p)[i]);
    default: return oracle_bf16_to_f32(((const uint16_t*)p)[i]);
    }
}

static inline void st(int dt, void* p, int64_t i, float v) {
    switch (dt) {
    case OR_F32: ((float*)p)[i] = v; break;
    case OR_F16: ((uint16_t*)p)[i] = oracle_f32_to_f16(v); break;
    default: ((uint16_t*)p)[i] = oracle_f32_to_bf16(v); break;
    }
}

/* round a float32 to the storage type and back (the reference's T.fromAccum) */
static inline float rt(int dt, float v) {
    switch (dt) {
    case OR_F32: return v;
    case OR_F16: return oracle_f16_to_f32(oracle_f32_to_f16(v));
    default: return oracle_bf16_to_f32(oracle_f32_to_bf16(v));
    }
}

typedef struct {
    int64_t n, cin, h, w, cout, kh, kw;
    int64_t sh, sw, ph, pw, dh, dw, groups;
    int64_t ho, wo;
} conv_geom;

static int geom_ok(const conv_geom* g) {
    if (g->n < 0 || g->cin <= 0 || g->cout <= 0 || g->groups <= 0) return 0;
    if (g->cin % g->groups || g->cout % g->groups) return 0;
    if (g->kh <= 0 || g->kw <= 0 || g->sh <= 0 || g->sw <= 0 || g->dh <= 0 || g->dw <= 0) return 0;
    return g->ho >= 0 && g->wo >= 0;
}

/* rows [m_begin, m_end) of output channels for sample n: the caller splits
 * work over threads */
int oracle_conv_fwd(int dt, const conv_geom* g, int64_t nb, int64_t ne, const void* x, const void* wt,
                    const void* bias, void* y) {
    if (!geom_ok(g)) return -1;
    const int64_t cx = g->cin / g->groups, cy = g->cout / g->groups;
    for (int64_t n = nb; n < ne; ++n)
        for (int64_t oc = 0; oc < g->cout; ++oc) {
            const int64_t grp = oc / cy;
            for (int64_t oh = 0; oh < g->ho; ++oh)
                for (int64_t ow = 0; ow < g->wo; ++ow) {
                    float acc = 0.0f;
                    for (int64_t c = 0; c < cx; ++c)
                        for (int64_t a = 0; a < g->kh; ++a)
                            for (int64_t b = 0; b < g->kw; ++b) {
                                const int64_t ih = oh * g->sh - g->ph + a * g->dh;
                                const int64_t iw = ow * g->sw - g->pw + b * g->dw;
                                float xv = 0.0f;
                                if (ih >= 0 && ih < g->h && iw >= 0 && iw < g->w)
                                    xv = ld(dt, x, ((n * g->cin + grp * cx + c) * g->h + ih) * g->w + iw);
                                const float wv = ld(dt, wt, ((oc * cx + c) * g->kh + a) * g->kw + b);
                                acc = fmaf(wv, xv, acc);
                            }
                    if (bias) acc = acc + ld(dt, bias, oc);
                    st(dt, y, ((n * g->cout + oc) * g->ho + oh) * g->wo + ow, acc);
                }
        }
    return 0;
}

int oracle_conv_dgrad(int dt, const conv_geom* g, int64_t nb, int64_t ne, const void* dy, const void* wt, void* dx) {
    if (!geom_ok(g)) return -1;
    const int64_t cx = g->cin / g->groups, cy = g->cout / g->groups;
    for (int64_t n = nb; n < ne; ++n)
        for (int64_t ic = 0; ic < g->cin; ++ic) {
            const int64_t grp = ic / cx, c = ic % cx;
            for (int64_t ih = 0; ih < g->h; ++ih)
                for (int64_t iw = 0; iw < g->w; ++iw) {
                    float acc = 0.0f;
                    for (int64_t m = 0; m < cy; ++m)
                        for (int64_t a = 0; a < g->kh; ++a)
                            for (int64_t b = 0; b < g->kw; ++b) {
                                const int64_t th = ih + g->ph - a * g->dh, tw = iw + g->pw - b * g->dw;
                                if (th < 0 || tw < 0 || th % g->sh || tw % g->sw) continue;
                                const int64_t oh = th / g->sh, ow = tw / g->sw;
                                if (oh >= g->ho || ow >= g->wo) continue;
                                const int64_t oc = grp * cy + m;
                                acc = fmaf(ld(dt, wt, ((oc * cx + c) * g->kh + a) * g->kw + b),
                                           ld(dt, dy, ((n * g->cout + oc) * g->ho + oh) * g->wo + ow), acc);
                            }
                    st(dt, dx, ((n * g->cin + ic) * g->h + ih) * g->w + iw, acc);
                }
        }
    return 0;
}

/* output channels [ob, oe) */
int oracle_conv_wgrad(int dt, const conv_geom* g, int64_t ob, int64_t oe, const void* x, const void* dy, void* dw,
                      int acc64) {
    if (!geom_ok(g)) return -1;
    const int64_t cx = g->cin / g->groups, cy = g->cout / g->groups;
    for (int64_t oc = ob; oc < oe; ++oc) {
        const int64_t grp = oc / cy;
        for (int64_t c = 0; c < cx; ++c)
            for (int64_t a = 0; a < g->kh; ++a)
                for (int64_t b = 0; b < g->kw; ++b) {
                    float acc = 0.0f;
                    double acc_d = 0.0;
                    for (int64_t n = 0; n < g->n; ++n)
                        for (int64_t oh = 0; oh < g->ho; ++oh)
                            for (int64_t ow = 0; ow < g->wo; ++ow) {
                                const int64_t ih = oh * g->sh - g->ph + a * g->dh;
                                const int64_t iw = ow * g->sw - g->pw + b * g->dw;
                                if (ih < 0 || ih >= g->h || iw < 0 || iw >= g->w) continue;
                                const float yv = ld(dt, dy, ((n * g->cout + oc) * g->ho + oh) * g->wo + ow);
                                const float xv = ld(dt, x, ((n * g->cin + grp * cx + c) * g->h + ih) * g->w + iw);
                                if (acc64) acc_d += (double)yv * (double)xv;
                                else acc = fmaf(yv, xv, acc);
                            }
                    st(dt, dw, ((oc * cx + c) * g->kh + a) * g->kw + b, acc64 ? (float)acc_d : acc);
                }
    }
    return 0;
}

/* Winograd F(2x2,3x3) forward of the reference, samples [nb, ne). Requires
 * kh = kw = 3, stride 1, dilation 1, groups 1. U, V and M are rounded to the
 * storage type between stages, as the reference stores them in it. */
int oracle_winograd_fwd(int dt, const conv_geom* g, int64_t nb, int64_t ne, const void* x, const void* wt,
                        const void* bias, void* y) {
    if (!geom_ok(g) || g->kh != 3 || g->kw != 3 || g->sh != 1 || g->sw != 1 || g->dh != 1 || g->dw != 1 || g->groups != 1)
        return -1;
    const int64_t ci = g->cin, co = g->cout;
    const int64_t th_n = (g->ho + 1) / 2, tw_n = (g->wo + 1) / 2;
    float* U = (float*)malloc(sizeof(float) * 16 * co * ci);
    float* V = (float*)malloc(sizeof(float) * 16 * ci);
    float* M = (float*)malloc(sizeof(float) * 16 * co);
    if (!U || !V || !M) { free(U); free(V); free(M); return -2; }
    /* filter transform G g G^T (winograd.slang:27-56) */
    for (int64_t r = 0; r < co; ++r)
        for (int64_t c = 0; c < ci; ++c) {
            float gg[3][3], t[4][3];
            for (int i = 0; i < 9; ++i) gg[i / 3][i % 3] = ld(dt, wt, (r * ci + c) * 9 + i);
            for (int j = 0; j < 3; ++j) {
                t[0][j] = gg[0][j];
                t[1][j] = 0.5f * (gg[0][j] + gg[1][j] + gg[2][j]);
                t[2][j] = 0.5f * (gg[0][j] - gg[1][j] + gg[2][j]);
                t[3][j] = gg[2][j];
            }
            for (int i = 0; i < 4; ++i) {
                U[((i * 4 + 0) * co + r) * ci + c] = rt(dt, t[i][0]);
                U[((i * 4 + 1) * co + r) * ci + c] = rt(dt, 0.5f * (t[i][0] + t[i][1] + t[i][2]));
                U[((i * 4 + 2) * co + r) * ci + c] = rt(dt, 0.5f * (t[i][0] - t[i][1] + t[i][2]));
                U[((i * 4 + 3) * co + r) * ci + c] = rt(dt, t[i][2]);
            }
        }
    for (int64_t n = nb; n < ne; ++n)
        for (int64_t th = 0; th < th_n; ++th)
            for (int64_t tw = 0; tw < tw_n; ++tw) {
                /* input transform B^T d B (winograd.slang:79-112) */
                for (int64_t c = 0; c < ci; ++c) {
                    float d[4][4], t[4][4];
                    for (int a = 0; a < 4; ++a)
                        for (int b = 0; b < 4; ++b) {
                            const int64_t h = 2 * th - g->ph + a, w = 2 * tw - g->pw + b;
                            d[a][b] = (h >= 0 && h < g->h && w >= 0 && w < g->w) ? ld(dt, x, ((n * ci + c) * g->h + h) * g->w + w) : 0.0f;
                        }
                    for (int b = 0; b < 4; ++b) {
                        t[0][b] = d[0][b] - d[2][b];
                        t[1][b] = d[1][b] + d[2][b];
                        t[2][b] = d[2][b] - d[1][b];
                        t[3][b] = d[1][b] - d[3][b];
                    }
                    for (int a = 0; a < 4; ++a) {
                        V[(a * 4 + 0) * ci + c] = rt(dt, t[a][0] - t[a][2]);
                        V[(a * 4 + 1) * ci + c] = rt(dt, t[a][1] + t[a][2]);
                        V[(a * 4 + 2) * ci + c] = rt(dt, t[a][2] - t[a][1]);
                        V[(a * 4 + 3) * ci + c] = rt(dt, t[a][1] - t[a][3]);
                    }
                }
                /* M = U V per transform position (the reference's bmm), rounded */
                for (int k = 0; k < 16; ++k)
                    for (int64_t r = 0; r < co; ++r) {
                        float acc = 0.0f;
                        for (int64_t c = 0; c < ci; ++c) acc = fmaf(U[(k * co + r) * ci + c], V[k * ci + c], acc);
                        M[k * co + r] = rt(dt, acc);
                    }
                /* output transform A^T M A + bias (winograd_transform.slang:27-47) */
                for (int64_t r = 0; r < co; ++r) {
                    const float bv = bias ? ld(dt, bias, r) : 0.0f;
                    float yv[4] = {bv, bv, bv, bv};
                    for (int k = 0; k < 16; ++k) {
                        const int a = k / 4, b = k % 4;
                        for (int q = 0; q < 4; ++q) {
                            const int i = q / 2, jj = q % 2;
                            const float wa = i == 0 ? (a == 3 ? 0.0f : 1.0f) : (a == 0 ? 0.0f : (a == 1 ? 1.0f : -1.0f));
                            const float wb = jj == 0 ? (b == 3 ? 0.0f : 1.0f) : (b == 0 ? 0.0f : (b == 1 ? 1.0f : -1.0f));
                            yv[q] = yv[q] + (wa * wb) * M[k * co + r];
                        }
                    }
                    for (int i = 0; i < 2; ++i)
                        for (int jj = 0; jj < 2; ++jj) {
                            const int64_t oh = 2 * th + i, ow = 2 * tw + jj;
                            if (oh < g->ho && ow < g->wo) st(dt, y, ((n * co + r) * g->ho + oh) * g->wo + ow, yv[i * 2 + jj]);
                        }
                }
            }
    free(U); free(V); free(M);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* 3-D convolution: the reference's implicit GEMM takes up to three spatial   */
/* dimensions (src/api/ops/conv.cpp:295-311; geometry padded to three,        */
/* conv.cpp:313-343; N-d gathers src/shaders/helpers/conv.slang:93-117).       */
/* Tensors NCDHW, weights [Cout][Cin/groups][KD][KH][KW]; k runs over          */
/* (c, kd, kh, kw) in that order, as in 2-D with the depth tap outermost.      */
/* ------------------------------------------------------------------------- */

typedef struct {
    int64_t n, cin, cout, groups;
    int64_t in[3], k[3], s[3], p[3], d[3], out[3];   /* (D, H, W) */
} conv3_geom;

static int geom3_ok(const conv3_geom* g) {
    if (g->n < 0 || g->cin <= 0 || g->cout <= 0 || g->groups <= 0) return 0;
    if (g->cin % g->groups || g->cout % g->groups) return 0;
    for (int i = 0; i < 3; ++i)
        if (g->in[i] <= 0 || g->k[i] <= 0 || g->s[i] <= 0 || g->d[i] <= 0 || g->p[i] < 0 || g->out[i] < 0) return 0;
    return 1;
}

static inline int64_t vol3(const int64_t* v) { return v[0] * v[1] * v[2]; }

/* samples [nb, ne) */
int oracle_conv3d_fwd(int dt, const conv3_geom* g, int64_t nb, int64_t ne, const void* x, const void* wt, const void* bias,
                      void* y) {
    if (!geom3_ok(g)) return -1;
    const int64_t cx = g->cin / g->groups, cy = g->cout / g->groups;
    const int64_t si = vol3(g->in), so = vol3(g->out), taps = vol3(g->k);
    for (int64_t n = nb; n < ne; ++n)
        for (int64_t oc = 0; oc < g->cout; ++oc) {
            const int64_t grp = oc / cy;
            for (int64_t od = 0; od < g->out[0]; ++od)
                for (int64_t oh = 0; oh < g->out[1]; ++oh)
                    for (int64_t ow = 0; ow < g->out[2]; ++ow) {
                        float acc = 0.0f;
                        for (int64_t c = 0; c < cx; ++c)
                            for (int64_t a = 0; a < g->k[0]; ++a)
                                for (int64_t b = 0; b < g->k[1]; ++b)
                                    for (int64_t e = 0; e < g->k[2]; ++e) {
                                        const int64_t id = od * g->s[0] - g->p[0] + a * g->d[0];
                                        const int64_t ih = oh * g->s[1] - g->p[1] + b * g->d[1];
                                        const int64_t iw = ow * g->s[2] - g->p[2] + e * g->d[2];
                                        float xv = 0.0f;
                                        if (id >= 0 && id < g->in[0] && ih >= 0 && ih < g->in[1] && iw >= 0 && iw < g->in[2])
                                            xv = ld(dt, x, (n * g->cin + grp * cx + c) * si + (id * g->in[1] + ih) * g->in[2] + iw);
                                        const float wv = ld(dt, wt, (oc * cx + c) * taps + (a * g->k[1] + b) * g->k[2] + e);
                                        acc = fmaf(wv, xv, acc);
                                    }
                        if (bias) acc = acc + ld(dt, bias, oc);
                        st(dt, y, (n * g->cout + oc) * so + (od * g->out[1] + oh) * g->out[2] + ow, acc);
                    }
        }
    return 0;
}

int oracle_conv3d_dgrad(int dt, const conv3_geom* g, int64_t nb, int64_t ne, const void* dy, const void* wt, void* dx) {
    if (!geom3_ok(g)) return -1;
    const int64_t cx = g->cin / g->groups, cy = g->cout / g->groups;
    const int64_t si = vol3(g->in), so = vol3(g->out), taps = vol3(g->k);
    for (int64_t n = nb; n < ne; ++n)
        for (int64_t ic = 0; ic < g->cin; ++ic) {
            const int64_t grp = ic / cx, c = ic % cx;
            for (int64_t id = 0; id < g->in[0]; ++id)
                for (int64_t ih = 0; ih < g->in[1]; ++ih)
                    for (int64_t iw = 0; iw < g->in[2]; ++iw) {
                        float acc = 0.0f;
                        for (int64_t m = 0; m < cy; ++m)
                            for (int64_t a = 0; a < g->k[0]; ++a)
                                for (int64_t b = 0; b < g->k[1]; ++b)
                                    for (int64_t e = 0; e < g->k[2]; ++e) {
                                        const int64_t td = id + g->p[0] - a * g->d[0];
                                        const int64_t th = ih + g->p[1] - b * g->d[1];
                                        const int64_t tw = iw + g->p[2] - e * g->d[2];
                                        if (td < 0 || th < 0 || tw < 0 || td % g->s[0] || th % g->s[1] || tw % g->s[2]) continue;
                                        const int64_t od = td / g->s[0], oh = th / g->s[1], ow = tw / g->s[2];
                                        if (od >= g->out[0] || oh >= g->out[1] || ow >= g->out[2]) continue;
                                        const int64_t oc = grp * cy + m;
                                        acc = fmaf(ld(dt, wt, (oc * cx + c) * taps + (a * g->k[1] + b) * g->k[2] + e),
                                                   ld(dt, dy, (n * g->cout + oc) * so + (od * g->out[1] + oh) * g->out[2] + ow), acc);
                                    }
                        st(dt, dx, (n * g->cin + ic) * si + (id * g->in[1] + ih) * g->in[2] + iw, acc);
                    }
        }
    return 0;
}

/* output channels [ob, oe) */
int oracle_conv3d_wgrad(int dt, const conv3_geom* g, int64_t ob, int64_t oe, const void* x, const void* dy, void* dw,
                        int acc64) {
    if (!geom3_ok(g)) return -1;
    const int64_t cx = g->cin / g->groups, cy = g->cout / g->groups;
    const int64_t si = vol3(g->in), so = vol3(g->out), taps = vol3(g->k);
    for (int64_t oc = ob; oc < oe; ++oc) {
        const int64_t grp = oc / cy;
        for (int64_t c = 0; c < cx; ++c)
            for (int64_t a = 0; a < g->k[0]; ++a)
                for (int64_t b = 0; b < g->k[1]; ++b)
                    for (int64_t e = 0; e < g->k[2]; ++e) {
                        float acc = 0.0f;
                        double acc_d = 0.0;
                        for (int64_t n = 0; n < g->n; ++n)
                            for (int64_t od = 0; od < g->out[0]; ++od)
                                for (int64_t oh = 0; oh < g->out[1]; ++oh)
                                    for (int64_t ow = 0; ow < g->out[2]; ++ow) {
                                        const int64_t id = od * g->s[0] - g->p[0] + a * g->d[0];
                                        const int64_t ih = oh * g->s[1] - g->p[1] + b * g->d[1];
                                        const int64_t iw = ow * g->s[2] - g->p[2] + e * g->d[2];
                                        if (id < 0 || id >= g->in[0] || ih < 0 || ih >= g->in[1] || iw < 0 || iw >= g->in[2])
                                            continue;
                                        const float yv = ld(dt, dy, (n * g->cout + oc) * so + (od * g->out[1] + oh) * g->out[2] + ow);
                                        const float xv = ld(dt, x, (n * g->cin + grp * cx + c) * si + (id * g->in[1] + ih) * g->in[2] + iw);
                                        if (acc64) acc_d += (double)yv * (double)xv;
                                        else acc = fmaf(yv, xv, acc);
                                    }
                        st(dt, dw, (oc * cx + c) * taps + (a * g->k[1] + b) * g->k[2] + e, acc64 ? (float)acc_d : acc);
                    }
    }
    return 0;
}
