/*
 * oracle.c -- double-precision CPU restatement of lanternl's pure-Lua path.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).  Not part of the product.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ====================================================================== */
/* GEMM family                                                             */
/* ====================================================================== */

/* matrix.lua:514-539 (local function mm) */
void or_mm(const double* a, const double* b, double* r, int m, int k, int n, int acc)
{
    for (int i = 0; i < m; ++i) {
        const double* ar = a + (long)i * k;
        double* rr = r + (long)i * n;
        int p0 = 0;
        if (!acc) {
            const double av = ar[0];
            if (av != 0) {
                for (int j = 0; j < n; ++j) rr[j] = av * b[j];
            } else {
                for (int j = 0; j < n; ++j) rr[j] = 0;
            }
            p0 = 1;
        }
        for (int p = p0; p < k; ++p) {
            const double av = ar[p];
            if (av != 0) {
                const double* br = b + (long)p * n;
                for (int j = 0; j < n; ++j) rr[j] = rr[j] + av * br[j];
            }
        }
    }
}

/* matrix.lua:597-625 */
void or_matmul_nt(const double* a, const double* b, double* r, int m, int k, int n, int acc)
{
    for (int i = 0; i < m; ++i) {
        const double* ar = a + (long)i * k;
        double* rr = r + (long)i * n;
        for (int j = 0; j < n; ++j) {
            const double* br = b + (long)j * k;
            double s = 0;
            for (int p = 0; p < k; ++p) s = s + ar[p] * br[p];
            if (acc) rr[j] = rr[j] + s; else rr[j] = s;
        }
    }
}

/* matrix.lua:627-660 */
void or_matmul_tn(const double* a, const double* b, double* r, int m, int k, int n, int acc)
{
    if (!acc) for (long i = 0; i < (long)k * n; ++i) r[i] = 0;
    if (m == 0 || k == 0 || n == 0) return;
    for (int i = 0; i < m; ++i) {
        const double* ar = a + (long)i * k;
        const double* br = b + (long)i * n;
        for (int p = 0; p < k; ++p) {
            const double av = ar[p];
            if (av != 0) {
                double* rr = r + (long)p * n;
                for (int j = 0; j < n; ++j) rr[j] = rr[j] + av * br[j];
            }
        }
    }
}

/* ====================================================================== */
/* RMSNorm: tensor2.lua:609-666                                            */
/* ====================================================================== */

void or_rmsnorm_fwd(const double* x, const double* w, double* out, double* inv,
                    int rows, int cols, double eps)
{
    for (int i = 0; i < rows; ++i) {
        const double* xr = x + (long)i * cols;
        double* orow = out + (long)i * cols;
        double ss = 0;
        for (int j = 0; j < cols; ++j) { const double v = xr[j]; ss = ss + v * v; }
        const double r = 1 / sqrt(ss / cols + eps);
        if (inv) inv[i] = r;
        for (int j = 0; j < cols; ++j) orow[j] = xr[j] * r * w[j];
    }
}

void or_rmsnorm_bwd(const double* x, const double* w, const double* inv, const double* g,
                    double* xg, double* wg, int rows, int cols)
{
    for (int i = 0; i < rows; ++i) {
        const long base = (long)i * cols;
        const double r = inv[i];
        double dot = 0;
        for (int j = 0; j < cols; ++j) dot = dot + g[base + j] * w[j] * x[base + j];
        const double coef = dot * r * r * r / cols;
        for (int j = 0; j < cols; ++j) {
            const double xv = x[base + j];
            const double gv = g[base + j];
            if (xg) xg[base + j] = xg[base + j] + gv * w[j] * r - xv * coef;
            if (wg) wg[j] = wg[j] + gv * xv * r;
        }
    }
}

/* ====================================================================== */
/* row softmax: tensor2.lua:332-408                                        */
/* ====================================================================== */

static int softmax_limit(int i, int cols, int causal, int offset)
{
    if (!causal) return cols;
    int lim = (i + 1) + offset;          /* Lua: lim = i + offset, i 1-based */
    if (lim > cols) lim = cols;
    if (lim < 1) lim = 1;
    return lim;
}

void or_softmax_fwd(const double* x, double* y, int rows, int cols, int causal, int offset)
{
    for (int i = 0; i < rows; ++i) {
        const double* xr = x + (long)i * cols;
        double* yr = y + (long)i * cols;
        const int n = softmax_limit(i, cols, causal, offset);
        double mx = -HUGE_VAL;
        for (int j = 0; j < n; ++j) if (xr[j] > mx) mx = xr[j];
        if (mx == -HUGE_VAL || mx != mx) mx = 0;
        double sum = 0;
        for (int j = 0; j < n; ++j) { const double e = exp(xr[j] - mx); yr[j] = e; sum = sum + e; }
        if (!(sum > 0)) sum = 1;
        const double inv = 1 / sum;
        for (int j = 0; j < n; ++j) yr[j] = yr[j] * inv;
        for (int j = n; j < cols; ++j) yr[j] = 0;
    }
}

void or_softmax_bwd(const double* y, const double* g, double* xg, int rows, int cols,
                    int causal, int offset)
{
    for (int i = 0; i < rows; ++i) {
        const long base = (long)i * cols;
        const int n = softmax_limit(i, cols, causal, offset);
        double dot = 0;
        for (int j = 0; j < n; ++j) dot = dot + g[base + j] * y[base + j];
        for (int j = 0; j < n; ++j) {
            const double yv = y[base + j];
            xg[base + j] = xg[base + j] + yv * (g[base + j] - dot);
        }
    }
}

/* ====================================================================== */
/* SiLU / SwiGLU                                                           */
/* ====================================================================== */

/* tensor2.lua:272-291: sigmoid evaluated by sign for stability */
static double sigmoid_by_sign(double v)
{
    if (v >= 0) return 1 / (1 + exp(-v));
    const double z = exp(v);
    return z / (1 + z);
}

void or_silu_fwd(const double* x, double* y, double* sig, long n)
{
    for (long k = 0; k < n; ++k) {
        const double v = x[k];
        const double s = sigmoid_by_sign(v);
        if (sig) sig[k] = s;
        y[k] = v * s;
    }
}

/* tensor2.lua:293-303 */
void or_silu_bwd(const double* x, const double* sig, const double* g, double* xg, long n)
{
    for (long k = 0; k < n; ++k) {
        const double s = sig[k];
        xg[k] = xg[k] + s * (1 + x[k] * (1 - s)) * g[k];
    }
}

/* transformer.lua:246-248: g = silu(h2 W1); u = h2 W3; h = g (.) u */
void or_swiglu_fwd(const double* gate, const double* up, double* h, long n)
{
    for (long k = 0; k < n; ++k) {
        const double v = gate[k];
        const double sv = v * sigmoid_by_sign(v);
        h[k] = sv * up[k];                   /* matrix.hadamard (matrix.lua:461) */
    }
}

/* BACKWARD.mul (tensor2.lua:172-183) feeding BACKWARD.silu (:293-303) */
void or_swiglu_bwd(const double* gate, const double* up, const double* dh,
                   double* dgate, double* dup, long n)
{
    for (long k = 0; k < n; ++k) {
        const double v = gate[k];
        const double s = sigmoid_by_sign(v);
        const double sv = v * s;
        const double dsv = up[k] * dh[k];    /* grad of silu output */
        if (dup) dup[k] = dup[k] + sv * dh[k];
        if (dgate) dgate[k] = dgate[k] + s * (1 + v * (1 - s)) * dsv;
    }
}

/* ====================================================================== */
/* RoPE                                                                    */
/* ====================================================================== */

/* transformer.lua:30-48 */
void or_rope_angles(double base, int hd, int maxpos, double* cosv, double* sinv)
{
    const int npairs = hd / 2;
    double* inv = (double*)malloc(sizeof(double) * (npairs > 0 ? npairs : 1));
    for (int k = 0; k < npairs; ++k) inv[k] = 1 / pow(base, (double)(2 * k) / hd);
    for (int p = 0; p <= maxpos; ++p)
        for (int k = 0; k < npairs; ++k) {
            const double ang = p * inv[k];
            cosv[(long)p * npairs + k] = cos(ang);
            sinv[(long)p * npairs + k] = sin(ang);
        }
    free(inv);
}

/* tensor2.lua:410-446 */
void or_rope_fwd(const double* x, double* y, int rows, int cols,
                 const double* cosr, const double* sinr, int npairs)
{
    for (int i = 0; i < rows; ++i) {
        const long base = (long)i * cols;
        const double* c = cosr + (long)i * npairs;
        const double* s = sinr + (long)i * npairs;
        for (int k = 0; k < npairs; ++k) {
            const long p = base + 2 * k;
            const double x0 = x[p], x1 = x[p + 1];
            y[p] = x0 * c[k] - x1 * s[k];
            y[p + 1] = x0 * s[k] + x1 * c[k];
        }
        for (int j = 2 * npairs; j < cols; ++j) y[base + j] = x[base + j];
    }
}

/* tensor2.lua:451-473 */
void or_rope_bwd(const double* g, double* xg, int rows, int cols,
                 const double* cosr, const double* sinr, int npairs)
{
    for (int i = 0; i < rows; ++i) {
        const long base = (long)i * cols;
        const double* c = cosr + (long)i * npairs;
        const double* s = sinr + (long)i * npairs;
        for (int k = 0; k < npairs; ++k) {
            const long p = base + 2 * k;
            const double g0 = g[p], g1 = g[p + 1];
            xg[p] = xg[p] + g0 * c[k] + g1 * s[k];
            xg[p + 1] = xg[p + 1] - g0 * s[k] + g1 * c[k];
        }
        for (int j = 2 * npairs; j < cols; ++j) xg[base + j] = xg[base + j] + g[base + j];
    }
}

/* luaTL_rope contract (cuda/luaTL_train.cu:719-767), restated in double */
void or_rope_heads(double* x, const int* pos_ids, int rows, int heads, int hd,
                   int row_stride, int pos_offset, double theta, int interleaved, int inverse)
{
    const int pairs = hd / 2;
    for (int r = 0; r < rows; ++r) {
        const int pos = pos_ids ? pos_ids[r] : r + pos_offset;
        for (int h = 0; h < heads; ++h) {
            const long base = (long)r * row_stride + (long)h * hd;
            for (int p = 0; p < pairs; ++p) {
                const double freq = pow(theta, -2.0 * p / hd);
                const double ang = pos * freq;
                const double c = cos(ang);
                const double s = inverse ? -sin(ang) : sin(ang);
                const long i0 = interleaved ? base + 2 * p : base + p;
                const long i1 = interleaved ? base + 2 * p + 1 : base + p + pairs;
                const double x0 = x[i0], x1 = x[i1];
                x[i0] = x0 * c - x1 * s;
                x[i1] = x1 * c + x0 * s;
            }
        }
    }
}

/* ====================================================================== */
/* cross-entropy                                                           */
/* ====================================================================== */

/* tensor2.lua:809-857 */
double or_cross_entropy(const double* logits, const int* tgt, int rows, int cols,
                        int has_ignore, int ignore_index, double* sm, int* count)
{
    double total = 0;
    int counted = 0;
    for (int i = 0; i < rows; ++i) {
        const double* x = logits + (long)i * cols;
        double* s = sm + (long)i * cols;
        const int t = tgt[i];
        if (has_ignore && t == ignore_index) {
            for (int j = 0; j < cols; ++j) s[j] = 0;
            continue;
        }
        double mx = -HUGE_VAL;
        for (int j = 0; j < cols; ++j) if (x[j] > mx) mx = x[j];
        if (mx == -HUGE_VAL || mx != mx) mx = 0;
        double sum = 0;
        for (int j = 0; j < cols; ++j) { const double e = exp(x[j] - mx); s[j] = e; sum = sum + e; }
        const double inv = 1 / sum;
        for (int j = 0; j < cols; ++j) s[j] = s[j] * inv;
        total = total + ((mx + log(sum)) - x[t]);
        counted = counted + 1;
    }
    if (counted == 0) counted = 1;
    if (count) *count = counted;
    return total / counted;
}

/* tensor2.lua:862-882 */
void or_cross_entropy_bwd(const double* sm, const int* tgt, int rows, int cols,
                          int has_ignore, int ignore_index, double g, int count, double* lg)
{
    const double gv = g / count;
    for (int i = 0; i < rows; ++i) {
        const int t = tgt[i];
        if (has_ignore && t == ignore_index) continue;
        const long base = (long)i * cols;
        for (int j = 0; j < cols; ++j) {
            double gval = sm[base + j];
            if (j == t) gval = gval - 1;
            lg[base + j] = lg[base + j] + gval * gv;
        }
    }
}

/* luaTL_cross_entropy contract (cuda/luaTL_train.cu:837-891) in double */
void or_ce_fused(const double* logits, const int* tgt, double* losses, double* dlogits,
                 int rows, int vocab, int ignore_index, double gscale)
{
    for (int r = 0; r < rows; ++r) {
        const double* x = logits + (long)r * vocab;
        double* d = dlogits ? dlogits + (long)r * vocab : NULL;
        const int t = tgt[r];
        if (t < 0 || t >= vocab || t == ignore_index) {
            if (losses) losses[r] = 0;
            if (d) for (int j = 0; j < vocab; ++j) d[j] = 0;
            continue;
        }
        double mx = -HUGE_VAL;
        for (int j = 0; j < vocab; ++j) if (x[j] > mx) mx = x[j];
        double sum = 0;
        for (int j = 0; j < vocab; ++j) sum += exp(x[j] - mx);
        const double lse = log(sum) + mx;
        if (losses) losses[r] = lse - x[t];
        if (d) {
            for (int j = 0; j < vocab; ++j) {
                double p = exp(x[j] - mx) / sum;
                if (j == t) p -= 1;
                d[j] = gscale * p;
            }
        }
    }
}

/* ====================================================================== */
/* argmax / embedding                                                      */
/* ====================================================================== */

/* lmtrain.lua:1200-1209 */
void or_argmax_rows(const double* x, int* out, int rows, int cols)
{
    for (int r = 0; r < rows; ++r) {
        const double* xr = x + (long)r * cols;
        int best = 0;
        double bv = -HUGE_VAL;
        for (int c = 0; c < cols; ++c) {
            const double v = xr[c];
            if (v > bv) { bv = v; best = c; }
        }
        out[r] = best;
    }
}

/* tensor2.lua:572-590 */
void or_embed_fwd(const double* w, const int* ids, double* out, int n, int dim)
{
    for (int i = 0; i < n; ++i) {
        const double* src = w + (long)ids[i] * dim;
        double* dst = out + (long)i * dim;
        for (int j = 0; j < dim; ++j) dst[j] = src[j];
    }
}

/* tensor2.lua:592-607 (scale generalises luaTL_embed_bwd's argument) */
void or_embed_bwd(const double* g, const int* ids, double* wg, int n, int dim, double scale)
{
    for (int i = 0; i < n; ++i) {
        double* dst = wg + (long)ids[i] * dim;
        const double* src = g + (long)i * dim;
        for (int j = 0; j < dim; ++j) dst[j] = dst[j] + scale * src[j];
    }
}

/* ====================================================================== */
/* optimizer                                                               */
/* ====================================================================== */

double or_grad_norm(const double* g, long n)
{
    double s = 0;
    for (long k = 0; k < n; ++k) { const double v = g[k]; s = s + v * v; }
    return sqrt(s);
}

void or_scale(double* g, long n, double f)
{
    for (long k = 0; k < n; ++k) g[k] = g[k] * f;
}

/* optim2.lua:72-99 */
void or_sgd_step(double* p, const double* g, double* v, long n,
                 double lr, double momentum, double wd, int nesterov)
{
    for (long k = 0; k < n; ++k) {
        double gk = g[k];
        if (wd != 0) gk = gk + wd * p[k];
        if (momentum > 0) {
            const double vk = momentum * v[k] + gk;
            v[k] = vk;
            if (nesterov) p[k] = p[k] - lr * (gk + momentum * vk);
            else p[k] = p[k] - lr * vk;
        } else {
            p[k] = p[k] - lr * gk;
        }
    }
}

/* optim2.lua:116-147 (AdamW.step after self.t has been advanced to t):
 * m = b1 m + (1-b1) g, v = b2 v + (1-b2) g^2, p -= lr*wd*p (decoupled),
 * p -= (lr / (1 - b1^t)) * m / (sqrt(v / (1 - b2^t)) + eps). */
void or_adamw_step(double* p, const double* g, double* m, double* v, long n,
                   double lr, double b1, double b2, double eps, double wd, int t)
{
    const double bc1 = 1 - pow(b1, t);
    const double bc2 = 1 - pow(b2, t);
    const double step_size = lr / bc1;
    const double inv_bc2 = 1 / bc2;
    const double decay = wd != 0 ? lr * wd : 0;
    for (long k = 0; k < n; ++k) {
        const double gk = g[k];
        const double mk = b1 * m[k] + (1 - b1) * gk;
        const double vk = b2 * v[k] + (1 - b2) * gk * gk;
        m[k] = mk;
        v[k] = vk;
        const double denom = sqrt(vk * inv_bc2) + eps;
        double pk = p[k];
        if (decay != 0) pk = pk - decay * pk;
        p[k] = pk - step_size * mk / denom;
    }
}

/* ====================================================================== */
/* Transformer window forward/backward and the LMTrain SGD step            */
/* ====================================================================== */

enum { P_LN1, P_WQ, P_WK, P_WV, P_WO, P_LN2, P_W1, P_W3, P_W2, P_PER_LAYER };

int or_lm_param_offsets(const or_lm_cfg* c, long* offs, int* rows, int* cols)
{
    const int D = c->dim, F = c->ffn, V = c->vocab;
    int idx = 0;
    long off = 0;
#define ADD(R, C) do {                     \
        if (offs) offs[idx] = off;             \
        if (rows) rows[idx] = (R);             \
        if (cols) cols[idx] = (C);             \
        off += (long)(R) * (C);                \
        ++idx;                                 \
    } while (0)
    ADD(V, D);
    for (int l = 0; l < c->layers; ++l) {
        ADD(1, D); ADD(D, D); ADD(D, D); ADD(D, D); ADD(D, D);
        ADD(1, D); ADD(D, F); ADD(D, F); ADD(F, D);
    }
    ADD(1, D);
#undef ADD
    return idx;
}

long or_lm_num_params(const or_lm_cfg* c)
{
    const long D = c->dim, F = c->ffn, V = c->vocab;
    return V * D + c->layers * (2 * D + 4 * D * D + 3 * D * F) + D;
}

static double* zalloc(long n) { return (double*)calloc((size_t)(n > 0 ? n : 1), sizeof(double)); }

/* Per-layer saved activations for the backward pass */
typedef struct {
    double *x_in, *h, *inv1, *q, *k, *v;
    double *qr, *kr;         /* per head roped q/k: [H][T][hd] */
    double *pr;              /* per head softmax probs: [H][T][T] */
    double *ctx, *x_mid, *h2, *inv2, *z1, *sig, *gs, *u, *a;
} layer_acts;

/* copies columns [c0, c0+w) of a (rows x cols) into out (rows x w): slice_cols (tensor2.lua:475-496) */
static void slice_cols(const double* a, double* out, int rows, int cols, int c0, int w)
{
    for (int i = 0; i < rows; ++i)
        for (int j = 0; j < w; ++j) out[(long)i * w + j] = a[(long)i * cols + c0 + j];
}

double or_lm_window(const or_lm_cfg* c, const double* params, const int* ids, const int* tgt,
                    int T, double* grads, double* logits_out, int* correct)
{
    const int V = c->vocab, D = c->dim, L = c->layers, H = c->heads, F = c->ffn;
    const int hd = D / H, npairs = hd / 2;
    const double scale = 1 / sqrt((double)hd);
    const int ntens = 2 + P_PER_LAYER * L;
    long* off = (long*)malloc(sizeof(long) * ntens);
    or_lm_param_offsets(c, off, NULL, NULL);
    const double* emb = params + off[0];
    const double* lnf = params + off[ntens - 1];
    double* gemb = grads + off[0];
    double* glnf = grads + off[ntens - 1];

    /* RoPE tables for positions 0..T-1 (Transformer:rope_rows(T, 0), transformer.lua:166-175) */
    double* cosr = zalloc((long)T * npairs);
    double* sinr = zalloc((long)T * npairs);
    or_rope_angles(c->rope_base, hd, T - 1, cosr, sinr);

    /* ---------------- forward (transformer.lua:228-257) ---------------- */
    layer_acts* A = (layer_acts*)calloc((size_t)L, sizeof(layer_acts));
    double* x = zalloc((long)T * D);
    or_embed_fwd(emb, ids, x, T, D);
    double* qh = zalloc((long)T * hd);
    double* kh = zalloc((long)T * hd);
    double* vh = zalloc((long)T * hd);
    double* sc = zalloc((long)T * T);
    double* oh = zalloc((long)T * hd);
    double* o = zalloc((long)T * D);
    double* f = zalloc((long)T * D);
    for (int l = 0; l < L; ++l) {
        const double* P = params + off[1 + P_PER_LAYER * l];
        const double* ln1 = params + off[1 + P_PER_LAYER * l + P_LN1];
        const double* wq = params + off[1 + P_PER_LAYER * l + P_WQ];
        const double* wk = params + off[1 + P_PER_LAYER * l + P_WK];
        const double* wv = params + off[1 + P_PER_LAYER * l + P_WV];
        const double* wo = params + off[1 + P_PER_LAYER * l + P_WO];
        const double* ln2 = params + off[1 + P_PER_LAYER * l + P_LN2];
        const double* w1 = params + off[1 + P_PER_LAYER * l + P_W1];
        const double* w3 = params + off[1 + P_PER_LAYER * l + P_W3];
        const double* w2 = params + off[1 + P_PER_LAYER * l + P_W2];
        (void)P;
        layer_acts* a = &A[l];
        a->x_in = x;
        a->h = zalloc((long)T * D); a->inv1 = zalloc(T);
        or_rmsnorm_fwd(x, ln1, a->h, a->inv1, T, D, c->eps);
        /* _attention (transformer.lua:196-226) */
        a->q = zalloc((long)T * D); a->k = zalloc((long)T * D); a->v = zalloc((long)T * D);
        or_mm(a->h, wq, a->q, T, D, D, 0);
        or_mm(a->h, wk, a->k, T, D, D, 0);
        or_mm(a->h, wv, a->v, T, D, D, 0);
        a->qr = zalloc((long)H * T * hd); a->kr = zalloc((long)H * T * hd);
        a->pr = zalloc((long)H * T * T);
        a->ctx = zalloc((long)T * D);
        for (int hh = 0; hh < H; ++hh) {
            double* qrh = a->qr + (long)hh * T * hd;
            double* krh = a->kr + (long)hh * T * hd;
            double* prh = a->pr + (long)hh * T * T;
            slice_cols(a->q, qh, T, D, hh * hd, hd);
            slice_cols(a->k, kh, T, D, hh * hd, hd);
            slice_cols(a->v, vh, T, D, hh * hd, hd);
            or_rope_fwd(qh, qrh, T, hd, cosr, sinr, npairs);
            or_rope_fwd(kh, krh, T, hd, cosr, sinr, npairs);
            or_matmul_nt(qrh, krh, sc, T, hd, T, 0);
            for (long e = 0; e < (long)T * T; ++e) sc[e] = sc[e] * scale;   /* Tensor.scale */
            or_softmax_fwd(sc, prh, T, T, c->causal, 0);
            or_mm(prh, vh, oh, T, T, hd, 0);
            for (int i = 0; i < T; ++i)                                    /* concat_cols */
                for (int j = 0; j < hd; ++j) a->ctx[(long)i * D + hh * hd + j] = oh[(long)i * hd + j];
        }
        or_mm(a->ctx, wo, o, T, D, D, 0);
        a->x_mid = zalloc((long)T * D);
        for (long e = 0; e < (long)T * D; ++e) a->x_mid[e] = x[e] + o[e];
        a->h2 = zalloc((long)T * D); a->inv2 = zalloc(T);
        or_rmsnorm_fwd(a->x_mid, ln2, a->h2, a->inv2, T, D, c->eps);
        a->z1 = zalloc((long)T * F); a->sig = zalloc((long)T * F); a->gs = zalloc((long)T * F);
        a->u = zalloc((long)T * F); a->a = zalloc((long)T * F);
        or_mm(a->h2, w1, a->z1, T, D, F, 0);
        or_silu_fwd(a->z1, a->gs, a->sig, (long)T * F);
        or_mm(a->h2, w3, a->u, T, D, F, 0);
        for (long e = 0; e < (long)T * F; ++e) a->a[e] = a->gs[e] * a->u[e];
        or_mm(a->a, w2, f, T, F, D, 0);
        double* xn = zalloc((long)T * D);
        for (long e = 0; e < (long)T * D; ++e) xn[e] = a->x_mid[e] + f[e];
        x = xn;
    }
    double* xf = zalloc((long)T * D);
    double* invf = zalloc(T);
    or_rmsnorm_fwd(x, lnf, xf, invf, T, D, c->eps);
    double* lg = zalloc((long)T * V);
    or_matmul_nt(xf, emb, lg, T, D, V, 0);                 /* tied head */
    if (logits_out) memcpy(logits_out, lg, sizeof(double) * (size_t)T * V);
    if (correct) {
        int* am = (int*)malloc(sizeof(int) * T);
        or_argmax_rows(lg, am, T, V);
        for (int i = 0; i < T; ++i) if (am[i] == tgt[i]) ++*correct;
        free(am);
    }
    double* sm = zalloc((long)T * V);
    int count = 1;
    const double loss = or_cross_entropy(lg, tgt, T, V, 0, 0, sm, &count);

    /* ---------------- backward (seed 1) ---------------- */
    double* dlg = zalloc((long)T * V);
    or_cross_entropy_bwd(sm, tgt, T, V, 0, 0, 1.0, count, dlg);
    double* dxf = zalloc((long)T * D);
    or_mm(dlg, emb, dxf, T, V, D, 1);                      /* BACKWARD.matmul_nt */
    or_matmul_tn(dlg, xf, gemb, T, V, D, 1);
    double* dx = zalloc((long)T * D);
    or_rmsnorm_bwd(x, lnf, invf, dxf, dx, glnf, T, D);

    double* da = zalloc((long)T * F);
    double* dz1 = zalloc((long)T * F);
    double* dgs = zalloc((long)T * F);
    double* du = zalloc((long)T * F);
    double* dh2 = zalloc((long)T * D);
    double* dctx = zalloc((long)T * D);
    double* dq = zalloc((long)T * D);
    double* dk = zalloc((long)T * D);
    double* dv = zalloc((long)T * D);
    double* dh = zalloc((long)T * D);
    double* doh = zalloc((long)T * hd);
    double* dpr = zalloc((long)T * T);
    double* dsc = zalloc((long)T * T);
    double* dqr = zalloc((long)T * hd);
    double* dkr = zalloc((long)T * hd);
    double* dvh = zalloc((long)T * hd);
    double* dqh = zalloc((long)T * hd);
    double* dkh = zalloc((long)T * hd);
    for (int l = L - 1; l >= 0; --l) {
        layer_acts* a = &A[l];
        const int b0 = 1 + P_PER_LAYER * l;
        const double* ln1 = params + off[b0 + P_LN1];
        const double* wq = params + off[b0 + P_WQ];
        const double* wk = params + off[b0 + P_WK];
        const double* wv = params + off[b0 + P_WV];
        const double* wo = params + off[b0 + P_WO];
        const double* ln2 = params + off[b0 + P_LN2];
        const double* w1 = params + off[b0 + P_W1];
        const double* w3 = params + off[b0 + P_W3];
        const double* w2 = params + off[b0 + P_W2];
        /* x_out = x_mid + f: dx flows to both; f = a . W2 */
        memset(da, 0, sizeof(double) * (size_t)T * F);
        or_matmul_nt(dx, w2, da, T, D, F, 1);
        or_matmul_tn(a->a, dx, grads + off[b0 + P_W2], T, F, D, 1);
        memset(dgs, 0, sizeof(double) * (size_t)T * F);
        memset(du, 0, sizeof(double) * (size_t)T * F);
        for (long e = 0; e < (long)T * F; ++e) {                /* BACKWARD.mul */
            dgs[e] = dgs[e] + a->u[e] * da[e];
            du[e] = du[e] + a->gs[e] * da[e];
        }
        memset(dh2, 0, sizeof(double) * (size_t)T * D);
        or_matmul_nt(du, w3, dh2, T, F, D, 1);                  /* u = h2 . W3 */
        or_matmul_tn(a->h2, du, grads + off[b0 + P_W3], T, D, F, 1);
        memset(dz1, 0, sizeof(double) * (size_t)T * F);
        or_silu_bwd(a->z1, a->sig, dgs, dz1, (long)T * F);
        or_matmul_nt(dz1, w1, dh2, T, F, D, 1);                 /* z1 = h2 . W1 */
        or_matmul_tn(a->h2, dz1, grads + off[b0 + P_W1], T, D, F, 1);
        /* h2 = rmsnorm(x_mid): dx (residual) += rmsnorm bwd */
        or_rmsnorm_bwd(a->x_mid, ln2, a->inv2, dh2, dx, grads + off[b0 + P_LN2], T, D);
        /* x_mid = x_in + o: do = dx */
        memset(dctx, 0, sizeof(double) * (size_t)T * D);
        or_matmul_nt(dx, wo, dctx, T, D, D, 1);
        or_matmul_tn(a->ctx, dx, grads + off[b0 + P_WO], T, D, D, 1);
        memset(dq, 0, sizeof(double) * (size_t)T * D);
        memset(dk, 0, sizeof(double) * (size_t)T * D);
        memset(dv, 0, sizeof(double) * (size_t)T * D);
        for (int hh = H - 1; hh >= 0; --hh) {
            const double* qrh = a->qr + (long)hh * T * hd;
            const double* krh = a->kr + (long)hh * T * hd;
            const double* prh = a->pr + (long)hh * T * T;
            slice_cols(dctx, doh, T, D, hh * hd, hd);
            slice_cols(a->v, vh, T, D, hh * hd, hd);
            memset(dpr, 0, sizeof(double) * (size_t)T * T);
            memset(dvh, 0, sizeof(double) * (size_t)T * hd);
            or_matmul_nt(doh, vh, dpr, T, hd, T, 1);            /* oh = pr . vh */
            or_matmul_tn(prh, doh, dvh, T, T, hd, 1);
            memset(dsc, 0, sizeof(double) * (size_t)T * T);
            or_softmax_bwd(prh, dpr, dsc, T, T, c->causal, 0);  /* into d(scaled scores) */
            for (long e = 0; e < (long)T * T; ++e) dsc[e] = dsc[e] * scale;  /* BACKWARD.scale */
            memset(dqr, 0, sizeof(double) * (size_t)T * hd);
            memset(dkr, 0, sizeof(double) * (size_t)T * hd);
            or_mm(dsc, krh, dqr, T, T, hd, 1);                  /* sc = qr . kr^T */
            or_matmul_tn(dsc, qrh, dkr, T, T, hd, 1);
            memset(dqh, 0, sizeof(double) * (size_t)T * hd);
            memset(dkh, 0, sizeof(double) * (size_t)T * hd);
            or_rope_bwd(dqr, dqh, T, hd, cosr, sinr, npairs);
            or_rope_bwd(dkr, dkh, T, hd, cosr, sinr, npairs);
            for (int i = 0; i < T; ++i)                         /* BACKWARD.slice_cols */
                for (int j = 0; j < hd; ++j) {
                    dq[(long)i * D + hh * hd + j] += dqh[(long)i * hd + j];
                    dk[(long)i * D + hh * hd + j] += dkh[(long)i * hd + j];
                    dv[(long)i * D + hh * hd + j] += dvh[(long)i * hd + j];
                }
        }
        memset(dh, 0, sizeof(double) * (size_t)T * D);
        or_matmul_nt(dq, wq, dh, T, D, D, 1);
        or_matmul_tn(a->h, dq, grads + off[b0 + P_WQ], T, D, D, 1);
        or_matmul_nt(dk, wk, dh, T, D, D, 1);
        or_matmul_tn(a->h, dk, grads + off[b0 + P_WK], T, D, D, 1);
        or_matmul_nt(dv, wv, dh, T, D, D, 1);
        or_matmul_tn(a->h, dv, grads + off[b0 + P_WV], T, D, D, 1);
        or_rmsnorm_bwd(a->x_in, ln1, a->inv1, dh, dx, grads + off[b0 + P_LN1], T, D);
    }
    or_embed_bwd(dx, ids, gemb, T, D, 1.0);

    /* ---------------- cleanup ---------------- */
    /* A[0].x_in is the embedding output, A[l].x_in the residual stream after
     * layer l-1, and x the stream after the last layer: all distinct buffers. */
    for (int l = 0; l < L; ++l) {
        layer_acts* a = &A[l];
        free(a->x_in);
        free(a->h); free(a->inv1); free(a->q); free(a->k); free(a->v);
        free(a->qr); free(a->kr); free(a->pr); free(a->ctx); free(a->x_mid);
        free(a->h2); free(a->inv2); free(a->z1); free(a->sig); free(a->gs); free(a->u); free(a->a);
    }
    free(x);
    free(A);
    free(qh); free(kh); free(vh); free(sc); free(oh); free(o); free(f);
    free(xf); free(invf); free(lg); free(sm); free(dlg); free(dxf); free(dx);
    free(da); free(dz1); free(dgs); free(du); free(dh2); free(dctx); free(dq); free(dk); free(dv);
    free(dh); free(doh); free(dpr); free(dsc); free(dqr); free(dkr); free(dvh); free(dqh); free(dkh);
    free(cosr); free(sinr); free(off);
    return loss;
}

/* the batch part of lmtrain.lua:1183-1222 shared by both optimizers: zero
 * grads, every window, scale 1/B, norm, finite check, clip.  Returns 1 when
 * the optimizer step is to be applied. */
/* lmtrain.lua:1183-1226: windows b < nwin, window b holding lens[b] tokens
 * (lens NULL: T) at ids/tgt + b*T (build_windows' short last window,
 * lmtrain.lua:535-558); each window's loss is its own mean
 * (tensor2.lua:845-857); gradients summed, then scaled by 1/nwin when nwin > 1
 * (the short last batch runs n_in_batch windows). */
static int lm_batch_grads(const or_lm_cfg* c, const double* params, const int* ids, const int* tgt,
                          int nwin, int T, const int* lens, double clip_norm, double* losses, double* gnorm,
                          int* correct, double* grads)
{
    const long n = or_lm_num_params(c);
    for (long e = 0; e < n; ++e) grads[e] = 0;                       /* opt.zero_grad() */
    int corr = 0;
    for (int b = 0; b < nwin; ++b) {
        const int len = lens ? lens[b] : T;
        const double l = or_lm_window(c, params, ids + (long)b * T, tgt + (long)b * T, len,
                                      grads, NULL, &corr);
        if (losses) losses[b] = l;
    }
    if (correct) *correct = corr;
    if (nwin > 1) or_scale(grads, n, 1.0 / nwin);                    /* scale_grads */
    const double norm = or_grad_norm(grads, n);
    if (gnorm) *gnorm = norm;
    if (!(norm == norm) || norm == HUGE_VAL || norm == -HUGE_VAL) return 0;
    if (clip_norm > 0 && norm > clip_norm) or_scale(grads, n, clip_norm / norm);
    return 1;
}

/* lmtrain.lua:1183-1227 with optimizer = "adamw" (optim2.lua:104-164); *t is
 * the AdamW step count, advanced only when the step is applied. */
int or_lm_step_adamw(const or_lm_cfg* c, double* params, double* m, double* v, int* t,
                     const int* ids, const int* tgt, int B, int T,
                     double lr, double b1, double b2, double eps, double wd, double clip_norm,
                     double* losses, double* gnorm, int* correct, double* grads)
{
    return or_lm_step_adamw_ex(c, params, m, v, t, ids, tgt, B, T, NULL, lr, b1, b2, eps, wd, clip_norm,
                               losses, gnorm, correct, grads);
}

int or_lm_step_adamw_ex(const or_lm_cfg* c, double* params, double* m, double* v, int* t,
                        const int* ids, const int* tgt, int nwin, int T, const int* lens,
                        double lr, double b1, double b2, double eps, double wd, double clip_norm,
                        double* losses, double* gnorm, int* correct, double* grads)
{
    if (!lm_batch_grads(c, params, ids, tgt, nwin, T, lens, clip_norm, losses, gnorm, correct, grads)) return 0;
    *t = *t + 1;
    or_adamw_step(params, grads, m, v, or_lm_num_params(c), lr, b1, b2, eps, wd, *t);
    return 1;
}

/* lmtrain.lua:1183-1227 with optimizer = "sgd" (optim2.lua:48-102) */
int or_lm_step_sgd(const or_lm_cfg* c, double* params, double* vel,
                   const int* ids, const int* tgt, int B, int T,
                   double lr, double momentum, double wd, double clip_norm,
                   double* losses, double* gnorm, int* correct, double* grads)
{
    return or_lm_step_sgd_ex(c, params, vel, ids, tgt, B, T, NULL, lr, momentum, wd, clip_norm, losses, gnorm,
                             correct, grads);
}

int or_lm_step_sgd_ex(const or_lm_cfg* c, double* params, double* vel,
                      const int* ids, const int* tgt, int nwin, int T, const int* lens,
                      double lr, double momentum, double wd, double clip_norm,
                      double* losses, double* gnorm, int* correct, double* grads)
{
    if (!lm_batch_grads(c, params, ids, tgt, nwin, T, lens, clip_norm, losses, gnorm, correct, grads)) return 0;
    or_sgd_step(params, grads, vel, or_lm_num_params(c), lr, momentum, wd, 0);
    return 1;
}


/* ======================================================================
 * The luaTL operation set: the reference GPU path's kernels in double.
 * ====================================================================== */

/* 1/(1+e^-v) by sign (no overflow on either side) */
static double or_sigmoid(double v)
{
    if (v >= 0) return 1.0 / (1.0 + exp(-v));
    const double z = exp(v);
    return z / (1.0 + z);
}

/* cuda/luaTL_core.cu:370-383: the tanh-form GELU and its derivative */
static double or_gelu(double x)
{
    const double c0 = sqrt(2.0 / 3.14159265358979323846), c1 = 0.044715;
    return 0.5 * x * (1.0 + tanh(c0 * (x + c1 * x * x * x)));
}

static double or_gelu_grad(double x)
{
    const double c0 = sqrt(2.0 / 3.14159265358979323846), c1 = 0.044715;
    const double th = tanh(c0 * (x + c1 * x * x * x));
    const double dt = c0 * (1.0 + 3.0 * c1 * x * x);
    return 0.5 * (1.0 + th) + 0.5 * x * (1.0 - th * th) * dt;
}

static double or_silu_grad(double x)
{
    const double s = or_sigmoid(x);
    return s * (1.0 + x * (1.0 - s));
}

/* cuda/luaTL_core.cu:909-934 */
static double or_ew1(int op, double a, double b, double alpha, double beta)
{
    switch (op) {
    case 0: return a;
    case 1: return alpha * a + beta * b;
    case 2: return alpha * a - beta * b;
    case 3: return alpha * a * b;
    case 4: return alpha * a / (b + 1e-20);
    case 5: return alpha * a + beta;
    case 6: return alpha * a + b;
    case 7: return alpha;
    case 8: return a > 0 ? a : 0.0;
    case 9: return or_gelu(a);
    case 10: return a * or_sigmoid(a);
    case 11: return tanh(a);
    case 12: return or_sigmoid(a);
    case 13: return exp(a);
    case 14: return sqrt(a > 0 ? a : 0.0);
    case 15: return 1.0 / sqrt(a > 1e-20 ? a : 1e-20);
    case 16: return -a;
    case 17: return 1.0 / (a + 1e-20);
    case 18: return fabs(a);
    case 19: { double v = a > alpha ? a : alpha; return v < beta ? v : beta; }
    case 20: return a > 0 ? b : 0.0;
    case 21: return b * or_silu_grad(a);
    case 22: return b * or_gelu_grad(a);
    default: return a;
    }
}

void or_ew(int op, const double* a, const double* b, double* c, long n, double alpha, double beta)
{
    for (long i = 0; i < n; ++i) c[i] = or_ew1(op, a ? a[i] : 0.0, b ? b[i] : 0.0, alpha, beta);
}

static double or_act(int act, double v)
{
    switch (act) {
    case 1: return v > 0 ? v : 0.0;
    case 2: return or_gelu(v);
    case 3: return v * or_sigmoid(v);
    case 4: return tanh(v);
    case 5: return or_sigmoid(v);
    default: return v;
    }
}

/* cuda/luaTL_train.cu:127-234 (luaTL_gemm_ex_kernel), one output at a time */
void or_gemm_ex(const double* A, const double* B, double* C, const double* bias, const double* gamma,
                const double* rowscale, int M, int N, int K, long a_rs, long a_cs, long b_rs, long b_cs,
                long c_rs, long c_cs, long a_bs, long b_bs, long c_bs, int batch, double alpha, double beta,
                double eps, int pre_op, int post_op)
{
    if (batch < 1) batch = 1;
    for (int z = 0; z < batch; ++z) {
        const double* Az = A + (long)z * a_bs;
        const double* Bz = B + (long)z * b_bs;
        double* Cz = C + (long)z * c_bs;
        for (int i = 0; i < M; ++i) {
            double rsc = 1.0;
            if (pre_op == 1) {
                if (rowscale) {
                    rsc = rowscale[i];
                } else {
                    double ss = 0;
                    for (int k = 0; k < K; ++k) {
                        const double a = Az[i * a_rs + k * a_cs];
                        ss += a * a;
                    }
                    rsc = 1.0 / sqrt(ss / K + eps);
                }
            }
            for (int j = 0; j < N; ++j) {
                double acc = 0;
                for (int k = 0; k < K; ++k) {
                    double a = Az[i * a_rs + k * a_cs];
                    if (pre_op == 1) a = a * rsc * (gamma ? gamma[k] : 1.0);
                    else if (pre_op == 2) a = or_gelu(a);
                    else if (pre_op == 3) a = a * or_sigmoid(a);
                    else if (pre_op == 4) a = a > 0 ? a : 0.0;
                    acc += a * Bz[k * b_rs + j * b_cs];
                }
                double v = alpha * acc;
                if (bias) v += bias[j];
                v = or_act(post_op, v);
                double* cp = Cz + i * c_rs + j * c_cs;
                if (beta != 0) v += beta * *cp;
                *cp = v;
            }
        }
    }
}

/* cuda/luaTL_train.cu:545-585 */
void or_softmax_ex(const double* x, const double* bias, double* y, int rows, int cols, double scale,
                   int causal, int group, int moff)
{
    for (int r = 0; r < rows; ++r) {
        const int lrow = group > 0 ? r % group : r;
        const int limit = causal ? lrow + moff : cols - 1;
        const double* xr = x + (long)r * cols;
        double* yr = y + (long)r * cols;
        double mx = -INFINITY;
        for (int i = 0; i < cols && i <= limit; ++i) {
            double v = xr[i] * scale + (bias ? bias[i] : 0.0);
            if (v > mx) mx = v;
        }
        const double base = mx == -INFINITY ? 0.0 : mx;
        double sum = 0;
        for (int i = 0; i < cols; ++i) {
            double e = 0;
            if (i <= limit) e = exp(xr[i] * scale + (bias ? bias[i] : 0.0) - base);
            yr[i] = e;
            sum += e;
        }
        const double inv = sum > 0 ? 1.0 / sum : 0.0;
        for (int i = 0; i < cols; ++i) yr[i] *= inv;
    }
}

/* cuda/luaTL_train.cu:589-619 */
void or_softmax_bwd_ex(const double* y, const double* dy, double* dx, int rows, int cols, double scale,
                       int causal, int group, int moff)
{
    for (int r = 0; r < rows; ++r) {
        const int lrow = group > 0 ? r % group : r;
        const int limit = causal ? lrow + moff : cols - 1;
        const long o = (long)r * cols;
        double dot = 0;
        for (int i = 0; i < cols && i <= limit; ++i) dot += dy[o + i] * y[o + i];
        for (int i = 0; i < cols; ++i) dx[o + i] = i <= limit ? scale * y[o + i] * (dy[o + i] - dot) : 0.0;
    }
}

/* cuda/luaTL_train.cu:489-526 */
void or_rmsnorm_bwd_luatl(const double* x, const double* g, const double* dy, double* dx, double* dgamma,
                          int rows, int cols, double eps)
{
    for (int r = 0; r < rows; ++r) {
        const double* xr = x + (long)r * cols;
        const double* dyr = dy + (long)r * cols;
        double ss = 0;
        for (int i = 0; i < cols; ++i) ss += xr[i] * xr[i];
        const double s = 1.0 / sqrt(ss / cols + eps);
        double dot = 0;
        for (int i = 0; i < cols; ++i) dot += dyr[i] * (g ? g[i] : 1.0) * xr[i];
        const double c = (s * s * s / cols) * dot;
        for (int i = 0; i < cols; ++i) {
            dx[(long)r * cols + i] = s * (g ? g[i] : 1.0) * dyr[i] - c * xr[i];
            if (dgamma) dgamma[i] += dyr[i] * xr[i] * s;
        }
    }
}

/* cuda/luaTL_core.cu:1346-1380 with the corrections of cuda/luaTL_train.cu:1427-1449 */
void or_adamw_luatl(double* w, const double* g, double* m, double* v, long n, int step, double lr,
                    double b1, double b2, double eps, double wd, double clip)
{
    const int t = step < 1 ? 1 : step;
    const double bc1 = 1.0 / (1.0 - pow(b1, t));
    const double bc2 = 1.0 / (1.0 - pow(b2, t));
    for (long i = 0; i < n; ++i) {
        double gr = g[i];
        if (clip > 0) gr = gr < -clip ? -clip : (gr > clip ? clip : gr);
        const double mi = b1 * m[i] + (1 - b1) * gr;
        const double vi = b2 * v[i] + (1 - b2) * gr * gr;
        m[i] = mi;
        v[i] = vi;
        double wi = w[i];
        wi -= lr * wd * wi;
        wi -= lr * (mi * bc1) / (sqrt(vi * bc2) + eps);
        w[i] = wi;
    }
}

/* cuda/luaTL_train.cu:895-906 */
void or_reduce_cols(const double* x, double* out, int rows, int cols, long rs, double alpha, double beta)
{
    for (int c = 0; c < cols; ++c) {
        double acc = 0;
        for (int r = 0; r < rows; ++r) acc += x[(long)r * rs + c];
        out[c] = alpha * acc + beta * out[c];
    }
}

/* cuda/luaTL_train.cu:947-965 */
void or_clip_by_nsq(double* x, long n, double nsq, double max_norm)
{
    const double nrm = sqrt(nsq > 0 ? nsq : 0.0);
    double f = 1.0;
    if (max_norm > 0 && nrm > max_norm) f = max_norm / (nrm + 1e-6);
    if (f == 1.0) return;
    for (long i = 0; i < n; ++i) x[i] *= f;
}
