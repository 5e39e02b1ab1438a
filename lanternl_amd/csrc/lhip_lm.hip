// lhip_lm.hip -- one LMTrain optimizer step of the CPU path, resident on the GPU.
//
// Model and step semantics are the CPU LMTrain path's:
//   ai/nn/transformer.lua:84-257 (pre-norm decoder: RMSNorm, separate wq/wk/wv,
//     per-head attention with interleaved-pair RoPE, causal softmax of
//     scores/sqrt(hd), wo, residual, RMSNorm, SwiGLU with separate w1/w3/w2,
//     residual, final RMSNorm, head tied to the embedding via matmul_nt);
//   ai/core/tensor2.lua (each op's forward and backward);
//   ai/optim/lmtrain.lua:1183-1227 (B windows of T tokens per step, the loss
//     of each window the mean over its T targets, grads summed over windows
//     then scaled by 1/B, global-norm skip/clip, optimizer step) with
//     optimizer "sgd" (ai/optim/optim2.lua:48-102).
// The B windows are independent sequences, so they are processed together as
// one [B*T, dim] block: every projection is one GEMM over all B*T rows, the
// attention products are 2-level batched GEMMs over (window, head), the
// causal mask restarts every T rows (group = T), and RoPE positions are
// row % T.  Parameters, gradients and velocities are single flat device
// buffers in Transformer:parameters() order (transformer.lua:150-164), so the
// global norm and the SGD update are one reduction and one elementwise pass.
// The GPU-resident reference path (ai/gpu/gpu_transformer.lua) has different
// numerics (fused weights, half-split RoPE, AdamW); it is not what this follows.
//
// The whole step is enqueued on the library stream with no host round trip
// (the norm, the skip decision and the clip factor stay on the device) and no
// allocation, so it can be captured once into a hipGraph and replayed.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include "lhip_internal.h"

namespace lhip {
namespace {

enum { P_LN1, P_WQ, P_WK, P_WV, P_WO, P_LN2, P_W1, P_W3, P_W2, P_PER_LAYER };

enum { OPT_SGD = 0, OPT_ADAMW = 1 };

// Optimizer hyper-parameters of one step.  Eager launches pass them by value;
// a captured step reads them from the device copy m.hyper, laid out as
// {lr, momentum, wd, clip, nesterov, beta1, beta2, eps, parity, gscale}, which
// set_hyper_kernel refreshes before each replay.  gscale is the batch's
// scale_grads factor, 1/n for n > 1 windows (lmtrain.lua:1211).
struct Hyper {
    float lr, momentum, wd, clip, nesterov, beta1, beta2, eps, parity, gscale;
    int opt;
};

__global__ void set_hyper_kernel(float* hp, const Hyper h)
{
    if (threadIdx.x == 0) {
        hp[0] = h.lr; hp[1] = h.momentum; hp[2] = h.wd; hp[3] = h.clip; hp[4] = h.nesterov;
        hp[5] = h.beta1; hp[6] = h.beta2; hp[7] = h.eps; hp[8] = h.parity; hp[9] = h.gscale;
    }
}

struct LmModel {
    lhip_lm_config_t c{};
    int N = 0, D = 0, F = 0, V = 0, H = 0, hd = 0, L = 0, T = 0, B = 0;
    long long nparam = 0;
    std::vector<long long> off;   // float offset of each parameter tensor
    void* arena = nullptr;        // every device buffer below lives in it
    size_t arena_bytes = 0;
    float *params = nullptr, *grads = nullptr, *vel = nullptr;
    int *ids = nullptr, *tgt = nullptr, *amax = nullptr, *applied = nullptr;
    int* wlen = nullptr;          // tokens of each window slot (0: empty slot)
    float *losses = nullptr, *gnorm = nullptr, *hyper = nullptr;
    float *adam_m = nullptr, *adam_v = nullptr;   // AdamW moments
    int* tcount = nullptr;                         // AdamW step count, two parity slots
    long long adam_calls = 0;                      // AdamW steps enqueued (slot parity)
    double *ss = nullptr, *ss_part = nullptr;
    int ss_blocks = 0;   // the stand-alone partial kernel's block count
    int ss_cap = 0;      // ss_part's length (also holds the grouped launch's per-workgroup partials)
    // saved activations
    float *x = nullptr, *h = nullptr, *inv1 = nullptr, *qkv = nullptr, *P = nullptr, *ctx = nullptr;
    float *xmid = nullptr, *h2 = nullptr, *inv2 = nullptr, *zu = nullptr, *a = nullptr;
    float *xf = nullptr, *invf = nullptr, *logits = nullptr;
    // backward: gradient-chain buffers are per layer (gx[l] = dL/dx_l,
    // gmid[l] = dL/dxmid_l, dzu[l], dqkv[l], the dw partials of each norm) so
    // that the weight gradients, issued after the whole chain, still find them
    float *dxf = nullptr, *gx = nullptr, *gmid = nullptr, *da = nullptr, *dzu = nullptr, *dh2 = nullptr;
    float *dctx = nullptr, *dP = nullptr, *dS = nullptr, *dqkv = nullptr, *dh = nullptr, *work = nullptr;
    size_t work_floats = 0;       // per norm call; work holds 2L+1 of them
    float* splitk = nullptr;      // split-K partials
    size_t splitk_floats = 0;
    float2* rope_cs = nullptr;    // (cos, sin) of positions 0..T-1, pairs 0..hd/2-1
    bool fused_attn = false;      // per-(window, head) fused attention kernels
    bool fused_gemm = false;      // norm / SwiGLU stages fused into their GEMMs
    // graph
    bool use_graph = false;
    int graph_opt = -1;           // optimizer of the captured step
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int steps = 0;
    bool have_batch = false;
    std::vector<int> h_tgt;       // targets per row, -1 past a window's length
    std::vector<int> h_len;       // window lengths (0 for empty slots)
    int nwin = 0;                 // windows in the batch (slots 0 .. nwin-1)

    const float* prm(int tensor) const { return params + off[tensor]; }
    float* grd(int tensor) const { return grads + off[tensor]; }
    int lt(int l, int which) const { return 1 + P_PER_LAYER * l + which; }
};

long long count_params(const lhip_lm_config_t& c)
{
    const long long D = c.dim, F = c.ffn, V = c.vocab;
    return V * D + static_cast<long long>(c.layers) * (2 * D + 4 * D * D + 3 * D * F) + D;
}

// model dimensions only (parameter layout)
int check_dims(const lhip_lm_config_t* c)
{
    if (!c) return fail(LHIP_E_NULL, "lm: config is NULL");
    if (c->vocab <= 0 || c->dim <= 0 || c->layers <= 0 || c->heads <= 0 || c->ffn <= 0)
        return fail(LHIP_E_SHAPE, "lm: every model size must be > 0 (vocab=%d dim=%d layers=%d heads=%d ffn=%d)",
                    c->vocab, c->dim, c->layers, c->heads, c->ffn);
    return LHIP_OK;
}

int check_config(const lhip_lm_config_t* c)
{
    if (int rc = check_dims(c)) return rc;
    if (c->batch <= 0 || c->seq <= 0)
        return fail(LHIP_E_SHAPE, "lm: batch=%d and seq=%d must be > 0", c->batch, c->seq);
    if (c->dim % c->heads) return fail(LHIP_E_SHAPE, "lm: dim %d not divisible by heads %d", c->dim, c->heads);
    const int hd = c->dim / c->heads;
    if (hd % 2) return fail(LHIP_E_SHAPE, "lm: head_dim %d must be even for RoPE", hd);
    if (hd > 256) return fail(LHIP_E_CAPACITY, "lm: head_dim %d > 256", hd);
    if (!(c->eps >= 0.0) || !(c->rope_base > 0.0)) return fail(LHIP_E_ARG, "lm: eps must be >= 0 and rope_base > 0");
    if (static_cast<long long>(c->batch) * c->seq > (1LL << 28))
        return fail(LHIP_E_CAPACITY, "lm: batch*seq too large");
    return LHIP_OK;
}

// ---- the step ------------------------------------------------------------
struct Enq {
    LmModel& m;
    hipStream_t s;
    float* ws;   // split-K partials

    GemmOpts opts(int inner = 1) const
    {
        GemmOpts o;
        o.inner = inner;
        o.ws = ws;
        o.ws_floats = m.splitk_floats;
        return o;
    }
    // C = sum_j A_j . op(B_j) over kb blocks (A_j = A + j*sak, B_j = B + j*sbk)
    int brgemm(int tb, int M, int Nn, int K, int kb, const float* A, int lda, long long sak, const float* Bm,
               int ldb, long long sbk, float* C, int ldc) const
    {
        GemmOpts o = opts();
        o.kblocks = kb;
        o.sAk = sak;
        o.sBk = sbk;
        return sgemm_run(0, tb, M, Nn, K, 1.f, A, lda, 0, Bm, ldb, 0, 0.f, C, ldc, 0, 1, o, s);
    }
    int gemm(int ta, int tb, int M, int Nn, int K, const float* A, int lda, const float* Bm, int ldb, float beta,
             float* C, int ldc) const
    {
        return sgemm_run(ta, tb, M, Nn, K, 1.f, A, lda, 0, Bm, ldb, 0, beta, C, ldc, 0, 1, opts(), s);
    }
    // C = A.B + R (the residual add fused into the GEMM epilogue)
    int gemm_res(int M, int Nn, int K, const float* A, int lda, const float* Bm, int ldb, const float* R, float* C,
                 int ldc) const
    {
        GemmOpts o = opts();
        o.R = R;
        o.ldr = ldc;
        return sgemm_run(0, 0, M, Nn, K, 1.f, A, lda, 0, Bm, ldb, 0, 1.f, C, ldc, 0, 1, o, s);
    }
    int bgemm(int ta, int tb, int M, int Nn, int K, const float* A, int lda, long long sa, const float* Bm, int ldb,
              long long sb, float beta, float* C, int ldc, long long sc, int batch) const
    {
        return sgemm_run(ta, tb, M, Nn, K, 1.f, A, lda, sa, Bm, ldb, sb, beta, C, ldc, sc, batch, opts(batch), s);
    }
    // batch (window b, head h): operand offsets b*X2 + h*X
    int hgemm(int ta, int tb, int M, int Nn, int K, const float* A, int lda, long long sa, long long sa2,
              const float* Bm, int ldb, long long sb, long long sb2, float* C, int ldc, long long sc,
              long long sc2) const
    {
        GemmOpts o = opts(m.H);
        o.sA2 = sa2; o.sB2 = sb2; o.sC2 = sc2;
        return sgemm_run(ta, tb, M, Nn, K, 1.f, A, lda, sa, Bm, ldb, sb, 0.f, C, ldc, sc, m.B * m.H, o, s);
    }
};

#define LM_TRY(expr)                       \
    do {                                   \
        int _rc = (expr);                  \
        if (_rc != LHIP_OK) return _rc;    \
    } while (0)

// device_hyper: read the hyper-parameters from m.hyper (captured steps)
int enqueue_step(LmModel& m, hipStream_t s, const Hyper& hp, bool device_hyper)
{
    const Enq q{m, s, m.splitk};
    const int N = m.N, D = m.D, F = m.F, V = m.V, H = m.H, hd = m.hd, T = m.T, L = m.L;
    const long long ND = static_cast<long long>(N) * D, NF = static_cast<long long>(N) * F;
    const long long TT = static_cast<long long>(T) * T, HTT = H * TT, TD = static_cast<long long>(T) * D;
    const long long PL = static_cast<long long>(m.B) * HTT;          // softmax block per layer
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    const int causal = m.c.causal ? 1 : 0;
    const float eps = static_cast<float>(m.c.eps);
    const double base = m.c.rope_base;
    const float* emb = m.prm(0);
    const float* lnf = m.prm(1 + P_PER_LAYER * L);

    // opt.zero_grad() needs no pass: every gradient tensor's first writer in
    // the backward overwrites it (beta = 0 GEMMs, accumulate = 0 column sums)

    // ---------------- forward (transformer.lua:228-257) ----------------
    // x_0 = emb[ids]: with fused GEMMs, gathered by layer 0's norm + q/k/v GEMM
    if (!m.fused_gemm) LM_TRY(embed_fwd(emb, m.ids, m.x, N, D, V, s));
    for (int l = 0; l < L; ++l) {
        const float* xl = m.x + l * ND;
        float* h = m.h + l * ND;
        float* inv1 = m.inv1 + static_cast<long long>(l) * N;
        float* qkv = m.qkv + l * 3 * ND;
        float* P = m.P + l * PL;
        float* ctx = m.ctx + l * ND;
        float* xmid = m.xmid + l * ND;
        float* h2 = m.h2 + l * ND;
        float* inv2 = m.inv2 + static_cast<long long>(l) * N;
        float* zu = m.zu + l * 2 * NF;
        float* a = m.a + l * NF;
        float* xn = m.x + (l + 1) * ND;
        // h = rmsnorm(x); q, k, v = h.Wq, h.Wk, h.Wv (the three weights are adjacent)
        if (m.fused_gemm) {
            FuseCall c;
            c.mode = FUSE_NORM; c.M = N; c.N = D; c.K = D; c.batch = 3;
            c.A = xl; c.lda = D; c.B = m.prm(m.lt(l, P_WQ)); c.ldb = D; c.sB = static_cast<long long>(D) * D;
            if (l == 0) { c.A = emb; c.gather = m.ids; c.gather_rows = V; c.xout = m.x; }
            c.C = qkv; c.ldc = D; c.sC = ND;
            c.nw = m.prm(m.lt(l, P_LN1)); c.eps = eps; c.h = h; c.inv = inv1;
            LM_TRY(lm_fused_gemm(c, s));
        } else {
            LM_TRY(rmsnorm_fwd(xl, m.prm(m.lt(l, P_LN1)), h, inv1, N, D, eps, s));
            LM_TRY(q.bgemm(0, 0, N, D, D, h, D, 0, m.prm(m.lt(l, P_WQ)), D, static_cast<long long>(D) * D, 0.f, qkv, D,
                           ND, 3));
        }
        if (m.fused_attn) {
            // RoPE, scores, causal softmax and P.v per (window, head) in one launch;
            // qkv keeps the unrotated q, k (the backward rotates again)
            LM_TRY(attn_fwd(qkv, m.rope_cs, P, ctx, m.B, H, T, hd, scale, causal, s, m.wlen));
        } else {
            // RoPE on q and k (2N rows, positions row % T), interleaved pairs
            LM_TRY(rope(qkv, nullptr, 2 * N, H, hd, D, 0, T, base, 1, 0, s));
            // scores = q_bh . k_bh^T per (window, head), into the (forward-idle) dP
            // scratch; P = softmax(scale * scores)
            LM_TRY(q.hgemm(0, 1, T, T, hd, qkv, D, hd, TD, qkv + ND, D, hd, TD, m.dP, T, TT, HTT));
            LM_TRY(softmax_fwd(m.dP, P, m.B * H * T, T, scale, causal, 0, T, s));
            // ctx[:, h*hd:] = P_bh . v_bh
            LM_TRY(q.hgemm(0, 0, T, hd, T, P, T, TT, HTT, qkv + 2 * ND, D, hd, TD, ctx, D, hd, TD));
        }
        // x_mid = x + ctx . Wo
        LM_TRY(q.gemm_res(N, D, D, ctx, D, m.prm(m.lt(l, P_WO)), D, xl, xmid, D));
        // h2 = rmsnorm(x_mid); z1 = h2.W1, u = h2.W3; a = silu(z1) * u
        if (m.fused_gemm) {
            FuseCall c;
            c.mode = FUSE_NORM_SWIGLU; c.M = N; c.N = F; c.K = D;
            c.A = xmid; c.lda = D; c.B = m.prm(m.lt(l, P_W1)); c.ldb = F; c.B2 = m.prm(m.lt(l, P_W3));
            c.C = zu; c.C2 = zu + NF; c.Aout = a; c.ldc = F;
            c.nw = m.prm(m.lt(l, P_LN2)); c.eps = eps; c.h = h2; c.inv = inv2;
            LM_TRY(lm_fused_gemm(c, s));
        } else {
            LM_TRY(rmsnorm_fwd(xmid, m.prm(m.lt(l, P_LN2)), h2, inv2, N, D, eps, s));
            LM_TRY(q.bgemm(0, 0, N, F, D, h2, D, 0, m.prm(m.lt(l, P_W1)), F, static_cast<long long>(D) * F, 0.f, zu, F,
                           NF, 2));
            LM_TRY(swiglu_fwd(zu, F, zu + NF, F, a, F, N, F, s));
        }
        // x_{l+1} = x_mid + a . W2
        LM_TRY(q.gemm_res(N, D, F, a, F, m.prm(m.lt(l, P_W2)), D, xmid, xn, D));
    }
    const float* xL = m.x + static_cast<long long>(L) * ND;
    LM_TRY(rmsnorm_fwd(xL, lnf, m.xf, m.invf, N, D, eps, s));
    // tied head: logits = xf . emb^T
    LM_TRY(q.gemm(0, 1, N, V, D, m.xf, D, emb, D, 0.f, m.logits, V));
    // per-row losses; dlogits = (softmax - onehot) / len(window) written over
    // the logits; rows past a window's length (target -1) give 0 and 0
    LM_TRY(ce_fused(m.logits, m.tgt, m.losses, m.logits, N, V, -1, 1.0f, s, m.amax, m.wlen, T));

    // ---------------- backward ----------------
    // The chain dlogits -> dx_L -> ... -> dx_0 first, then the weight gradients.
    const float* dlg = m.logits;
    const size_t wf = m.work_floats;
    auto gxl = [&](int l) { return m.gx + l * ND; };
    // An RMSNorm backward whose dx rows the next NT GEMM of the chain consumes:
    // with fused GEMMs it runs as that GEMM's A prologue, otherwise as its own
    // launch just before.  Its gain's dw partials are column-summed after the chain.
    struct NormBwd {
        const float *x, *w, *inv, *dy, *dres;
        float *out, *part, *gw;
        int parts;
        int dy_parts;   // dy = sum of this many [N][D] slices (unreduced split-K)
    };
    const int tiles_m = ceil_div(N, 16);
    auto norm_standalone = [&](NormBwd& nb) {
        return rmsnorm_bwd_rows(nb.x, nb.w, nb.inv, nb.dy, nb.out, nb.dres, nb.part, wf, N, D, &nb.parts, s);
    };
    auto norm_prologue = [&](FuseCall& c, NormBwd& nb) {
        c.A = nb.dy; c.lda = D; c.nw = nb.w; c.nbx = nb.x; c.nbres = nb.dres; c.nbinv = nb.inv;
        c.nbout = nb.out; c.nbpart = nb.part;
        c.a_parts = nb.dy_parts; c.a_pstride = ND;
        nb.parts = tiles_m;
    };
    // Weight gradients dW = X^T . dY and the norm gains' column sums are
    // collected and issued after the backward chain, as one grouped launch and
    // one column-sum launch (every buffer they read is per layer, so nothing is
    // overwritten before then).  Forking them per layer onto a second stream
    // was measured slower: each event record + stream wait costs ~13 us of host
    // time on this ROCm, and the forks kept the host behind the GPU.
    GroupedTN dw_all[kGroupedMax];
    int ndw = 0;
    const float* cs_p[kColsumJobs];
    int cs_n[kColsumJobs];
    float* cs_o[kColsumJobs];
    int ncs = 0;
    bool flushed = false;   // some products or column sums were issued before the final launch
    GroupedTN gemb{dlg, V, m.xf, D, m.grd(0), D, V, D};                           // gemb = dlogits^T . xf
    // the tied table's second term, dx_0 scattered to the token rows (gemb[id_i] += dx_0[i]),
    // when the final launch can fold it in
    gemb.sc_ids = m.ids; gemb.sc_rows = gxl(0); gemb.sc_ld = D; gemb.sc_n = N; gemb.sc_scale = 1.f;
    dw_all[ndw++] = gemb;
    // dxf = dlogits . emb; with fused GEMMs its split-K slices are left
    // unreduced and summed by the norm-backward prologue that consumes dxf
    int dxf_parts = 1;
    {
        GemmOpts o = q.opts();
        if (m.fused_gemm) o.splits_out = &dxf_parts;
        LM_TRY(sgemm_run(0, 0, N, D, V, 1.f, dlg, V, 0, emb, D, 0, 0.f, m.dxf, D, 0, 1, o, s));
    }
    NormBwd pend{xL, lnf, m.invf, dxf_parts > 1 ? q.ws : m.dxf, nullptr, gxl(L), m.work,
                 m.grd(1 + P_PER_LAYER * L), 0, dxf_parts};
    for (int l = L - 1; l >= 0; --l) {
        const float* xl = m.x + l * ND;
        const float* h = m.h + l * ND;
        const float* inv1 = m.inv1 + static_cast<long long>(l) * N;
        const float* qkv = m.qkv + l * 3 * ND;
        const float* P = m.P + l * PL;
        const float* ctx = m.ctx + l * ND;
        const float* xmid = m.xmid + l * ND;
        const float* h2 = m.h2 + l * ND;
        const float* inv2 = m.inv2 + static_cast<long long>(l) * N;
        const float* zu = m.zu + l * 2 * NF;
        const float* a = m.a + l * NF;
        const float* gin = gxl(l + 1);                 // dL/dx_{l+1} (written by the pending norm backward)
        float* gmid = m.gmid + l * ND;                 // dL/dxmid_l
        float* dzu = m.dzu + l * 2 * NF;
        float* dqkv = m.dqkv + l * 3 * ND;
        // f = a . W2 ; a = silu(z1) * u:  da = gin . W2^T, then the SwiGLU backward into dz1, du
        if (m.fused_gemm) {
            FuseCall c;
            c.mode = FUSE_NB_SWIGLU_BWD; c.M = N; c.N = F; c.K = D;
            c.B = m.prm(m.lt(l, P_W2)); c.ldb = D; c.ldc = F;
            c.Z = zu; c.U = zu + NF; c.dZ = dzu; c.dU = dzu + NF;
            norm_prologue(c, pend);
            LM_TRY(lm_fused_gemm(c, s));
        } else {
            LM_TRY(norm_standalone(pend));
            LM_TRY(q.gemm(0, 1, N, F, D, gin, D, m.prm(m.lt(l, P_W2)), D, 0.f, m.da, F));
            LM_TRY(swiglu_bwd(zu, F, zu + NF, F, m.da, F, dzu, F, dzu + NF, F, N, F, 0, s));
        }
        // dh2 = dz1 . W1^T + du . W3^T (adjacent weights: one batch-reduce GEMM)
        LM_TRY(q.brgemm(1, N, D, F, 2, dzu, F, NF, m.prm(m.lt(l, P_W1)), F, static_cast<long long>(D) * F, m.dh2, D));
        // gmid = gin + RMSNorm backward (ln2); o = ctx . Wo: dctx = gmid . Wo^T
        NormBwd n2{xmid, m.prm(m.lt(l, P_LN2)), inv2, m.dh2, gin, gmid, m.work + (2 * l + 1) * wf,
                   m.grd(m.lt(l, P_LN2)), 0, 1};
        if (m.fused_gemm) {
            FuseCall c;
            c.mode = FUSE_NB_NT; c.M = N; c.N = D; c.K = D;
            c.B = m.prm(m.lt(l, P_WO)); c.ldb = D; c.C = m.dctx; c.ldc = D;
            norm_prologue(c, n2);
            LM_TRY(lm_fused_gemm(c, s));
        } else {
            LM_TRY(norm_standalone(n2));
            LM_TRY(q.gemm(0, 1, N, D, D, gmid, D, m.prm(m.lt(l, P_WO)), D, 0.f, m.dctx, D));
        }
        if (m.fused_attn) {
            // dP, dv, softmax backward, dq, dk and the inverse RoPE per (window, head)
            LM_TRY(attn_bwd(qkv, m.rope_cs, P, ctx, m.dctx, dqkv, m.B, H, T, hd, scale, causal, s));
        } else {
            // per (window, head): dP = dO . v^T ; dv = P^T . dO
            LM_TRY(q.hgemm(0, 1, T, T, hd, m.dctx, D, hd, TD, qkv + 2 * ND, D, hd, TD, m.dP, T, TT, HTT));
            LM_TRY(q.hgemm(1, 0, T, hd, T, P, T, TT, HTT, m.dctx, D, hd, TD, dqkv + 2 * ND, D, hd, TD));
            // dS = scale * softmax_bwd(P, dP)
            LM_TRY(softmax_bwd(P, m.dP, m.dS, m.B * H * T, T, scale, causal, 0, T, 0, s));
            // dq = dS . k_rot ; dk = dS^T . q_rot
            LM_TRY(q.hgemm(0, 0, T, hd, T, m.dS, T, TT, HTT, qkv + ND, D, hd, TD, dqkv, D, hd, TD));
            LM_TRY(q.hgemm(1, 0, T, hd, T, m.dS, T, TT, HTT, qkv, D, hd, TD, dqkv + ND, D, hd, TD));
            // RoPE backward (inverse rotation) on dq and dk
            LM_TRY(rope(dqkv, nullptr, 2 * N, H, hd, D, 0, T, base, 1, 1, s));
        }
        // This layer's share of the deferred work: the two norm gains' column
        // sums (the pending norm above this layer and ln2) and the layer's
        // seven weight gradients dW = X^T . dY.
        {
            const float* parts_p[2] = {pend.part, n2.part};
            const int parts_n[2] = {pend.parts, n2.parts};
            float* parts_o[2] = {pend.gw, n2.gw};
            const long long DD = static_cast<long long>(D) * D;
            const GroupedTN gw[7] = {
                {a, F, gin, D, m.grd(m.lt(l, P_W2)), D, F, D},                 // gW2 = a^T . gin
                {h2, D, dzu, F, m.grd(m.lt(l, P_W1)), F, D, F},                // gW1 = h2^T . dz1
                {h2, D, dzu + NF, F, m.grd(m.lt(l, P_W3)), F, D, F},           // gW3 = h2^T . du
                {ctx, D, gmid, D, m.grd(m.lt(l, P_WO)), D, D, D},              // gWo = ctx^T . gmid
                {h, D, dqkv, D, m.grd(m.lt(l, P_WQ)), D, D, D},                // gWq = h^T . dq
                {h, D, dqkv + ND, D, m.grd(m.lt(l, P_WQ)) + DD, D, D, D},      // gWk = h^T . dk
                {h, D, dqkv + 2 * ND, D, m.grd(m.lt(l, P_WQ)) + 2 * DD, D, D, D},  // gWv = h^T . dv
            };
            // a full batch is issued now (deep models); the rest waits for the end
            if (ndw + 7 > kGroupedMax) {
                LM_TRY(sgemm_grouped_tn(dw_all, ndw, N, s));
                ndw = 0;
                flushed = true;
            }
            if (ncs + 2 > kColsumJobs) {
                LM_TRY(rmsnorm_bwd_colsum_multi(cs_p, cs_n, cs_o, ncs, D, 0, s));
                ncs = 0;
                flushed = true;
            }
            for (int i = 0; i < 7; ++i) dw_all[ndw++] = gw[i];
            for (int i = 0; i < 2; ++i) { cs_p[ncs] = parts_p[i]; cs_n[ncs] = parts_n[i]; cs_o[ncs] = parts_o[i]; ++ncs; }
        }
        // dh = dq.Wq^T + dk.Wk^T + dv.Wv^T (adjacent weights: one batch-reduce GEMM)
        LM_TRY(q.brgemm(1, N, D, D, 3, dqkv, D, ND, m.prm(m.lt(l, P_WQ)), D, static_cast<long long>(D) * D, m.dh, D));
        // dx_l = gmid + RMSNorm backward (ln1): runs with the next layer's first GEMM
        pend = NormBwd{xl, m.prm(m.lt(l, P_LN1)), inv1, m.dh, gmid, gxl(l), m.work + (2 * l + 2) * wf,
                       m.grd(m.lt(l, P_LN1)), 0, 1};
    }
    LM_TRY(norm_standalone(pend));                       // dx_0 (no GEMM follows it)
    if (ncs + 1 > kColsumJobs) {
        LM_TRY(rmsnorm_bwd_colsum_multi(cs_p, cs_n, cs_o, ncs, D, 0, s));
        ncs = 0;
        flushed = true;
    }
    cs_p[ncs] = pend.part; cs_n[ncs] = pend.parts; cs_o[ncs] = pend.gw; ++ncs;
    int ss_parts = 0;   // squared-norm partials the optimizer sums
    {
        // the last products and the gains' column sums in one launch
        ColsumSet cs{};
        for (int i = 0; i < ncs; ++i) { cs.partial[i] = cs_p[i]; cs.nparts[i] = cs_n[i]; cs.out[i] = cs_o[i]; }
        cs.njobs = ncs; cs.cols = D; cs.acc = 0;
        // with every gradient stored by this launch (nothing issued earlier),
        // it also runs the scatter and leaves the squared-norm partials
        GroupedExtras ex;
        if (!flushed) {
            ex.ss_out = m.ss_part;
            ex.ss_cap = m.ss_cap;
        }
        LM_TRY(sgemm_grouped_tn(dw_all, ndw, N, s, &cs, &ex));
        ss_parts = ex.fused ? ex.ss_parts : 0;
    }
    // ---------------- optimizer (lmtrain.lua:1212-1226) ----------------
    if (ss_parts == 0) {
        LM_TRY(embed_bwd(gxl(0), m.ids, m.grd(0), N, D, V, 1.f, 1, s));    // after gemb (same launch order)
        // squared-norm partials; the optimizer kernel finishes the sum itself
        LM_TRY(sumsq_partials(m.grads, m.nparam, m.ss_part, m.ss_blocks, s));
        ss_parts = m.ss_blocks;
    }
    const float gscale = hp.gscale;
    const float* hdev = device_hyper ? m.hyper : nullptr;
    if (hp.opt == OPT_ADAMW)
        LM_TRY(adamw_step(m.params, m.grads, m.adam_m, m.adam_v, m.nparam, m.ss_part, ss_parts, hp.lr, hp.beta1,
                          hp.beta2, hp.eps, hp.wd, gscale, hp.clip, 0, m.tcount, hp.parity != 0.f ? 1 : 0, m.gnorm,
                          m.applied, s, hdev));
    else
        LM_TRY(sgd_step(m.params, m.grads, m.vel, m.nparam, m.ss_part, hp.lr, hp.momentum, hp.wd, gscale, hp.clip,
                        hp.nesterov != 0.f ? 1 : 0, m.gnorm, m.applied, s, hdev, ss_parts));
    return LHIP_OK;
}

void drop_graph(LmModel& m)
{
    if (m.exec) (void)hipGraphExecDestroy(m.exec);
    if (m.graph) (void)hipGraphDestroy(m.graph);
    m.exec = nullptr;
    m.graph = nullptr;
}

int capture_step(LmModel& m, hipStream_t s, const Hyper& hp)
{
    drop_graph(m);
    LHIP_CHECK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "lm: begin capture");
    const int rc = enqueue_step(m, s, hp, true);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(s, &g);
    if (rc != LHIP_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return hip_fail(e, "lm: end capture");
    m.graph = g;
    const hipError_t e2 = hipGraphInstantiate(&m.exec, m.graph, nullptr, nullptr, 0);
    if (e2 != hipSuccess) {
        drop_graph(m);
        return hip_fail(e2, "lm: graph instantiate");
    }
    m.graph_opt = hp.opt;
    return LHIP_OK;
}

// One step with the given optimizer: graph replay (capturing first when
// needed) or eager launches.
int run_step(LmModel& m, Hyper hp)
{
    hipStream_t s = st().stream;
    hp.gscale = m.nwin > 1 ? 1.0f / static_cast<float>(m.nwin) : 1.0f;   // optim2.scale_grads(1/n)
    if (m.use_graph) {
        // a graph replay's kernels are not launched through klaunch, so the
        // kernel timer could not time them (lhip_program_begin refuses too)
        if (ktimer().on)
            return fail(LHIP_E_UNSUPPORTED, "lm step: graph mode while the kernel timer is on");
        klaunch(set_hyper_kernel, 1, 64, 0, s, m.hyper, hp);
        if (int rc = check_launch("lm step: hyper")) return rc;
        if (!m.exec || m.graph_opt != hp.opt)
            if (int rc = capture_step(m, s, hp)) return rc;
        LHIP_CHECK_HIP(hipGraphLaunch(m.exec, s), "lm step: graph launch");
    } else {
        if (int rc = enqueue_step(m, s, hp, false)) return rc;
    }
    ++m.steps;
    if (hp.opt == OPT_ADAMW) ++m.adam_calls;
    return LHIP_OK;
}

LmModel* as_model(void* p) { return static_cast<LmModel*>(p); }

// Device resources of a model (graph, arena); the caller has synchronized.
void release(LmModel& m)
{
    drop_graph(m);
    if (m.arena) (void)hipFree(m.arena);
    m.arena = nullptr;
}

}  // namespace
}  // namespace lhip

using lhip::fail;
using lhip::st;

extern "C" {

LHIP_API long long lhip_lm_num_params(const lhip_lm_config_t* cfg)
{
    if (lhip::check_dims(cfg) != LHIP_OK) return -1;
    return lhip::count_params(*cfg);
}

LHIP_API int lhip_lm_param_offsets(const lhip_lm_config_t* cfg, long long* offsets, int* rows, int* cols)
{
    if (int rc = lhip::check_dims(cfg)) return rc;
    const int D = cfg->dim, F = cfg->ffn, V = cfg->vocab;
    long long off = 0;
    int idx = 0;
    auto add = [&](int r, int c) {
        if (offsets) offsets[idx] = off;
        if (rows) rows[idx] = r;
        if (cols) cols[idx] = c;
        off += static_cast<long long>(r) * c;
        ++idx;
    };
    add(V, D);
    for (int l = 0; l < cfg->layers; ++l) {
        add(1, D); add(D, D); add(D, D); add(D, D); add(D, D);
        add(1, D); add(D, F); add(D, F); add(F, D);
    }
    add(1, D);
    return LHIP_OK;
}

LHIP_API int lhip_lm_create(const lhip_lm_config_t* cfg, void** model)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_create: model is NULL");
    *model = nullptr;
    if (int rc = lhip::check_config(cfg)) return rc;
    auto* m = new (std::nothrow) lhip::LmModel();
    if (!m) return fail(LHIP_E_OOM, "lhip_lm_create: host allocation");
    m->c = *cfg;
    m->D = cfg->dim; m->F = cfg->ffn; m->V = cfg->vocab; m->H = cfg->heads; m->L = cfg->layers;
    m->T = cfg->seq; m->B = cfg->batch; m->hd = m->D / m->H; m->N = m->B * m->T;
    m->nparam = lhip::count_params(*cfg);
    const int ntens = 2 + lhip::P_PER_LAYER * m->L;
    m->off.resize(ntens);
    lhip_lm_param_offsets(cfg, m->off.data(), nullptr, nullptr);

    const long long N = m->N, D = m->D, F = m->F, V = m->V, L = m->L;
    const long long ND = N * D, NF = N * F, PL = static_cast<long long>(m->B) * m->H * m->T * m->T;
    m->ss_blocks = lhip::sumsq_blocks(m->nparam);
    m->ss_cap = std::max(m->ss_blocks, 4096);
    // dw partials of one norm backward: the stand-alone kernel's, or one row per 16-row tile when fused
    m->work_floats = static_cast<size_t>(std::max(lhip::rmsnorm_bwd_parts(m->N, m->D), lhip::ceil_div(m->N, 16))) *
                     m->D;
    m->splitk_floats = static_cast<size_t>(1) << 22;   // 16 MiB; the planner caps splits to fit
    // carve every buffer out of one allocation, each 256-byte aligned
    struct Slot { void** dst; size_t bytes; };
    std::vector<Slot> slots = {
        {reinterpret_cast<void**>(&m->params), sizeof(float) * m->nparam},
        {reinterpret_cast<void**>(&m->grads), sizeof(float) * m->nparam},
        {reinterpret_cast<void**>(&m->vel), sizeof(float) * m->nparam},
        {reinterpret_cast<void**>(&m->ids), sizeof(int) * N},
        {reinterpret_cast<void**>(&m->tgt), sizeof(int) * N},
        {reinterpret_cast<void**>(&m->amax), sizeof(int) * N},
        {reinterpret_cast<void**>(&m->wlen), sizeof(int) * m->B},
        {reinterpret_cast<void**>(&m->applied), sizeof(int) * 4},
        {reinterpret_cast<void**>(&m->losses), sizeof(float) * N},
        {reinterpret_cast<void**>(&m->gnorm), sizeof(float) * 4},
        {reinterpret_cast<void**>(&m->hyper), sizeof(float) * 16},
        {reinterpret_cast<void**>(&m->adam_m), sizeof(float) * m->nparam},
        {reinterpret_cast<void**>(&m->adam_v), sizeof(float) * m->nparam},
        {reinterpret_cast<void**>(&m->tcount), sizeof(int) * 4},
        {reinterpret_cast<void**>(&m->ss), sizeof(double) * 2},
        {reinterpret_cast<void**>(&m->ss_part), sizeof(double) * m->ss_cap},
        {reinterpret_cast<void**>(&m->x), sizeof(float) * (L + 1) * ND},
        {reinterpret_cast<void**>(&m->h), sizeof(float) * L * ND},
        {reinterpret_cast<void**>(&m->inv1), sizeof(float) * L * N},
        {reinterpret_cast<void**>(&m->qkv), sizeof(float) * L * 3 * ND},
        {reinterpret_cast<void**>(&m->P), sizeof(float) * L * PL},
        {reinterpret_cast<void**>(&m->ctx), sizeof(float) * L * ND},
        {reinterpret_cast<void**>(&m->xmid), sizeof(float) * L * ND},
        {reinterpret_cast<void**>(&m->h2), sizeof(float) * L * ND},
        {reinterpret_cast<void**>(&m->inv2), sizeof(float) * L * N},
        {reinterpret_cast<void**>(&m->zu), sizeof(float) * L * 2 * NF},
        {reinterpret_cast<void**>(&m->a), sizeof(float) * L * NF},
        {reinterpret_cast<void**>(&m->xf), sizeof(float) * ND},
        {reinterpret_cast<void**>(&m->invf), sizeof(float) * N},
        {reinterpret_cast<void**>(&m->logits), sizeof(float) * N * V},
        {reinterpret_cast<void**>(&m->dxf), sizeof(float) * ND},
        {reinterpret_cast<void**>(&m->gx), sizeof(float) * (L + 1) * ND},
        {reinterpret_cast<void**>(&m->gmid), sizeof(float) * L * ND},
        {reinterpret_cast<void**>(&m->da), sizeof(float) * NF},
        {reinterpret_cast<void**>(&m->dzu), sizeof(float) * L * 2 * NF},
        {reinterpret_cast<void**>(&m->dh2), sizeof(float) * ND},
        {reinterpret_cast<void**>(&m->dctx), sizeof(float) * ND},
        {reinterpret_cast<void**>(&m->dP), sizeof(float) * PL},
        {reinterpret_cast<void**>(&m->dS), sizeof(float) * PL},
        {reinterpret_cast<void**>(&m->dqkv), sizeof(float) * L * 3 * ND},
        {reinterpret_cast<void**>(&m->dh), sizeof(float) * ND},
        {reinterpret_cast<void**>(&m->work), sizeof(float) * (2 * L + 1) * m->work_floats},
        {reinterpret_cast<void**>(&m->splitk), sizeof(float) * m->splitk_floats},
        {reinterpret_cast<void**>(&m->rope_cs), sizeof(float2) * m->T * (m->hd / 2)},
    };
    size_t total = 0;
    for (auto& sl : slots) total += (sl.bytes + 255) & ~static_cast<size_t>(255);
    hipError_t e = hipMalloc(&m->arena, total);
    if (e != hipSuccess) {
        delete m;
        return fail(LHIP_E_OOM, "lhip_lm_create: %zu bytes of device memory: %s", total, hipGetErrorString(e));
    }
    m->arena_bytes = total;
    char* p = static_cast<char*>(m->arena);
    for (auto& sl : slots) {
        *sl.dst = p;
        p += (sl.bytes + 255) & ~static_cast<size_t>(255);
    }
    // zero state: params, grads, velocity, ids (a fresh model is all zeros until set_params)
    int rc = lhip::zero_bytes(m->arena, total, st().stream);
    if (rc == LHIP_OK) {
        hipError_t se = hipStreamSynchronize(st().stream);
        if (se != hipSuccess) rc = lhip::hip_fail(se, "lhip_lm_create: sync");
    }
    if (rc != LHIP_OK) {
        (void)hipFree(m->arena);
        delete m;
        return rc;
    }
    // RoPE table for positions 0..T-1: angle = t / base^(2p/hd) in double, as
    // build_rope (transformer.lua:30-48), rounded to fp32 once
    {
        const int pairs = m->hd / 2;
        std::vector<float2> tab(static_cast<size_t>(m->T) * pairs);
        for (int p = 0; p < pairs; ++p) {
            const double inv = 1.0 / std::pow(cfg->rope_base, static_cast<double>(2 * p) / m->hd);
            for (int t = 0; t < m->T; ++t) {
                const double ang = t * inv;
                tab[static_cast<size_t>(t) * pairs + p] =
                    make_float2(static_cast<float>(std::cos(ang)), static_cast<float>(std::sin(ang)));
            }
        }
        hipError_t ue = hipMemcpy(m->rope_cs, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice);
        if (ue != hipSuccess) {
            (void)hipFree(m->arena);
            delete m;
            return lhip::hip_fail(ue, "lhip_lm_create: rope table");
        }
    }
    m->fused_attn = lhip::attn_fused_ok(m->T, m->hd);
    m->fused_gemm = lhip::lm_fuse_ok(m->D, m->D, m->D) && m->F % 4 == 0;
    m->h_tgt.assign(static_cast<size_t>(N), 0);
    m->h_len.assign(static_cast<size_t>(m->B), 0);
    *model = m;
    return LHIP_OK;
}

LHIP_API int lhip_lm_destroy(void* model)
{
    if (!model) return LHIP_OK;
    if (st().ready) LHIP_REFUSE_RECORDING();
    auto* m = lhip::as_model(model);
    if (st().ready) {
        (void)hipStreamSynchronize(st().stream);
        lhip::release(*m);
    }
    delete m;
    return LHIP_OK;
}

static int lm_copy(void* model, float* host, long long n, int which, int to_device)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model || !host) return fail(LHIP_E_NULL, "lhip_lm: NULL argument");
    auto* m = lhip::as_model(model);
    if (n != m->nparam) return fail(LHIP_E_SHAPE, "lhip_lm: %lld values given, model has %lld", n, m->nparam);
    float* d = which == 0 ? m->params : (which == 1 ? m->grads : m->vel);
    const size_t bytes = static_cast<size_t>(n) * sizeof(float);
    hipError_t e = to_device ? hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, st().stream)
                             : hipMemcpyAsync(host, d, bytes, hipMemcpyDeviceToHost, st().stream);
    if (e != hipSuccess) return lhip::hip_fail(e, "lhip_lm: copy");
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "lhip_lm: sync");
    return LHIP_OK;
}

LHIP_API int lhip_lm_set_params(void* model, const float* host, long long n)
{
    return lm_copy(model, const_cast<float*>(host), n, 0, 1);
}

LHIP_API int lhip_lm_get_params(void* model, float* host, long long n) { return lm_copy(model, host, n, 0, 0); }

LHIP_API int lhip_lm_get_grads(void* model, float* host, long long n) { return lm_copy(model, host, n, 1, 0); }

LHIP_API int lhip_lm_set_velocity(void* model, const float* host, long long n)
{
    return lm_copy(model, const_cast<float*>(host), n, 2, 1);
}

LHIP_API int lhip_lm_get_velocity(void* model, float* host, long long n) { return lm_copy(model, host, n, 2, 0); }

LHIP_API int lhip_lm_set_batch_ex(void* model, const int* ids, const int* targets, const int* lengths,
                                  int n_windows)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model || !ids || !targets) return fail(LHIP_E_NULL, "lhip_lm_set_batch: NULL argument");
    auto* m = lhip::as_model(model);
    if (n_windows < 1 || n_windows > m->B)
        return fail(LHIP_E_SHAPE, "lhip_lm_set_batch: %d windows for %d slots", n_windows, m->B);
    std::vector<int> len(static_cast<size_t>(m->B), 0);
    bool short_batch = n_windows < m->B;
    for (int b = 0; b < n_windows; ++b) {
        len[b] = lengths ? lengths[b] : m->T;
        if (len[b] < 1 || len[b] > m->T)
            return fail(LHIP_E_SHAPE, "lhip_lm_set_batch: window %d has %d tokens, outside [1, %d]", b, len[b], m->T);
        short_batch = short_batch || len[b] < m->T;
    }
    // Rows past a window's length (and empty slots) carry id 0, which keeps
    // their forward finite, and target -1, which the CE turns into a zero
    // loss and a zero gradient; with the causal mask, or the key limit of the
    // fused attention, no counted row sees them.
    if (short_batch && !m->c.causal && !m->fused_attn)
        return fail(LHIP_E_UNSUPPORTED, "lhip_lm_set_batch: short windows in a non-causal model with seq %d or "
                    "head_dim %d past the fused attention's limits", m->T, m->hd);
    std::vector<int> hid(static_cast<size_t>(m->N), 0), htg(static_cast<size_t>(m->N), -1);
    for (int b = 0; b < n_windows; ++b) {
        for (int t = 0; t < len[b]; ++t) {
            const size_t i = static_cast<size_t>(b) * m->T + t;
            if (ids[i] < 0 || ids[i] >= m->V)
                return fail(LHIP_E_ARG, "lhip_lm_set_batch: ids[%zu] = %d outside [0, %d)", i, ids[i], m->V);
            if (targets[i] < 0 || targets[i] >= m->V)
                return fail(LHIP_E_ARG, "lhip_lm_set_batch: targets[%zu] = %d outside [0, %d)", i, targets[i], m->V);
            hid[i] = ids[i];
            htg[i] = targets[i];
        }
    }
    const size_t bytes = static_cast<size_t>(m->N) * sizeof(int);
    hipStream_t s = st().stream;
    LHIP_CHECK_HIP(hipMemcpyAsync(m->ids, hid.data(), bytes, hipMemcpyHostToDevice, s), "lhip_lm_set_batch: ids");
    LHIP_CHECK_HIP(hipMemcpyAsync(m->tgt, htg.data(), bytes, hipMemcpyHostToDevice, s), "lhip_lm_set_batch: targets");
    LHIP_CHECK_HIP(hipMemcpyAsync(m->wlen, len.data(), sizeof(int) * m->B, hipMemcpyHostToDevice, s),
                   "lhip_lm_set_batch: lengths");
    LHIP_CHECK_HIP(hipStreamSynchronize(s), "lhip_lm_set_batch: sync");
    m->h_tgt = htg;
    m->h_len = len;
    m->nwin = n_windows;
    m->have_batch = true;
    return LHIP_OK;
}

LHIP_API int lhip_lm_set_batch(void* model, const int* ids, const int* targets)
{
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_set_batch: NULL argument");
    return lhip_lm_set_batch_ex(model, ids, targets, nullptr, lhip::as_model(model)->B);
}

LHIP_API int lhip_lm_use_graph(void* model, int on)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_use_graph: model is NULL");
    auto* m = lhip::as_model(model);
    m->use_graph = on != 0;
    if (!m->use_graph) {
        (void)hipStreamSynchronize(st().stream);
        lhip::drop_graph(*m);
    }
    return LHIP_OK;
}

LHIP_API int lhip_lm_step_sgd(void* model, float lr, float momentum, float weight_decay, float clip_norm,
                              int nesterov)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_step_sgd: model is NULL");
    auto* m = lhip::as_model(model);
    if (!m->have_batch) return fail(LHIP_E_ARG, "lhip_lm_step_sgd: no batch (call lhip_lm_set_batch)");
    if (!(lr >= 0.f) || !(momentum >= 0.f) || !(weight_decay >= 0.f) || !(clip_norm >= 0.f))
        return fail(LHIP_E_ARG, "lhip_lm_step_sgd: lr, momentum, weight_decay and clip_norm must be >= 0");
    lhip::Hyper hp{};
    hp.lr = lr; hp.momentum = momentum; hp.wd = weight_decay; hp.clip = clip_norm;
    hp.nesterov = nesterov ? 1.f : 0.f;
    hp.opt = lhip::OPT_SGD;
    return lhip::run_step(*m, hp);
}

LHIP_API int lhip_lm_step_adamw(void* model, float lr, float beta1, float beta2, float eps, float weight_decay,
                                float clip_norm)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_step_adamw: model is NULL");
    auto* m = lhip::as_model(model);
    if (!m->have_batch) return fail(LHIP_E_ARG, "lhip_lm_step_adamw: no batch (call lhip_lm_set_batch)");
    if (!(lr >= 0.f) || !(beta1 >= 0.f && beta1 < 1.f) || !(beta2 >= 0.f && beta2 < 1.f) || !(eps >= 0.f) ||
        !(weight_decay >= 0.f) || !(clip_norm >= 0.f))
        return fail(LHIP_E_ARG, "lhip_lm_step_adamw: lr, eps, weight_decay, clip_norm >= 0 and betas in [0, 1)");
    lhip::Hyper hp{};
    hp.lr = lr; hp.wd = weight_decay; hp.clip = clip_norm;
    hp.beta1 = beta1; hp.beta2 = beta2; hp.eps = eps;
    hp.parity = static_cast<float>(m->adam_calls & 1);
    hp.opt = lhip::OPT_ADAMW;
    return lhip::run_step(*m, hp);
}

LHIP_API int lhip_lm_save(void* model, const char* path, const lhip_ckpt_info_t* info)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_save: model is NULL");
    auto* m = lhip::as_model(model);
    return lhip::lm_checkpoint_io(m->c, m->params, path, info, nullptr, true);
}

LHIP_API int lhip_lm_load(void* model, const char* path, lhip_ckpt_header_t* header)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_load: model is NULL");
    auto* m = lhip::as_model(model);
    return lhip::lm_checkpoint_io(m->c, m->params, path, nullptr, header, false);
}

LHIP_API int lhip_lm_set_adam_state(void* model, const float* mom, const float* var, long long n, int step)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_set_adam_state: model is NULL");
    auto* m = lhip::as_model(model);
    if (n != m->nparam) return fail(LHIP_E_SHAPE, "lhip_lm_set_adam_state: %lld values given, model has %lld", n,
                                    m->nparam);
    if (step < 0) return fail(LHIP_E_ARG, "lhip_lm_set_adam_state: step %d < 0", step);
    hipStream_t s = st().stream;
    const size_t bytes = static_cast<size_t>(n) * sizeof(float);
    if (mom) LHIP_CHECK_HIP(hipMemcpyAsync(m->adam_m, mom, bytes, hipMemcpyHostToDevice, s), "set_adam_state: m");
    if (var) LHIP_CHECK_HIP(hipMemcpyAsync(m->adam_v, var, bytes, hipMemcpyHostToDevice, s), "set_adam_state: v");
    // the slot the next AdamW step reads
    int* slot = m->tcount + (m->adam_calls & 1);
    LHIP_CHECK_HIP(hipMemcpyAsync(slot, &step, sizeof(int), hipMemcpyHostToDevice, s), "set_adam_state: step");
    LHIP_CHECK_HIP(hipStreamSynchronize(s), "set_adam_state: sync");
    return LHIP_OK;
}

LHIP_API int lhip_lm_get_adam_state(void* model, float* mom, float* var, long long n, int* step)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model) return fail(LHIP_E_NULL, "lhip_lm_get_adam_state: model is NULL");
    auto* m = lhip::as_model(model);
    if (n != m->nparam) return fail(LHIP_E_SHAPE, "lhip_lm_get_adam_state: %lld values asked, model has %lld", n,
                                    m->nparam);
    hipStream_t s = st().stream;
    const size_t bytes = static_cast<size_t>(n) * sizeof(float);
    if (mom) LHIP_CHECK_HIP(hipMemcpyAsync(mom, m->adam_m, bytes, hipMemcpyDeviceToHost, s), "get_adam_state: m");
    if (var) LHIP_CHECK_HIP(hipMemcpyAsync(var, m->adam_v, bytes, hipMemcpyDeviceToHost, s), "get_adam_state: v");
    int t = 0;
    LHIP_CHECK_HIP(hipMemcpyAsync(&t, m->tcount + (m->adam_calls & 1), sizeof(int), hipMemcpyDeviceToHost, s),
                   "get_adam_state: step");
    LHIP_CHECK_HIP(hipStreamSynchronize(s), "get_adam_state: sync");
    if (step) *step = t;
    return LHIP_OK;
}

LHIP_API int lhip_lm_stats(void* model, lhip_lm_stats_t* out, float* window_losses, int nwin)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model || !out) return fail(LHIP_E_NULL, "lhip_lm_stats: NULL argument");
    auto* m = lhip::as_model(model);
    if (window_losses && nwin != m->B)
        return fail(LHIP_E_SHAPE, "lhip_lm_stats: %d window slots given, batch is %d", nwin, m->B);
    std::vector<float> losses(static_cast<size_t>(m->N));
    std::vector<int> am(static_cast<size_t>(m->N));
    float gn = 0.f;
    int applied = 0;
    hipStream_t s = st().stream;
    LHIP_CHECK_HIP(hipMemcpyAsync(losses.data(), m->losses, losses.size() * sizeof(float), hipMemcpyDeviceToHost, s),
                   "lhip_lm_stats: losses");
    LHIP_CHECK_HIP(hipMemcpyAsync(am.data(), m->amax, am.size() * sizeof(int), hipMemcpyDeviceToHost, s),
                   "lhip_lm_stats: argmax");
    LHIP_CHECK_HIP(hipMemcpyAsync(&gn, m->gnorm, sizeof(float), hipMemcpyDeviceToHost, s), "lhip_lm_stats: norm");
    LHIP_CHECK_HIP(hipMemcpyAsync(&applied, m->applied, sizeof(int), hipMemcpyDeviceToHost, s),
                   "lhip_lm_stats: applied");
    LHIP_CHECK_HIP(hipStreamSynchronize(s), "lhip_lm_stats: sync");
    // each window's mean over its own tokens (Tensor.cross_entropy), then the
    // batch loss LMTrain reports: sum_w loss_w * len_w / sum_w len_w
    // (lmtrain.lua:1197-1198,1233-1234); empty slots report 0
    double total = 0.0;
    long long tokens = 0;
    for (int b = 0; b < m->B; ++b) {
        const int len = m->h_len[b];
        double w = 0.0;
        for (int t = 0; t < len; ++t) w += losses[static_cast<size_t>(b) * m->T + t];
        if (len > 0) w /= len;
        if (window_losses) window_losses[b] = static_cast<float>(w);
        total += w * len;
        tokens += len;
    }
    int correct = 0;
    for (int i = 0; i < m->N; ++i) correct += am[i] == m->h_tgt[i];
    out->loss = static_cast<float>(tokens > 0 ? total / tokens : 0.0);
    out->grad_norm = gn;
    out->applied = applied;
    out->correct = correct;
    out->steps = m->steps;
    return LHIP_OK;
}

LHIP_API int lhip_lm_get_argmax(void* model, int* host, int n)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!model || !host) return fail(LHIP_E_NULL, "lhip_lm_get_argmax: NULL argument");
    auto* m = lhip::as_model(model);
    if (n != m->N) return fail(LHIP_E_SHAPE, "lhip_lm_get_argmax: n=%d, batch*seq=%d", n, m->N);
    LHIP_CHECK_HIP(hipMemcpyAsync(host, m->amax, sizeof(int) * n, hipMemcpyDeviceToHost, st().stream), "argmax copy");
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "lhip_lm_get_argmax: sync");
    return LHIP_OK;
}

}  // extern "C"
