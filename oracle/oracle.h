/*
 * oracle.h -- CPU restatement of lanternl's pure-Lua CPU path, in double precision.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (lanternl_amd/, the HIP
 * library, bench.py's measured leg) may call, link or load this code.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker (or as the timed CPU stand-in for the LuaJIT path).
 *
 * Each function follows the reference loop it cites (path:line under the
 * reference tree).  Conventions:
 *   - row-major, 0-based indices (Lua is 1-based: a Lua id t is t-1 here);
 *   - all arithmetic in double, no FMA contraction (built with
 *     -ffp-contract=off), in the same loop order as the Lua code;
 *   - "accumulate" outputs add into the destination like the Lua BACKWARD.*
 *     functions do (grad_of(...) += ...).
 *
 * How each function is pinned (the checks live in tests/test_oracle.py):
 *   or_mm / or_matmul_nt / or_matmul_tn : reference known answers
 *       (tests/core_test.lua:31-34, tests/test.lua:445-449), numpy float64 '@',
 *       (AB)^T = B^T A^T, zero-skip NaN semantics (tests/core_test.lua:95-100).
 *   or_rmsnorm_*      : central finite differences (tests/test.lua:209-243 pattern).
 *   or_softmax_*      : rows sum to 1, mask exact zeros, equal logits -> 1/n
 *                       (tests/core_test.lua:48-51), closed-form bwd
 *                       (tests/test.lua:184-205), finite differences.
 *   or_silu_* / or_swiglu_* : closed forms (tests/test.lua:245-275), finite diff.
 *   or_rope_*         : identity at pos 0 (tests/core_test.lua:88-92),
 *                       bwd = inverse rotation (tests/test.lua:277-289), norm
 *                       preservation, angle formula vs numpy.
 *   or_cross_entropy* : CE([2,1,0.1], t=1) = 0.41703 (tests/core_test.lua:54-57),
 *                       dlogits rows sum to 0 (tests/test.lua:347-355), finite diff.
 *   or_argmax_rows    : argmax({1,9,2;8,3,4}) = {1,0} (tests/test.lua:375-379),
 *                       ties/NaN/-inf brute force.
 *   or_embed_*        : scatter of ids {3,0,7,3,1} (tests/test.lua:291-320).
 *   or_sgd_step / or_grad_norm : closed forms; l2(3,4)=25 (tests/test.lua:157-164).
 *   or_adamw_step     : closed forms (no reference test holds AdamW vectors):
 *                       constant gradient g gives m/bc1 = g, v/bc2 = g^2 at every
 *                       t, so each step is p(1-lr*wd) - lr*g/(|g|+eps); zero
 *                       gradient gives p(1-lr*wd)^t; moments vs their recurrences.
 *   or_lm_*           : float64 torch.autograd of the same model (independent
 *                       derivative), finite differences on a tiny model, ln V at
 *                       near-uniform logits.
 *   or_ew             : sigmoid against scipy's expit, tanh/exp/sqrt against
 *                       numpy, silu'/gelu' against central differences of
 *                       silu/gelu, the tanh-form GELU within 1e-3 of x*Phi(x)
 *                       (its published accuracy), each binary operator on
 *                       hand-picked values.
 *   or_gemm_ex        : numpy float64 products of explicitly transposed,
 *                       batched copies; the RMSNorm prologue against
 *                       or_rmsnorm_fwd then '@'; activations against
 *                       scipy/numpy; beta == 0 with NaN in C.
 *   or_softmax_ex / or_softmax_bwd_ex : scipy softmax of the kept prefix,
 *                       all-zero rows when nothing is kept, equality with
 *                       or_softmax_fwd/bwd where their contracts coincide,
 *                       central differences for the backward.
 *   or_rmsnorm_bwd_luatl : or_rmsnorm_bwd with 1/rms recomputed (pinned
 *                       above), dgamma accumulation, gamma NULL = ones.
 *   or_adamw_luatl    : constant-gradient closed form (every step is
 *                       w(1-lr*wd) - lr*g/(|g|+eps)), the clamp, moments vs
 *                       their recurrences.
 *   or_reduce_cols / or_clip_by_nsq : numpy column sums; the clip's fixed
 *                       point (norm after = max_norm*nrm/(nrm+1e-6)).
 */
#ifndef LANTERNL_ORACLE_H
#define LANTERNL_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---- GEMM family: ai/core/matrix.lua ---------------------------------- */
/* r(m x n) = a(m x k) . b(k x n); i-p-j order, skips a==0 terms
 * (matrix.lua:514-539).  acc != 0 adds into r (matrix.multiply(..., acc)). */
void or_mm(const double* a, const double* b, double* r, int m, int k, int n, int acc);
/* r(m x n) = a(m x k) . b(n x k)^T; dot-product order p=1..k (matrix.lua:597-625). */
void or_matmul_nt(const double* a, const double* b, double* r, int m, int k, int n, int acc);
/* r(k x n) = a(m x k)^T . b(m x n); i-p-j order, skips a==0 (matrix.lua:627-660). */
void or_matmul_tn(const double* a, const double* b, double* r, int m, int k, int n, int acc);

/* ---- RMSNorm: ai/core/tensor2.lua:609-666 ------------------------------ */
void or_rmsnorm_fwd(const double* x, const double* w, double* out, double* inv,
                    int rows, int cols, double eps);
/* accumulates xg (rows x cols) and wg (cols) */
void or_rmsnorm_bwd(const double* x, const double* w, const double* inv, const double* g,
                    double* xg, double* wg, int rows, int cols);

/* ---- row softmax: ai/core/tensor2.lua:332-408 -------------------------- */
/* causal: row i (0-based) keeps columns 0..min(i+offset, cols-1), at least 1. */
void or_softmax_fwd(const double* x, double* y, int rows, int cols, int causal, int offset);
void or_softmax_bwd(const double* y, const double* g, double* xg, int rows, int cols,
                    int causal, int offset);

/* ---- SiLU / SwiGLU: tensor2.lua:167-183 (mul), 272-303 (silu) ----------- */
void or_silu_fwd(const double* x, double* y, double* sig, long n);
void or_silu_bwd(const double* x, const double* sig, const double* g, double* xg, long n);
/* h = silu(gate) * up, composed as at ai/nn/transformer.lua:246-248 */
void or_swiglu_fwd(const double* gate, const double* up, double* h, long n);
/* accumulates dgate, dup (BACKWARD.mul then BACKWARD.silu) */
void or_swiglu_bwd(const double* gate, const double* up, const double* dh,
                   double* dgate, double* dup, long n);

/* ---- RoPE: angles ai/nn/transformer.lua:30-48 (= ai/core/rope.lua:24-56),
 *      rotation ai/core/tensor2.lua:410-473 (interleaved pairs) ---------- */
/* cosv/sinv are (maxpos+1) x npairs, npairs = hd/2 */
void or_rope_angles(double base, int hd, int maxpos, double* cosv, double* sinv);
/* row i uses cosr[i*npairs ...]; columns past 2*npairs are copied */
void or_rope_fwd(const double* x, double* y, int rows, int cols,
                 const double* cosr, const double* sinr, int npairs);
void or_rope_bwd(const double* g, double* xg, int rows, int cols,
                 const double* cosr, const double* sinr, int npairs);
/* Multi-head in-place RoPE with the luaTL_rope contract (cuda/luaTL_train.cu:719-767):
 * pos = pos_ids ? pos_ids[r] : r + pos_offset; freq = theta^(-2p/hd);
 * interleaved: pairs (2p, 2p+1), else half-split (p, p+hd/2); inverse negates sin. */
void or_rope_heads(double* x, const int* pos_ids, int rows, int heads, int hd,
                   int row_stride, int pos_offset, double theta, int interleaved, int inverse);

/* ---- cross-entropy: ai/core/tensor2.lua:809-882 ------------------------ */
/* Returns the mean loss over counted rows; tgt is 0-based; rows whose target
 * equals ignore_index (when has_ignore) are skipped.  sm receives the softmax
 * (zeros for ignored rows); *count receives the (>=1) divisor. */
double or_cross_entropy(const double* logits, const int* tgt, int rows, int cols,
                        int has_ignore, int ignore_index, double* sm, int* count);
/* lg += (sm - onehot) * (g / count) for non-ignored rows */
void or_cross_entropy_bwd(const double* sm, const int* tgt, int rows, int cols,
                          int has_ignore, int ignore_index, double g, int count, double* lg);
/* Fused per-row contract of luaTL_cross_entropy (cuda/luaTL_train.cu:837-891):
 * rows with t<0, t>=V or t==ignore_index get loss 0 and dlogits 0; otherwise
 * losses[r] = logsumexp - x[t], dlogits = gscale*(softmax - onehot). */
void or_ce_fused(const double* logits, const int* tgt, double* losses, double* dlogits,
                 int rows, int vocab, int ignore_index, double gscale);

/* ---- argmax: ai/optim/lmtrain.lua:1200-1209 --------------------------- */
/* strict '>' scan from -inf: first maximum wins, NaN never wins, a row of
 * only NaN/-inf gives 0 (Lua's best_id = 1). */
void or_argmax_rows(const double* x, int* out, int rows, int cols);

/* ---- embedding: ai/core/tensor2.lua:572-607 ---------------------------- */
void or_embed_fwd(const double* w, const int* ids, double* out, int n, int dim);
void or_embed_bwd(const double* g, const int* ids, double* wg, int n, int dim, double scale);

/* ---- optimizer: ai/optim/optim2.lua ------------------------------------ */
double or_grad_norm(const double* g, long n);                 /* :27-38 */
void   or_scale(double* g, long n, double f);                 /* :40-46 */
void   or_sgd_step(double* p, const double* g, double* v, long n,
                   double lr, double momentum, double wd, int nesterov);  /* :72-99 */
/* AdamW.step with the step count already advanced to t (>= 1)  :116-147 */
void   or_adamw_step(double* p, const double* g, double* m, double* v, long n,
                     double lr, double b1, double b2, double eps, double wd, int t);

/* ---- the CPU LMTrain step: ai/nn/transformer.lua:84-257 +
 *      ai/optim/lmtrain.lua:1183-1227 --------------------------------- */
typedef struct {
    int vocab, dim, layers, heads, ffn;
    int causal;          /* transformer.lua:93 (default true) */
    double eps;          /* transformer.lua:98 (1e-5) */
    double rope_base;    /* transformer.lua:95 (10000) */
} or_lm_cfg;

/* Number of parameters, in Transformer:parameters() order (transformer.lua:150-164,
 * tied head, RoPE): emb, {ln1, wq, wk, wv, wo, ln2, w1, w3, w2} x layers, lnf. */
long or_lm_num_params(const or_lm_cfg* c);
/* Offsets (in doubles) of each parameter tensor in that order; returns the count
 * of tensors (2 + 9*layers).  offs may be NULL. */
int  or_lm_param_offsets(const or_lm_cfg* c, long* offs, int* rows, int* cols);

/* One window: forward, CE (mean over T), backward with seed 1; ACCUMULATES
 * into grads (params are leaves).  logits (T x vocab) optional.  Returns loss.
 * ids/tgt are 0-based.  *correct (optional) += argmax hits. */
double or_lm_window(const or_lm_cfg* c, const double* params, const int* ids, const int* tgt,
                    int T, double* grads, double* logits, int* correct);

/* One LMTrain batch step with optimizer="sgd": zero grads, run every window,
 * scale_grads(1/B) when B>1, global grad norm, skip if non-finite, clip to
 * clip_norm, SGD(lr, momentum, wd).  ids/tgt are B x T, 0-based.
 * Outputs: losses[B] per-window mean loss, *gnorm (pre-clip norm), *correct,
 * grads (final gradients handed to SGD, i.e. after scale and clip).
 * Returns 1 if the step was applied, 0 if skipped (non-finite norm). */
int or_lm_step_sgd(const or_lm_cfg* c, double* params, double* vel,
                   const int* ids, const int* tgt, int B, int T,
                   double lr, double momentum, double wd, double clip_norm,
                   double* losses, double* gnorm, int* correct, double* grads);

/* The same over a ragged batch: windows b < nwin (nwin <= B; the short last
 * batch), window b holding lens[b] <= T tokens at ids/tgt + b*T (lens NULL:
 * T each; build_windows' short last window, lmtrain.lua:535-558); each
 * window's loss is its own mean and the summed grads are scaled by 1/nwin. */
int or_lm_step_sgd_ex(const or_lm_cfg* c, double* params, double* vel,
                      const int* ids, const int* tgt, int nwin, int T, const int* lens,
                      double lr, double momentum, double wd, double clip_norm,
                      double* losses, double* gnorm, int* correct, double* grads);
int or_lm_step_adamw_ex(const or_lm_cfg* c, double* params, double* m, double* v, int* t,
                        const int* ids, const int* tgt, int nwin, int T, const int* lens,
                        double lr, double b1, double b2, double eps, double wd, double clip_norm,
                        double* losses, double* gnorm, int* correct, double* grads);

/* The same step with optimizer="adamw": *t (the AdamW step count) is advanced
 * and the AdamW update applied only when the norm is finite.  m, v: moments. */
int or_lm_step_adamw(const or_lm_cfg* c, double* params, double* m, double* v, int* t,
                     const int* ids, const int* tgt, int B, int T,
                     double lr, double b1, double b2, double eps, double wd, double clip_norm,
                     double* losses, double* gnorm, int* correct, double* grads);

/* ---- the luaTL operation set (the reference GPU path's kernels, restated
 *      in double for the adapter's resident calls and Program ops) ------- */
/* c[i] = op(a[i], b[i], alpha, beta) with luaTL's operator table
 * (cuda/luaTL_core.cu:49-72, 909-934); a or b NULL read as 0; GELU in the
 * tanh form of cuda/luaTL_core.cu:370-383. */
void or_ew(int op, const double* a, const double* b, double* c, long n, double alpha, double beta);
/* luaTL_gemm_ex_kernel (cuda/luaTL_train.cu:127-234): strided, batched,
 * C = act(alpha * pre(A).B + bias) + beta*C; pre 1 = RMSNorm of A's rows
 * (rowscale given, else 1/sqrt(mean a^2 + eps)) times gamma[k]; pre 2-4 =
 * gelu/silu/relu of a; beta == 0 does not read C. */
void or_gemm_ex(const double* A, const double* B, double* C, const double* bias, const double* gamma,
                const double* rowscale, int M, int N, int K, long a_rs, long a_cs, long b_rs, long b_cs,
                long c_rs, long c_cs, long a_bs, long b_bs, long c_bs, int batch, double alpha, double beta,
                double eps, int pre_op, int post_op);
/* luaTL_softmax_ex_kernel (cuda/luaTL_train.cu:545-585): v = x*scale + bias[j]
 * over j <= limit, limit = (group>0 ? r%group : r) + moff when causal, else
 * cols-1; masked 0; nothing kept -> all 0. */
void or_softmax_ex(const double* x, const double* bias, double* y, int rows, int cols, double scale,
                   int causal, int group, int moff);
/* luaTL_softmax_bwd_kernel (cuda/luaTL_train.cu:589-619), dx overwritten. */
void or_softmax_bwd_ex(const double* y, const double* dy, double* dx, int rows, int cols, double scale,
                       int causal, int group, int moff);
/* luaTL_rmsnorm_bwd_kernel (cuda/luaTL_train.cu:489-526): s from x and eps,
 * dx overwritten, dgamma (may be NULL) accumulated, gamma NULL = 1. */
void or_rmsnorm_bwd_luatl(const double* x, const double* g, const double* dy, double* dx, double* dgamma,
                          int rows, int cols, double eps);
/* luaTL_adamw_kernel (cuda/luaTL_core.cu:1346-1380) with bc1 = 1/(1-b1^t),
 * bc2 = 1/(1-b2^t), t = max(step, 1) (cuda/luaTL_train.cu:1427-1449). */
void or_adamw_luatl(double* w, const double* g, double* m, double* v, long n, int step, double lr,
                    double b1, double b2, double eps, double wd, double clip);
/* out[c] = alpha * sum_r x[r*rs + c] + beta * out[c] (cuda/luaTL_train.cu:895-906) */
void or_reduce_cols(const double* x, double* out, int rows, int cols, long rs, double alpha, double beta);
/* x *= max_norm/(sqrt(nsq)+1e-6) when sqrt(nsq) > max_norm > 0 (cuda/luaTL_train.cu:947-965) */
void or_clip_by_nsq(double* x, long n, double nsq, double max_norm);

#ifdef __cplusplus
}
#endif
#endif
