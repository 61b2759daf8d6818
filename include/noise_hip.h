/* C ABI of libnoise_hip.so: the MI355X (gfx950) population-perturbed forward of the Noise 37.7M GPT
 * and the EGGROLL update (fitness -> gradient estimate -> Adam).
 *
 * Conventions for every entry point:
 *  - pointers are device pointers (hipMalloc / torch CUDA tensors); bf16 buffers are passed as void*;
 *  - "members" are the population rows; member p uses perturbation row dir = p >> pair_shift
 *    (pair_shift = 1 when antithetic pairs 2j, 2j+1 share a_j, b_j, as train/val/eggroll.py:140-141
 *    builds them; 0 when a, b are given per member, as population_loss receives them) and
 *    sign[p] = +-sigma (train/val/eggroll.py:138);
 *  - rank-1 vectors follow the reference orientation (train/val/eggroll.py:56-63): for a weight
 *    W [out, in], `a` is [dirs, out] (output side) and `b` is [dirs, in] (input side); for an
 *    embedding W [V, d], `a` is [dirs, V] and `b` is [dirs, d];
 *  - activations are row-major [members * T, width]; member p owns rows p*T .. p*T+T-1; width 512
 *    (d_model) unless stated;
 *  - work is enqueued on `stream` (a hipStream_t); nothing is synchronised, nothing allocated: any
 *    scratch comes from the caller's workspace, sized by the matching *_workspace_size query;
 *  - return 0 on success, a negative NOISE_E* code for a rejected argument, or a positive hipError_t.
 */
#ifndef NOISE_HIP_H
#define NOISE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NOISE_OK 0
#define NOISE_EINVAL (-1)
#define NOISE_ENOSPC (-2)
#define NOISE_ENOTSUP (-3)

#define NOISE_FITNESS_ZSCORE 0 /* train/val/eggroll.py:151-152 */
#define NOISE_FITNESS_RANK 1   /* centred ranks, ties by index (config-4 option) */

/* Reductions of noise_head_ce's per-token losses. */
#define NOISE_CE_MEMBER_MEAN 0 /* loss[members]: mean over each member's T tokens (train/val/eggroll.py:101-102) */
#define NOISE_CE_NONE 1        /* loss[members*T] per token, 0 where the target is -1 (utils/model.py:205-208) */
#define NOISE_CE_SUM 2         /* loss[1]: sum over the tokens whose target is not -1 */
#define NOISE_CE_MEAN 3        /* loss[1]: that sum over their count (NaN when none is valid) */

/* Head formats of noise_head_ce (its fp32_head argument). */
#define NOISE_HEAD_BF16 0       /* w_head bf16 [vocab, 512]: the reference's autocast head (one bf16 GEMM) */
#define NOISE_HEAD_FP32_SPLIT 1 /* w_head bf16 [vocab, 1536] from noise_cast_bf16(split_cols = 512): fp32 head as three
                                 * bf16 products, ~2^-16 relative */
#define NOISE_HEAD_FP32 2       /* w_head fp32 [vocab, 512] (16-byte aligned): fp32 head as two fp16 products, h
                                 * rounded once to fp16 (11 significant bits, TF32's) against a 22-bit split of
                                 * the weight */

typedef void* noise_stream_t; /* hipStream_t */

/* Layouts of a bf16 activation [rows, cols] exchanged between entry points. */
#define NOISE_LAYOUT_ROWS 0   /* row-major, cols contiguous (the reference's tensor layout) */
#define NOISE_LAYOUT_TILE16 1 /* 1 KiB tiles of 16 rows x 32 cols (rows % 16 == 0, cols % 32 == 0): element
                               * (r, c) at (r/16)*16*cols + (c/32)*512 + 8*p + c%8 with
                               * p = 4*(r%16) + (((c%32)/8) ^ (((r%16)/2) % 4)). Same footprint as ROWS; a
                               * producer writes and the GEMM loads it as whole 128-byte lines. */
#define NOISE_LAYOUT_WTILE 2  /* a bf16 weight W [rows = out, cols = in] (rows % 64 == 0, cols % 32 == 0) in the
                               * order of the tile GEMM's 32-deep stages: the 1 KiB block (g, s) at element
                               * (g*cols/32 + s)*512 holds cols 32s .. 32s+31 of the 16 rows with tiled index
                               * i = 16g + r (r < 16), row r being weight row
                               * (i - i%64) + (r/4)*16 + ((i%64)/16)*4 + r%4, its 16-byte chunk c at
                               * c ^ ((r/2) % 4). Same footprint as ROWS; written by noise_weight_tiles. */

/* A c_proj output not yet added to the residual stream (a deferred residual): row r of member p receives
 *   y[r, c] + sign[p] * bf16(sum_{q < u_parts} u[r * u_row_stride + q * u_part_stride]) * a[dir * 512 + c]
 * with y = bf16(x W^T) from noise_dense_bf16: `x = x + linear(name, x_in)` of train/val/eggroll.py:92-93 with
 * the rank-1 term of `lowrank` (:56-58) applied where the residual stream is next read. y, a 16-byte
 * aligned; 1 <= u_parts <= 64. */
typedef struct noise_pending {
  const void* y;            /* bf16 [members*T, 512] */
  const float* u;           /* input-side dot partials of the c_proj input */
  int u_parts;
  long u_row_stride;
  long u_part_stride;
  const float* a;           /* [dirs, 512] output-side vectors of the c_proj weight */
} noise_pending_t;

/* Library version (major * 10000 + minor * 100 + patch). */
int noise_version(void);

/* ---------------------------------------------------------------- rank-1 perturbed linears */

/* y = x W^T + s_p (x . b_p) a_p^T per member, autocast rounding points: bf16 GEMM output, the GEMV
 * x.b rounded to bf16, the correction added in fp32.
 * Replaces `lowrank` (train/val/eggroll.py:56-58).
 *   x       bf16 [members, T, in], row r of member p at x + p*x_mstride + t*x_ld (x_mstride 0: one
 *           activation shared by every member); in % 64 == 0, out % 128 == 0
 *   w       bf16 [out, in]
 *   y_f32   fp32 [members*T, out] (nullable); accumulate != 0 adds into it (residual update)
 *   y_bf16  bf16 [members*T, out] (nullable)
 * Workspace: noise_lowrank_linear_workspace_size(). */
int noise_lowrank_linear_workspace_size(int members, int T, size_t* bytes);
int noise_lowrank_linear(const void* x, long x_ld, long x_mstride, const void* w, int in, int out,
                         const float* a, const float* b, const float* sign, int members, int T, int pair_shift,
                         float* y_f32, void* y_bf16, int accumulate, void* workspace, size_t workspace_bytes,
                         noise_stream_t stream);

/* The relu^2 MLP sublayer with rank-1 perturbations on both matrices, per member:
 *   h = relu(lowrank(x, w_fc, a_fc, b_fc))^2 ;  y = lowrank(h, w_proj, a_proj, b_proj)
 * Replaces `F.relu(linear('mlp.c_fc.weight', .)).square()` -> `linear('mlp.c_proj.weight', .)`
 * (train/val/eggroll.py:93; model form utils/model.py:106-107).
 *   x       bf16 [members, T, d] (x_mstride as above)
 *   w_fc    bf16 [f, d];  a_fc [dirs, f], b_fc [dirs, d]
 *   w_proj  bf16 [d, f];  a_proj [dirs, d], b_proj [dirs, f]
 *   y_f32 / y_bf16 / accumulate as in noise_lowrank_linear; d == 512, f % 256 == 0, T % 32 == 0.
 * Workspace: noise_lowrank_mlp_workspace_size() (the hidden, its dot partials and a WTILE copy of w_proj, made
 * on every call). */
int noise_lowrank_mlp_workspace_size(int members, int T, int d, int f, size_t* bytes);
int noise_lowrank_mlp(const void* x, long x_ld, long x_mstride, const void* w_fc, const void* w_proj, int d, int f,
                      const float* a_fc, const float* b_fc, const float* a_proj, const float* b_proj,
                      const float* sign, int members, int T, int pair_shift, float* y_f32, void* y_bf16,
                      int accumulate, void* workspace, size_t workspace_bytes, noise_stream_t stream);

/* ---------------------------------------------------------------- population forward, per stage
 * The stages below compose `population_loss` (train/val/eggroll.py:66-103) block by block; the host
 * (noise_amd/population.py) calls them in the reference's order. */

/* fp32 -> bf16 cast of n values (weights, once per step). split_cols > 0 writes the fp32-head
 * operand instead: each row of split_cols values becomes [bf16(w) | bf16(w - bf16(w)) | bf16(w)]
 * (out holds 3 n values). */
int noise_cast_bf16(const float* in, void* out, long n, int split_cols, noise_stream_t stream);

/* x0 = norm(W[idx] + s_p a_p[idx] b_p) fp32 [members*T, 512].
 * Replaces `norm(lowrank_embed(p['transformer.wte.weight'], ...))` (train/val/eggroll.py:61-63, :74). */
int noise_embed_norm(const float* w, long vocab, const float* a, const float* b, const float* sign,
                     const int64_t* idx, int members, int T, int pair_shift, float* x0, noise_stream_t stream);

/* Block entry: x_out = (lambda_r + s eps_r[dir]) x_in + (lambda_0 + s eps_0[dir]) x0; h = bf16(norm(x_out));
 * lambda_r / lambda_0 point at this block's entries of resid_lambdas / x0_lambdas (device memory);
 * u_qkv[row, 0..2] = bf16(h . bf16(b_{q,k,v}[dir])), u_qkv[row, 3] = sign[member] (row stride 4: the row
 * noise_qkv reads); when gate_w is not null the value
 * gate gate[row, 0..7] = 2 sigmoid(lowrank(h[:32], gate_w, gate_a, gate_b)) (gate_w [8, 32] and gate_b
 * [dirs, 32] 16-byte aligned).
 * Replaces train/val/eggroll.py:76-84, :88. eps_r / eps_0 point at this block's column of the
 * [dirs, n_layer] lambda noise (row stride eps_ld). x_out may alias x_in. The npend (<= 2) deferred
 * residuals in pend (the previous block's attention and MLP c_proj outputs) are added to x_in, in order,
 * before the mix. */
/* The embedding a block entry recomputes x0 from: x0 = norm(w[idx] + s a[dir, idx] b[dir]), the same
 * arithmetic as noise_embed_norm (bit-identical rows). Member p reads the token ids idx[p * idx_mstride ..
 * + T): idx_mstride 0 for one sequence shared by all members (population_loss), T for one sequence per
 * member (GPT.forward's batch rows, utils/model.py:193-196). */
typedef struct noise_embed {
  const float* w; /* [vocab, 512] */
  long vocab;
  const float* a; /* [dirs, vocab] */
  const float* b; /* [dirs, 512] */
  const int64_t* idx;
  long idx_mstride;
} noise_embed_t;
/* x0 may be null when x0_embed is given (x0 rows recomputed: no stored [members*T, 512] fp32 x0 stream);
 * x_in may be null at block 0 (x_in = x0). */
int noise_block_entry(const float* x_in, const float* x0, float* x_out, void* h, float* u_qkv, const float* b_q,
                      const float* b_k, const float* b_v, const float* lambda_r, const float* lambda_0, const float* eps_r,
                      const float* eps_0, long eps_ld, const float* gate_w, const float* gate_a,
                      const float* gate_b, float* gate, const float* sign, int members, int T, int pair_shift,
                      const noise_pending_t* pend, int npend, const noise_embed_t* x0_embed, noise_stream_t stream);

/* q | k | v = lowrank(h, [W_q; W_k; W_v]) with per-segment a vectors and the u_qkv dots, then rotary +
 * QK RMSNorm on q and k (utils/model.py:55-58, :46-47; train/val/eggroll.py:90) and, when gate is not
 * null, v += gate * (ve_w[idx] + s a_ve[idx] b_ve) (train/val/eggroll.py:85-89), member p reading the
 * token ids idx[p * idx_mstride .. + T] (0: one shared sequence; T: a sequence per member). Output
 * [members*T, 1536] fp16 (q | k | v, head h at columns h*64 of each segment), each rounded once from the
 * fp32 value the reference feeds flex attention (train/val/eggroll.py:58, :90-91), q multiplied by
 * log2(e) / 8 first (the softmax's score scale in base-2 units): the operand format NOISE_QK_F16_Q_LOG2 of
 * noise_attention. |v| must stay below 65504 (fp16's largest finite value).
 *   w_qkv    bf16 [1536, 512] = c_q ; c_k ; c_v
 *   rot_cos / rot_sin  bf16 [>= T, 32] (utils/model.py:177-183) */
/*   u_qkv    [members*T, 4] as noise_block_entry writes it (dots with b_q, b_k, b_v; the member's sign) */
int noise_qkv(const void* h, const void* w_qkv, const float* a_q, const float* a_k, const float* a_v,
              const float* u_qkv, const float* sign, int members, int T, int pair_shift, const void* rot_cos,
              const void* rot_sin, const float* gate, const float* ve_w, long vocab, const float* ve_a,
              const float* ve_b, const int64_t* idx, long idx_mstride, void* qkv, noise_stream_t stream);

/* q | k formats of noise_attention. */
#define NOISE_QK_BF16 0       /* q, k bf16 (the credit reruns' moved heads, train/val/run.py:186-189) */
#define NOISE_QK_F16 1        /* q, k fp16 */
#define NOISE_QK_F16_Q_LOG2 2 /* q, k fp16 with q pre-multiplied by log2(e) / 8, as noise_qkv writes them (qk_norm != 0) */
#define NOISE_QK_BF16_V_BF16 3 /* q, k and v bf16, probabilities rounded to bf16 for P V (qk_norm != 0): torch's
                                 * attention on bf16 operands, as GPT.forward runs it under autocast in
                                 * utils/eval.py:44-45 (flex on bf16 q, k, v, utils/model.py:31) */

/* Windowed causal attention on q | k | v rows of [members*T, 1536] 16-bit values (8 heads x 64): q and k in
 * qk_format (NOISE_QK_*); v fp16 (bf16 for NOISE_QK_BF16_V_BF16).
 * y bf16 [members*T, 512]; a query at s
 * sees keys s - window .. s (utils/model.py:14-31). When b_proj is not null, writes the c_proj
 * input-side dot partials upart [members*T, 8]. When mom is not null, writes per-(member, head)
 * means over tokens of y and y^2, mom [members, 8, 2, 64] ("credit moments"; no reference
 * function), using mom_work (noise_attention_workspace_size bytes). T % 128 == 0.
 * qk_norm != 0 declares that q and k rows are RMS-normalised (norm(q), norm(k) at train/val/eggroll.py:90,
 * as noise_qkv writes them): every score is then bounded by 8.03 and the softmax runs without a running
 * maximum; qk_norm == 0 accepts any q, k. */
int noise_attention_workspace_size(int members, int T, size_t* bytes);
int noise_attention(const void* qkv, int members, int T, int window, int qk_norm, int qk_format, const float* b_proj,
                    int pair_shift, void* y, float* upart, float* mom, void* mom_work, size_t mom_work_bytes,
                    noise_stream_t stream);

/* noise_attention without a workspace argument: no counterpart in the reference. It is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The moments' partials go to a library-owned device array of NOISE_ATTENTION_NOALLOC_MAX_PARTIALS floats
 * (16 MiB, one copy per GPU, held until the process ends), so with mom != null the call needs
 * members * (T / 128) * 8 * 128 <= NOISE_ATTENTION_NOALLOC_MAX_PARTIALS (P = 256 members at T = 2048 fits) and
 * returns NOISE_ENOSPC beyond it, before any GPU work. It calls no hipMalloc / hipFree. Calls that overlap on one
 * GPU share that array and race: serialise them (one stream, or events). Results equal noise_attention's. */
#define NOISE_ATTENTION_NOALLOC_MAX_PARTIALS (4 * 1024 * 1024)
int noise_attention_noalloc(const void* qkv, int members, int T, int window, int qk_norm, int qk_format,
                            const float* b_proj, int pair_shift, void* y, float* upart, float* mom,
                            noise_stream_t stream);

/* resid += lowrank(x, w) with the input-side dot of row r given as u_parts partial sums
 * u[r * u_row_stride + q * u_part_stride]: the attention c_proj (u from noise_attention: row stride 8,
 * part stride 1) and the MLP c_proj (u from noise_mlp_fc: row stride 1, part stride members*T).
 * Replaces `x = x + linear('attn.c_proj.weight', y)` (train/val/eggroll.py:92) and the MLP's
 * `x = x + linear('mlp.c_proj.weight', ...)` (:93). */
int noise_lowrank_resid(const void* x, const void* w, int in, int out, const float* a, const float* u, int u_parts,
                        long u_row_stride, long u_part_stride, const float* sign, int members, int T, int pair_shift,
                        float* resid, noise_stream_t stream);

/* The NOISE_LAYOUT_WTILE copy of a row-major bf16 weight w [rows, cols] into out (rows * cols bf16): the
 * per-step layout change of a GEMM weight, like the bf16 cast of train/val/eggroll.py:144's autocast done
 * once per step. rows % 64 == 0, cols % 32 == 0, 16-byte aligned pointers. */
int noise_weight_tiles(const void* w, int rows, int cols, void* out, noise_stream_t stream);

/* y = bf16(x W^T) [members*T, out] for x bf16 [members*T, in] (x_layout NOISE_LAYOUT_ROWS or
 * NOISE_LAYOUT_TILE16), w bf16 [out, in] (w_layout NOISE_LAYOUT_ROWS or NOISE_LAYOUT_WTILE, the layout the
 * K > 512 tile GEMM loads fastest): the dense product of a c_proj `lowrank` whose rank-1 term and residual
 * add are deferred to the row kernel that next reads the stream (noise_pending_t). in % 64 == 0,
 * out % 128 == 0; TILE16 also T % 16 == 0. */
int noise_dense_bf16(const void* x, int x_layout, int in, int out, const void* w, int w_layout, int members, int T,
                     void* y, noise_stream_t stream);

/* The clean forward's residual stream at the rounding points GPT.forward has under torch's bf16 autocast with bf16
 * embedding tables, as the speedrun's scorer runs it (utils/eval.py:44-45 on utils/model.py:193-210, tables bf16
 * per :171-175). Rows r = b * T + t of batch row b: every tensor is bf16 and every op rounds to bf16.
 *   x = x_in, or x0 = bf16(norm(wte[idx])) when x_in is null (:196-197; rms_norm of a bf16 input computes in
 *       fp32 with eps 2^-23 and casts back)
 *   x = bf16(x + y1), then bf16(x + y2) for the non-null block outputs y1, y2 (the residual adds of :118-119)
 *   x = bf16(bf16(bf16(l_r) x) + bf16(bf16(l_0) x0)) when lambda_r is not null (:199; the 0-d fp32 lambdas
 *       are cast to bf16 by type promotion against the bf16 stream)
 *   x_out = x (nullable); h = bf16(norm(x)) (nullable)
 *   gate = 2 bf16(sigmoid(bf16(h[:32] . bf16(gate_w)^T))) [rows, 8] when gate_w [8, 32] is not null (:89)
 * wte [vocab, 512] fp32 holding bf16 values; idx: row (b, t) reads idx[b * idx_mstride + t]. x_in, y1, y2,
 * x_out, h bf16 [rows, 512], 16-byte aligned. */
int noise_ac_stream(const void* x_in, const float* wte, long vocab, const int64_t* idx, long idx_mstride,
                    const void* y1, const void* y2, const float* lambda_r, const float* lambda_0, void* x_out, void* h,
                    const float* gate_w, float* gate, int rows, int T, noise_stream_t stream);

/* q | k | v [rows, 1536] bf16 (the bf16 outputs of c_q, c_k, c_v under autocast) updated in place as
 * utils/model.py:83-94 treats them under torch's bf16 autocast: q and k rotated with bf16 tables, every product
 * and sum rounded to bf16 (:55-58, :93), then norm per 64-dim head, bf16 out (:94); when gate is not null,
 * v = bf16(v + bf16(gate[row, head] ve_w[tok])) (:88-90, :200) with ve_w [vocab, 512] fp32 holding bf16 values.
 * The output is noise_attention's NOISE_QK_BF16_V_BF16 operand. */
int noise_ac_qkv(void* qkv, const void* rot_cos, const void* rot_sin, const float* gate, const float* ve_w,
                 long vocab, const int64_t* idx, long idx_mstride, int rows, int T, noise_stream_t stream);

/* h = bf16(norm(x)); u[row] = bf16(h . bf16(b[dir])) (MLP entry, train/val/eggroll.py:93). The npend (<= 2)
 * deferred residuals in pend are added to x, in order, before the norm; x itself is not written. */
int noise_norm_dot(const float* x, void* h, const float* b, float* u, const float* sign, int members, int T,
                   int pair_shift, const noise_pending_t* pend, int npend, noise_stream_t stream);

/* hidden = bf16(relu(lowrank(h, w_fc))^2) [members*T, f] in hidden_layout (NOISE_LAYOUT_ROWS or
 * NOISE_LAYOUT_TILE16, the layout noise_dense_bf16 loads fastest) and its dot partials with bf16(b_proj),
 * part-major: upart [noise_mlp_fc_parts(f), members*T] (one partial per 256 columns), for the
 * following noise_lowrank_resid or deferred residual. d == 512, f % 256 == 0, T % 32 == 0 (NOISE_ENOTSUP
 * otherwise). */
int noise_mlp_fc_parts(int f);
int noise_mlp_fc(const void* h, const void* w_fc, int d, int f, const float* a_fc, const float* u,
                 const float* b_proj, const float* sign, int members, int T, int pair_shift, void* hidden,
                 int hidden_layout, float* upart, noise_stream_t stream);

/* Soft-capped cross-entropy of the head (train/val/eggroll.py:94-103; utils/model.py:202-208): h = norm(x)
 * (times gain when gain is not null: the config-3 extension; null reproduces utils/model.py:46-47);
 * z = h W^T + s (h . b) a; z' = 15 tanh(z / 15); the token loss logsumexp(z'_t) - z'_t[target_t] reduced by
 * `reduction` (NOISE_CE_*) into loss: the per-member mean of population_loss, or F.cross_entropy's
 * 'none' / 'sum' / 'mean' with ignore_index = -1 (GPT.forward). Member p's targets are
 * targets[p * tgt_mstride .. + T]. When logits is not null the capped logits z' are also written, fp32
 * [members*T, vocab] (GPT.forward without targets); targets and loss may then both be null.
 *   x       [members*T, 512] fp32 (x_bf16 == 0) or bf16 (x_bf16 != 0)
 *   gain    [512] fp32 or null
 *   fp32_head  NOISE_HEAD_*: the format of w_head and the precision of z (the fp32 formats keep the dot h . b
 *              and the rank-1 term in fp32; NOISE_HEAD_BF16 follows the reference's autocast rounding points).
 * vocab % 256 == 0. Workspace: noise_head_ce_workspace_size(). The npend (<= 2) deferred residuals in
 * pend are added to an fp32 x, in order, before the norm (the last block's c_proj outputs). */
int noise_head_ce_workspace_size(int members, int T, int vocab, int fp32_head, size_t* bytes);
int noise_head_ce(const void* x, int x_bf16, const float* gain, const void* w_head, int vocab, int fp32_head,
                  const float* a, const float* b, const float* sign, const int64_t* targets, long tgt_mstride,
                  int members, int T, int pair_shift, int reduction, float* loss, float* logits, void* workspace,
                  size_t workspace_bytes, const noise_pending_t* pend, int npend, noise_stream_t stream);

/* Readout-probe forward differences (train/val/run.py:154-185, `cycle_derivatives` and `row_derivatives`):
 * for token i (logits base_i = W x_i [vocab], |x_i|^2 = sq[i], target targets[i], step steps[i]) and each of
 * its K directions j (dirs row j = W D_j, x_i . D_j = dots[i, k], |D_j|^2 = dir_sq), out[i, k] = (L_ij - L_i0) /
 * steps[i], L the soft-capped cross-entropy of the head on norm(x_i + steps[i] D_j) (its RMS from sq, dots and
 * dir_sq) and L_i0 on norm(x_i); 0 where the target is -1. rows null: every direction, K == P, dir_sq [P]
 * (cycle_derivatives); rows [n, K] int64: the token's own directions, dir_sq [n, K] with dir_sq_per_token != 0
 * (row_derivatives); a row outside [0, P) gives NaN at its entry (no read outside dirs). fp32; vocab % 256 == 0,
 * vocab <= 4096; width is the stream width of the RMS. */
int noise_readout_probes(const float* base, long base_ld, const float* dirs, long dirs_ld, const int64_t* rows, int K,
                         const int64_t* targets, const float* steps, const float* sq, const float* dots, long dots_ld,
                         const float* dir_sq, int dir_sq_per_token, int n, int vocab, int P, int width, float* out,
                         noise_stream_t stream);

/* Credit scoring around batched attention reruns (train/val/run.py:186-211, used by query_key_errors :594-634),
 * 64-dim heads, draws j, batch b, position t, head h:
 * noise_moved_heads: out row (j, b, t), head h = bf16(norm(rotary(raw[b, t, h] + sigma a[j, b, t, h]))) in fp32
 *   (`moved_heads`, :186-189; rotary of utils/model.py:55-58 with fp32 tables [>= T, 32]); raw fp32
 *   [batch, T, heads, 64], a bf16 [draws, batch, T, heads, 64], out bf16 rows of out_ld elements.
 * noise_head_scores: score[b, h, t, j] = sum_d (out[j, b, t, h, d] - baseline[b, t, h, d]) hub[b, t, h, d]
 *   (`head_scores`, :192-195); out bf16 rows of out_ld elements (noise_attention's y), baseline and hub fp32.
 * noise_code_estimate: est[b, t, h, d] = sum_j credited[b, h, t, j] a[j, b, t, h, d] (`code_estimate`,
 *   :208-210), fp32 out, draws summed in order. */
int noise_moved_heads(const float* raw, const void* a, float sigma, const float* rot_cos, const float* rot_sin, int draws,
                      int batch, int T, int heads, void* out, long out_ld, noise_stream_t stream);
int noise_head_scores(const void* out, long out_ld, const float* baseline, const float* hub, int draws, int batch, int T,
                      int heads, float* score, noise_stream_t stream);
int noise_code_estimate(const float* credited, const void* a, int draws, int batch, int T, int heads, float* est,
                        noise_stream_t stream);
/* noise_key_filter: the key scores of query_key_errors (train/val/run.py:622-623), (K.to(bf16) @ score.to(bf16)).float()
 *   per (b, h): out[b, h, t, j] = bf16(sum_s bf16(K[b, h, t, s]) bf16(score[b, h, s, j])) with fp32 accumulation;
 *   filter bf16 [batch, heads, T, T] (16-byte aligned), score and out fp32 [batch, heads, T, draws]; T % 64 == 0. */
int noise_key_filter(const void* filter, const float* score, int batch, int heads, int T, int draws, float* out,
                     noise_stream_t stream);

/* ---------------------------------------------------------------- EGGROLL update */

/* fitness[j] = L[2j+1] - L[2j] transformed by mode (z-score: divided by the unbiased std + 1e-8, no
 * centering; rank: centred ranks); weight[d] = sum of fitness[j] over j = d mod pairs.
 * Replaces train/val/eggroll.py:151-154. n = number of losses (even, >= 4). */
int noise_fitness(const float* losses, int n, int pairs, int mode, float* fitness, float* weight,
                  noise_stream_t stream);

/* grad[o, i] = scale * sum_j (w_j a_j[o]) b_j[i] over ndir directions; a null means out == 1 and
 * a_j = 1 (the lambda noise). Replaces the update loop of train/val/eggroll.py:155-166 with
 * scale = -1 / len(fitness). */
int noise_outer_update(const float* a, long a_ld, const float* b, long b_ld, const float* w, int ndir, int out,
                       int in, float scale, float* grad, noise_stream_t stream);

/* noise_outer_update for n matrices in one launch (every perturbed parameter of the model shares the
 * direction weights w and ndir): mats is a host array, read before the call returns. Same arithmetic per
 * matrix; replaces the per-parameter loop of train/val/eggroll.py:155-166. */
typedef struct noise_outer_mat {
  const float* a; /* [ndir, a_ld] or null (out == 1) */
  long a_ld;
  const float* b; /* [ndir, b_ld] */
  long b_ld;
  int out;
  int in;
  float* grad; /* [out, in] */
} noise_outer_mat_t;
int noise_outer_update_batch(const noise_outer_mat_t* mats, int n, const float* w, int ndir, float scale,
                             noise_stream_t stream);

/* The perturbation rows of a set of directions, gathered from the shared N(0, 1) noise buffer: for every
 * parameter k and direction j, the slice buffer[offsets_k[directions[j]] .. + out_k + in_k] split into
 * a_k[j, :out_k] and b_k[j, :in_k] (in_k == 0 and b_k null for a 1-D parameter's eps rows). Replaces
 * Eggroll.noise (train/val/eggroll.py:122-128): one launch for every parameter. params is a host array,
 * read before the call returns; offsets are [pairs] int64 device arrays. A direction outside [0, pairs) or
 * a slice outside the buffer writes NaN rows. */
typedef struct noise_gather_param {
  const int64_t* offsets;
  float* a;
  float* b;
  int out;
  int in;
} noise_gather_param_t;
int noise_gather_rows(const float* buffer, long buffer_len, const noise_gather_param_t* params, int nparams,
                      const int64_t* directions, int ndir, int pairs, noise_stream_t stream);

/* One torch.optim.AdamW step with weight_decay 0 on n fp32 values (train/val/eggroll.py:205, :167):
 * step_size = lr / (1 - beta1^t), bc2_sqrt = sqrt(1 - beta2^t). */
int noise_adam(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, long n, float step_size,
               float beta1, float beta2, float eps, float bc2_sqrt, noise_stream_t stream);

/* HBM streaming calibration (no counterpart in the reference): each of `rows` rows reads in_kib KiB of src and writes
 * out_kib KiB of dst (1..4 KiB each, 16-byte aligned buffers), one wave per row with the row kernels' 16-byte vector
 * accesses. It measures the bandwidth ceiling of a row kernel's read / write mix (bench.py --workload stream). */
int noise_hbm_stream(const void* src, int in_kib, void* dst, int out_kib, long rows, noise_stream_t stream);

/* noise_adam for every tensor of an optimizer step in one launch (torch.optim.AdamW's per-parameter loop,
 * train/val/eggroll.py:167): tensors is a host array, read before the call returns; each entry carries its own
 * step_size and bc2_sqrt (its own step count). Same arithmetic per element as noise_adam. */
typedef struct noise_adam_tensor {
  float* param;
  const float* grad;
  float* exp_avg;
  float* exp_avg_sq;
  long n;
  float step_size;
  float bc2_sqrt;
} noise_adam_tensor_t;
int noise_adam_batch(const noise_adam_tensor_t* tensors, int n, float beta1, float beta2, float eps,
                     noise_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* NOISE_HIP_H */
