// extern "C" entry points of libnoise_hip.so (declared in include/noise_hip.h).
#include <mutex>
#include <vector>

#include "../../include/noise_hip.h"
#include "attention.h"
#include "autocast.h"
#include "common.h"
#include "credit.h"
#include "eggroll.h"
#include "gemm.h"
#include "probes.h"
#include "rowops.h"

static_assert(NOISE_QK_BF16 == QK_BF16 && NOISE_QK_F16 == QK_F16 && NOISE_QK_F16_Q_LOG2 == QK_F16_Q_LOG2 &&
                  NOISE_QK_BF16_V_BF16 == QK_BF16_V_BF16,
              "q/k format codes");
static_assert(NOISE_CE_MEMBER_MEAN == CE_MEMBER_MEAN && NOISE_CE_NONE == CE_NONE && NOISE_CE_SUM == CE_SUM &&
                  NOISE_CE_MEAN == CE_MEAN,
              "reduction codes");

// The moment partials of noise_attention_noalloc live in this library-owned device array: every GPU the library
// runs on holds its own copy (16 MiB) until the process ends. In host code `scratch` only names the symbol, not a
// device address: its address on the current GPU comes from hipGetSymbolAddress, looked up once per device
// (scratch_address below), and only that address is passed to kernels.
static_assert(NOISE_ATTENTION_NOALLOC_MAX_PARTIALS % 64 == 0, "scratch size");
static __device__ __align__(256) float scratch[NOISE_ATTENTION_NOALLOC_MAX_PARTIALS];

namespace {

// Bump allocator over the caller's workspace (256-byte aligned slices).
struct Carve {
  char* base;
  size_t used = 0;
  explicit Carve(void* b) : base(static_cast<char*>(b)) {}
  template <class T>
  T* take(size_t count) {
    T* p = base ? reinterpret_cast<T*>(base + used) : nullptr;
    used += (count * sizeof(T) + 255) & ~size_t(255);
    return p;
  }
};

constexpr int DM = 512, NH = 8;

LowrankGemmArgs base_args(const void* x, long x_ld, long x_mstride, const void* w, int in, int out, const float* a,
                          const float* sign, int members, int T, int pair_shift) {
  LowrankGemmArgs g{};
  g.A = static_cast<const bf16*>(x);
  g.lda = x_ld;
  g.a_mstride = x_mstride;
  g.W = static_cast<const bf16*>(w);
  g.ldw = in;
  g.M = members * T;
  g.N = out;
  g.K = in;
  g.T = T;
  g.pair_shift = pair_shift;
  g.sign = sign;
  g.ra[0] = a;
  g.seg_n = out;
  g.ra_ld = out;
  g.u_qstride = 1;
  g.round_bf16 = 1;
  return g;
}

// Copies the C-ABI deferred residuals into the row kernels' descriptors (npend validated by the launch).
int copy_pending(const noise_pending_t* src, int npend, Pending* dst) {
  if (npend < 0 || npend > MAX_PENDING || (npend > 0 && !src)) return NOISE_EINVAL;
  for (int k = 0; k < npend; ++k)
    dst[k] = Pending{static_cast<const bf16*>(src[k].y), src[k].u, src[k].u_parts, src[k].u_row_stride,
                     src[k].u_part_stride, src[k].a};
  return NOISE_OK;
}

bool bad_members(int members, int T, int pair_shift) {
  return members <= 0 || T <= 0 || pair_shift < 0 || pair_shift > 1 || (long)members * T > 0x7fffffffL;
}

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_dev[MAX_DEVICES];

// The device address of `scratch` on the current device (looked up on this device's first call).
int scratch_address(void** out) {
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev)) return (int)e;
  if (dev < 0 || dev >= MAX_DEVICES) return NOISE_ENOTSUP;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_dev[dev]) {
    void* p = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) return (int)e;
    if (!p) return NOISE_ENOTSUP;
    scratch_dev[dev] = p;
  }
  *out = scratch_dev[dev];
  return NOISE_OK;
}

}  // namespace

extern "C" {

int noise_version(void) { return 200; }

int noise_lowrank_linear_workspace_size(int members, int T, size_t* bytes) {
  if (members <= 0 || T <= 0 || !bytes) return NOISE_EINVAL;
  Carve c(nullptr);
  c.take<float>((size_t)members * T);
  *bytes = c.used;
  return NOISE_OK;
}

int noise_lowrank_linear(const void* x, long x_ld, long x_mstride, const void* w, int in, int out, const float* a,
                         const float* b, const float* sign, int members, int T, int pair_shift, float* y_f32,
                         void* y_bf16, int accumulate, void* workspace, size_t workspace_bytes,
                         noise_stream_t stream) {
  size_t need = 0;
  if (int rc = noise_lowrank_linear_workspace_size(members, T, &need)) return rc;
  if (bad_members(members, T, pair_shift)) return NOISE_EINVAL;
  if (!workspace || workspace_bytes < need) return NOISE_ENOSPC;
  if (accumulate && (!y_f32 || y_bf16)) return NOISE_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carve c(workspace);
  float* u = c.take<float>((size_t)members * T);
  const int M = members * T;
  if (int rc = rowdot_launch(static_cast<const bf16*>(x), x_ld, x_mstride, M, in, T, pair_shift, b, in, u, s))
    return rc;
  LowrankGemmArgs g = base_args(x, x_ld, x_mstride, w, in, out, a, sign, members, T, pair_shift);
  g.u = u;
  g.u_parts = 1;
  g.u_ld = 1;
  g.out_f32 = y_f32;
  g.out_bf16 = static_cast<bf16*>(y_bf16);
  g.ldo = out;
  return lowrank_gemm_launch(accumulate ? EPI_RESID : EPI_STORE, g, s);
}

int noise_lowrank_mlp_workspace_size(int members, int T, int d, int f, size_t* bytes) {
  if (members <= 0 || T <= 0 || d <= 0 || f <= 0 || !bytes || !xs_relu2_parts(f)) return NOISE_EINVAL;
  const size_t M = (size_t)members * T;
  Carve c(nullptr);
  c.take<float>(M);                            // u_fc
  c.take<float>(M * xs_relu2_parts(f));        // partial dots h.b_proj, part-major
  c.take<bf16>(M * f);                         // hidden h
  c.take<bf16>((size_t)d * f);                 // w_proj in the tile GEMM's WTILE layout
  *bytes = c.used;
  return NOISE_OK;
}

int noise_lowrank_mlp(const void* x, long x_ld, long x_mstride, const void* w_fc, const void* w_proj, int d, int f,
                      const float* a_fc, const float* b_fc, const float* a_proj, const float* b_proj,
                      const float* sign, int members, int T, int pair_shift, float* y_f32, void* y_bf16,
                      int accumulate, void* workspace, size_t workspace_bytes, noise_stream_t stream) {
  size_t need = 0;
  if (int rc = noise_lowrank_mlp_workspace_size(members, T, d, f, &need)) return rc;
  if (bad_members(members, T, pair_shift)) return NOISE_EINVAL;
  if (!workspace || workspace_bytes < need) return NOISE_ENOSPC;
  if (accumulate && (!y_f32 || y_bf16)) return NOISE_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t M = (size_t)members * T;
  Carve c(workspace);
  float* u_fc = c.take<float>(M);
  const int parts = xs_relu2_parts(f);
  float* upart = c.take<float>(M * parts);
  bf16* hid = c.take<bf16>(M * f);
  bf16* wpt = c.take<bf16>((size_t)d * f);
  if (int rc = rowdot_launch(static_cast<const bf16*>(x), x_ld, x_mstride, (int)M, d, T, pair_shift, b_fc, d, u_fc, s))
    return rc;
  LowrankGemmArgs g1 = base_args(x, x_ld, x_mstride, w_fc, d, f, a_fc, sign, members, T, pair_shift);
  g1.u = u_fc;
  g1.u_parts = 1;
  g1.u_ld = 1;
  g1.out_bf16 = hid;
  g1.ldo = f;
  g1.out_tiled = 1;  // the hidden never leaves the library: TILE16, whole-line stores and loads
  g1.rb_next = b_proj;
  g1.rb_next_ld = f;
  g1.upart_out = upart;
  g1.upart_ld = parts;
  if (int rc = lowrank_gemm_launch(EPI_RELU2, g1, s)) return rc;
  // c_proj loads both operands as whole 128-byte lines: the hidden in TILE16, w_proj copied into WTILE
  if (int rc = weight_tiles_launch(static_cast<const bf16*>(w_proj), f, d, f, wpt, s)) return rc;
  LowrankGemmArgs g2 = base_args(hid, f, (long)T * f, wpt, f, d, a_proj, sign, members, T, pair_shift);
  g2.a_tiled = 1;
  g2.w_tiled = 1;
  g2.u = upart;
  g2.u_parts = parts;
  g2.u_ld = 1;
  g2.u_qstride = (long)M;
  g2.out_f32 = y_f32;
  g2.out_bf16 = static_cast<bf16*>(y_bf16);
  g2.ldo = d;
  return lowrank_gemm_launch(accumulate ? EPI_RESID : EPI_STORE, g2, s);
}

int noise_cast_bf16(const float* in, void* out, long n, int split_cols, noise_stream_t stream) {
  return cast_launch(in, static_cast<bf16*>(out), n, split_cols, split_cols > 0, static_cast<hipStream_t>(stream));
}

int noise_embed_norm(const float* w, long vocab, const float* a, const float* b, const float* sign,
                     const int64_t* idx, int members, int T, int pair_shift, float* x0, noise_stream_t stream) {
  if (bad_members(members, T, pair_shift)) return NOISE_EINVAL;
  EmbedNormArgs g{w, a, b, vocab, sign, idx, members * T, T, pair_shift, x0};
  return embed_norm_launch(g, static_cast<hipStream_t>(stream));
}

int noise_block_entry(const float* x_in, const float* x0, float* x_out, void* h, float* u_qkv, const float* b_q,
                      const float* b_k, const float* b_v, const float* lambda_r, const float* lambda_0, const float* eps_r,
                      const float* eps_0, long eps_ld, const float* gate_w, const float* gate_a,
                      const float* gate_b, float* gate, const float* sign, int members, int T, int pair_shift,
                      const noise_pending_t* pend, int npend, const noise_embed_t* x0_embed, noise_stream_t stream) {
  if (bad_members(members, T, pair_shift)) return NOISE_EINVAL;
  if (!x0 && !x0_embed) return NOISE_EINVAL;
  BlockEntryArgs g{};
  if (!x0) {
    if (x0_embed->idx_mstride < 0) return NOISE_EINVAL;
    g.emb = EmbedSrc{x0_embed->w, x0_embed->a, x0_embed->b, x0_embed->vocab, x0_embed->idx, x0_embed->idx_mstride};
  }
  if (int rc = copy_pending(pend, npend, g.pend)) return rc;
  g.npend = npend;
  g.x_in = x_in;
  g.x0 = x0;
  g.x_out = x_out;
  g.h = static_cast<bf16*>(h);
  g.u_qkv = u_qkv;
  g.b_qkv[0] = b_q;
  g.b_qkv[1] = b_k;
  g.b_qkv[2] = b_v;
  g.lambda_r = lambda_r;
  g.lambda_0 = lambda_0;
  g.eps_r = eps_r;
  g.eps_0 = eps_0;
  g.eps_ld = eps_ld;
  g.sign = sign;
  g.M = members * T;
  g.T = T;
  g.pair_shift = pair_shift;
  g.gate_w = gate_w;
  g.gate_a = gate_a;
  g.gate_b = gate_b;
  g.gate = gate;
  return block_entry_launch(g, static_cast<hipStream_t>(stream));
}

int noise_qkv(const void* h, const void* w_qkv, const float* a_q, const float* a_k, const float* a_v,
              const float* u_qkv, const float* sign, int members, int T, int pair_shift, const void* rot_cos,
              const void* rot_sin, const float* gate, const float* ve_w, long vocab, const float* ve_a,
              const float* ve_b, const int64_t* idx, long idx_mstride, void* qkv, noise_stream_t stream) {
  if (bad_members(members, T, pair_shift) || idx_mstride < 0) return NOISE_EINVAL;
  LowrankGemmArgs g = base_args(h, DM, (long)T * DM, w_qkv, DM, 3 * DM, a_q, sign, members, T, pair_shift);
  g.ra[1] = a_k;
  g.ra[2] = a_v;
  g.seg_n = DM;
  g.ra_ld = DM;
  g.u = u_qkv;
  g.u_parts = 1;
  g.u_ld = 4;
  g.out_bf16 = static_cast<bf16*>(qkv);
  g.ldo = 3 * DM;
  g.rot_cos = static_cast<const bf16*>(rot_cos);
  g.rot_sin = static_cast<const bf16*>(rot_sin);
  g.gate = gate;
  g.ve_w = ve_w;
  g.ve_a = ve_a;
  g.ve_b = ve_b;
  g.ve_v = vocab;
  g.idx = idx;
  g.tok_mstride = idx_mstride;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // q | k and v on the weight-resident kernel (rotary and the head RMSNorm, or the gated value embedding, in
  // its epilogue); both launches read the same h
  LowrankGemmArgs gqk = g;
  gqk.N = 2 * DM;
  if (xs_qk_supported(gqk)) {
    if (int rc = xs_qk_launch(gqk, s)) return rc;
    LowrankGemmArgs gv = g;
    gv.N = DM;
    gv.seg0 = 2;
    gv.W = g.W + (long)2 * DM * DM;
    gv.out_bf16 = g.out_bf16 + 2 * DM;
    if (xs_v_supported(gv)) return xs_v_launch(gv, s);
    if (xs_ve_supported(gv)) return xs_ve_launch(gv, s);
    return lowrank_gemm_launch(EPI_QKV, gv, s);
  }
  return lowrank_gemm_launch(EPI_QKV, g, s);
}

int noise_attention_workspace_size(int members, int T, size_t* bytes) {
  if (members <= 0 || T <= 0 || !bytes) return NOISE_EINVAL;
  *bytes = (size_t)attention_moment_partials(members, T, NH) * sizeof(float);
  return NOISE_OK;
}

int noise_attention(const void* qkv, int members, int T, int window, int qk_norm, int qk_format, const float* b_proj,
                    int pair_shift, void* y, float* upart, float* mom, void* mom_work, size_t mom_work_bytes,
                    noise_stream_t stream) {
  if (bad_members(members, T, pair_shift)) return NOISE_EINVAL;
  if (mom) {
    size_t need = 0;
    noise_attention_workspace_size(members, T, &need);
    if (!mom_work || mom_work_bytes < need) return NOISE_ENOSPC;
  }
  if ((b_proj == nullptr) != (upart == nullptr)) return NOISE_EINVAL;
  AttnArgs g{};
  g.qkv = static_cast<const bf16*>(qkv);
  g.ldq = 3 * DM;
  g.koff = DM;
  g.voff = 2 * DM;
  g.y = static_cast<bf16*>(y);
  g.ldy = DM;
  g.members = members;
  g.T = T;
  g.H = NH;
  g.window = window;
  g.qk_norm = qk_norm != 0;
  g.qk_format = qk_format;
  g.b_proj = b_proj;
  g.b_ld = DM;
  g.pair_shift = pair_shift;
  g.upart = upart;
  g.upart_ld = NH;
  g.mom = mom ? static_cast<float*>(mom_work) : nullptr;
  g.mom_out = mom;
  return attention_launch(g, static_cast<hipStream_t>(stream));
}

int noise_attention_noalloc(const void* qkv, int members, int T, int window, int qk_norm, int qk_format,
                            const float* b_proj, int pair_shift, void* y, float* upart, float* mom,
                            noise_stream_t stream) {
  if (bad_members(members, T, pair_shift)) return NOISE_EINVAL;
  void* work = nullptr;
  size_t bytes = 0;
  if (mom) {
    // the size check comes first: a rejected call touches no GPU state
    noise_attention_workspace_size(members, T, &bytes);
    if (bytes > sizeof(float) * (size_t)NOISE_ATTENTION_NOALLOC_MAX_PARTIALS) return NOISE_ENOSPC;
    if (int rc = scratch_address(&work)) return rc;
  }
  // the same kernels as noise_attention; every partial is written before it is read, so nothing is cleared
  return noise_attention(qkv, members, T, window, qk_norm, qk_format, b_proj, pair_shift, y, upart, mom, work, bytes,
                         stream);
}

int noise_lowrank_resid(const void* x, const void* w, int in, int out, const float* a, const float* u, int u_parts,
                        long u_row_stride, long u_part_stride, const float* sign, int members, int T, int pair_shift,
                        float* resid, noise_stream_t stream) {
  if (bad_members(members, T, pair_shift) || u_parts <= 0 || u_row_stride < 1 || u_row_stride > 0x7fffffffL ||
      u_part_stride < 1)
    return NOISE_EINVAL;
  LowrankGemmArgs g = base_args(x, in, (long)T * in, w, in, out, a, sign, members, T, pair_shift);
  g.u = u;
  g.u_parts = u_parts;
  g.u_ld = (int)u_row_stride;
  g.u_qstride = u_part_stride;
  g.out_f32 = resid;
  g.ldo = out;
  return lowrank_gemm_launch(EPI_RESID, g, static_cast<hipStream_t>(stream));
}

int noise_ac_stream(const void* x_in, const float* wte, long vocab, const int64_t* idx, long idx_mstride,
                    const void* y1, const void* y2, const float* lambda_r, const float* lambda_0, void* x_out, void* h,
                    const float* gate_w, float* gate, int rows, int T, noise_stream_t stream) {
  if (rows <= 0 || T <= 0 || rows % T) return NOISE_EINVAL;
  AcStreamArgs g{};
  g.x_in = static_cast<const bf16*>(x_in);
  g.emb_w = wte;
  g.V = vocab;
  g.idx = idx;
  g.idx_mstride = idx_mstride;
  g.add[0] = static_cast<const bf16*>(y1);
  g.add[1] = static_cast<const bf16*>(y2);
  g.lambda_r = lambda_r;
  g.lambda_0 = lambda_0;
  g.x_out = static_cast<bf16*>(x_out);
  g.h = static_cast<bf16*>(h);
  g.gate_w = gate_w;
  g.gate = gate;
  g.M = rows;
  g.T = T;
  return ac_stream_launch(g, static_cast<hipStream_t>(stream));
}

int noise_ac_qkv(void* qkv, const void* rot_cos, const void* rot_sin, const float* gate, const float* ve_w,
                 long vocab, const int64_t* idx, long idx_mstride, int rows, int T, noise_stream_t stream) {
  if (rows <= 0 || T <= 0 || rows % T) return NOISE_EINVAL;
  AcQkvArgs g{};
  g.qkv = static_cast<bf16*>(qkv);
  g.rot_cos = static_cast<const bf16*>(rot_cos);
  g.rot_sin = static_cast<const bf16*>(rot_sin);
  g.gate = gate;
  g.ve_w = ve_w;
  g.V = vocab;
  g.idx = idx;
  g.idx_mstride = idx_mstride;
  g.M = rows;
  g.T = T;
  return ac_qkv_launch(g, static_cast<hipStream_t>(stream));
}

int noise_norm_dot(const float* x, void* h, const float* b, float* u, const float* sign, int members, int T,
                   int pair_shift, const noise_pending_t* pend, int npend, noise_stream_t stream) {
  if (bad_members(members, T, pair_shift)) return NOISE_EINVAL;
  NormDotArgs g{x, static_cast<bf16*>(h), b, u, sign, members * T, T, pair_shift};
  if (int rc = copy_pending(pend, npend, g.pend)) return rc;
  g.npend = npend;
  return norm_dot_launch(g, static_cast<hipStream_t>(stream));
}

int noise_weight_tiles(const void* w, int rows, int cols, void* out, noise_stream_t stream) {
  return weight_tiles_launch(static_cast<const bf16*>(w), cols, rows, cols, static_cast<bf16*>(out),
                             static_cast<hipStream_t>(stream));
}

int noise_dense_bf16(const void* x, int x_layout, int in, int out, const void* w, int w_layout, int members, int T,
                     void* y, noise_stream_t stream) {
  if (members <= 0 || T <= 0 || (long)members * T > 0x7fffffffL || in <= 0 || out <= 0) return NOISE_EINVAL;
  if (x_layout != NOISE_LAYOUT_ROWS && x_layout != NOISE_LAYOUT_TILE16) return NOISE_EINVAL;
  if (w_layout != NOISE_LAYOUT_ROWS && w_layout != NOISE_LAYOUT_WTILE) return NOISE_EINVAL;
  LowrankGemmArgs g = base_args(x, in, (long)T * in, w, in, out, nullptr, nullptr, members, T, 0);
  g.a_tiled = x_layout == NOISE_LAYOUT_TILE16;
  g.w_tiled = w_layout == NOISE_LAYOUT_WTILE;
  g.out_bf16 = static_cast<bf16*>(y);
  g.ldo = out;
  return lowrank_gemm_launch(EPI_DENSE, g, static_cast<hipStream_t>(stream));
}

int noise_mlp_fc_parts(int f) { return xs_relu2_parts(f); }

int noise_mlp_fc(const void* h, const void* w_fc, int d, int f, const float* a_fc, const float* u,
                 const float* b_proj, const float* sign, int members, int T, int pair_shift, void* hidden,
                 int hidden_layout, float* upart, noise_stream_t stream) {
  if (bad_members(members, T, pair_shift) || !xs_relu2_parts(f)) return NOISE_EINVAL;
  if (hidden_layout != NOISE_LAYOUT_ROWS && hidden_layout != NOISE_LAYOUT_TILE16) return NOISE_EINVAL;
  LowrankGemmArgs g = base_args(h, d, (long)T * d, w_fc, d, f, a_fc, sign, members, T, pair_shift);
  g.u = u;
  g.u_parts = 1;
  g.u_ld = 1;
  g.out_bf16 = static_cast<bf16*>(hidden);
  g.ldo = f;
  g.out_tiled = hidden_layout == NOISE_LAYOUT_TILE16;
  g.rb_next = b_proj;
  g.rb_next_ld = f;
  g.upart_out = upart;
  g.upart_ld = xs_relu2_parts(f);
  return lowrank_gemm_launch(EPI_RELU2, g, static_cast<hipStream_t>(stream));
}

int noise_head_ce_workspace_size(int members, int T, int vocab, int fp32_head, size_t* bytes) {
  // the CE finalisation reads each row's partials four at a time: vocab / 64 partials, a multiple of 4
  if (members <= 0 || T <= 0 || !bytes || vocab <= 0 || vocab % 256 || !lowrank_gemm_parts(vocab) ||
      fp32_head < NOISE_HEAD_BF16 || fp32_head > NOISE_HEAD_FP32)
    return NOISE_EINVAL;
  const size_t M = (size_t)members * T;
  const int split = fp32_head == NOISE_HEAD_FP32_SPLIT;
  Carve c(nullptr);
  c.take<bf16>(M * (split ? 2 : 1) * DM);          // head operand ([hi | lo] rows for the split fp32 head)
  c.take<float>(M);                                // h . b
  c.take<float>(M * lowrank_gemm_parts(vocab));    // partial sums of exp(z')
  c.take<float>(M);                                // z' at the target
  c.take<bf16>((size_t)vocab * (split ? 3 : fp32_head ? 2 : 1) * DM);  // the weight (WTILE or row-major)
  c.take<float>(vocab);                            // NOISE_HEAD_FP32: the weight rows' scales
  *bytes = c.used;
  return NOISE_OK;
}

int noise_head_ce(const void* x, int x_bf16, const float* gain, const void* w_head, int vocab, int fp32_head,
                  const float* a, const float* b, const float* sign, const int64_t* targets, long tgt_mstride,
                  int members, int T, int pair_shift, int reduction, float* loss, float* logits, void* workspace,
                  size_t workspace_bytes, const noise_pending_t* pend, int npend, noise_stream_t stream) {
  size_t need = 0;
  if (int rc = noise_head_ce_workspace_size(members, T, vocab, fp32_head, &need)) return rc;
  if (bad_members(members, T, pair_shift) || !x || !w_head || tgt_mstride < 0 || reduction < NOISE_CE_MEMBER_MEAN ||
      reduction > NOISE_CE_MEAN)
    return NOISE_EINVAL;
  // targets and loss go together; without targets only the logits are produced
  if (!targets ? (!logits || loss) : !loss) return NOISE_EINVAL;
  if (!workspace || workspace_bytes < need) return NOISE_ENOSPC;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t M = (size_t)members * T;
  const bool split = fp32_head == NOISE_HEAD_FP32_SPLIT, f16 = fp32_head == NOISE_HEAD_FP32;
  const int K = (split ? 3 : f16 ? 2 : 1) * DM, lda = (split ? 2 : 1) * DM, parts = lowrank_gemm_parts(vocab);
  Carve c(workspace);
  bf16* hop = c.take<bf16>(M * lda);
  float* u = c.take<float>(M);
  float* part = c.take<float>(M * parts);
  float* tgt = c.take<float>(M);
  // The head's operands reach the GEMM as whole 128-byte lines: the norm writes its rows ([hi | lo] for the fp32
  // head) in TILE16 and the weight is copied into WTILE in the workspace (row-major operands' 32-deep stages load
  // half lines). Rows that do not fill whole 16-row groups, or a weight that is not 16-byte aligned, stay row-major.
  // NOISE_HEAD_FP32: the fp32 weight (16-byte aligned) becomes the fp16 split operand in the workspace, in either
  // layout.
  if (f16 && (((uintptr_t)w_head | (uintptr_t)gain) & 15)) return NOISE_EINVAL;
  const bool tiled = M % 16 == 0 && T % 16 == 0 && !((uintptr_t)w_head & 15);
  bf16* wt = c.take<bf16>((size_t)vocab * K);
  float* wscale = c.take<float>(vocab);
  HeadNormArgs hn{x, x_bf16 ? 1 : 0, gain, hop, b, u, sign, (int)M, T, pair_shift, fp32_head};
  hn.tiled = tiled ? 1 : 0;
  if (int rc = copy_pending(pend, npend, hn.pend)) return rc;
  hn.npend = npend;
  if (int rc = head_norm_launch(hn, s)) return rc;
  if (f16) {
    if (int rc = head_weight_f16_launch(static_cast<const float*>(w_head), DM, gain, vocab, tiled ? 1 : 0, wt, wscale, s))
      return rc;
  } else if (tiled) {
    if (int rc = weight_tiles_launch(static_cast<const bf16*>(w_head), K, vocab, K, wt, s)) return rc;
  }
  LowrankGemmArgs g =
      base_args(hop, lda, (long)T * lda, tiled || f16 ? wt : w_head, K, vocab, a, sign, members, T, pair_shift);
  g.a_tiled = tiled ? 1 : 0;
  g.w_tiled = tiled ? 1 : 0;
  g.a_fold = fp32_head ? DM : 0;
  g.col_scale = f16 ? wscale : nullptr;
  g.u = u;
  g.u_parts = 1;
  g.u_ld = 1;
  g.round_bf16 = fp32_head ? 0 : 1;
  g.targets = targets;
  g.tok_mstride = tgt_mstride;
  g.logits = logits;
  g.ce_tgt = tgt;
  g.upart_out = part;
  g.upart_ld = parts;
  g.ldo = vocab;
  if (int rc = lowrank_gemm_launch(f16 ? EPI_CE_F16 : EPI_CE, g, s)) return rc;
  if (!targets) return NOISE_OK;
  CeFinalizeArgs f{part, tgt, parts, members, T, loss, targets, tgt_mstride, reduction};
  return ce_finalize_launch(f, s);
}

int noise_fitness(const float* losses, int n, int pairs, int mode, float* fitness, float* weight,
                  noise_stream_t stream) {
  return fitness_launch(losses, n, pairs, mode, fitness, weight, static_cast<hipStream_t>(stream));
}

int noise_outer_update(const float* a, long a_ld, const float* b, long b_ld, const float* w, int ndir, int out,
                       int in, float scale, float* grad, noise_stream_t stream) {
  const OuterUpdateArgs u{a, a_ld, b, b_ld, out, in, grad};
  return outer_update_launch(&u, 1, w, ndir, scale, static_cast<hipStream_t>(stream));
}

int noise_outer_update_batch(const noise_outer_mat_t* mats, int n, const float* w, int ndir, float scale,
                             noise_stream_t stream) {
  if (n <= 0 || !mats) return NOISE_EINVAL;
  std::vector<OuterUpdateArgs> u(n);
  for (int k = 0; k < n; ++k) u[k] = OuterUpdateArgs{mats[k].a, mats[k].a_ld, mats[k].b, mats[k].b_ld, mats[k].out, mats[k].in, mats[k].grad};
  return outer_update_launch(u.data(), n, w, ndir, scale, static_cast<hipStream_t>(stream));
}

int noise_gather_rows(const float* buffer, long buffer_len, const noise_gather_param_t* params, int nparams,
                      const int64_t* directions, int ndir, int pairs, noise_stream_t stream) {
  if (nparams <= 0 || !params) return NOISE_EINVAL;
  std::vector<GatherParam> q(nparams);
  for (int k = 0; k < nparams; ++k)
    q[k] = GatherParam{params[k].offsets, params[k].a, params[k].b, params[k].out, params[k].in};
  return gather_rows_launch(q.data(), nparams, buffer, buffer_len, directions, ndir, pairs,
                            static_cast<hipStream_t>(stream));
}

int noise_readout_probes(const float* base, long base_ld, const float* dirs, long dirs_ld, const int64_t* rows, int K,
                         const int64_t* targets, const float* steps, const float* sq, const float* dots, long dots_ld,
                         const float* dir_sq, int dir_sq_per_token, int n, int vocab, int P, int width, float* out,
                         noise_stream_t stream) {
  const ProbeArgs g{base, base_ld, dirs, dirs_ld, rows, K, targets, steps, sq, dots, dots_ld, dir_sq,
                    dir_sq_per_token ? 1 : 0, n, vocab, P, width, out};
  return probe_launch(g, static_cast<hipStream_t>(stream));
}

int noise_moved_heads(const float* raw, const void* a, float sigma, const float* rot_cos, const float* rot_sin, int draws,
                      int batch, int T, int heads, void* out, long out_ld, noise_stream_t stream) {
  const MovedHeadsArgs g{raw, static_cast<const bf16*>(a), sigma, rot_cos, rot_sin, static_cast<bf16*>(out), out_ld,
                         draws, batch, T, heads, (long)draws * batch * T * heads};
  return moved_heads_launch(g, static_cast<hipStream_t>(stream));
}

int noise_head_scores(const void* out, long out_ld, const float* baseline, const float* hub, int draws, int batch, int T,
                      int heads, float* score, noise_stream_t stream) {
  const HeadScoresArgs g{static_cast<const bf16*>(out), out_ld, baseline, hub, score, draws, batch, T, heads,
                         (long)draws * batch * T * heads};
  return head_scores_launch(g, static_cast<hipStream_t>(stream));
}

int noise_key_filter(const void* filter, const float* score, int batch, int heads, int T, int draws, float* out,
                     noise_stream_t stream) {
  if (batch <= 0 || heads <= 0 || (long)batch * heads > 0x7fffffffL) return NOISE_EINVAL;
  const KeyFilterArgs g{static_cast<const bf16*>(filter), score, out, batch * heads, T, draws};
  return key_filter_launch(g, static_cast<hipStream_t>(stream));
}

int noise_code_estimate(const float* credited, const void* a, int draws, int batch, int T, int heads, float* est,
                        noise_stream_t stream) {
  const CodeEstimateArgs g{credited, static_cast<const bf16*>(a), est, draws, T, heads, (long)batch * T * heads * 64};
  return code_estimate_launch(g, static_cast<hipStream_t>(stream));
}

int noise_hbm_stream(const void* src, int in_kib, void* dst, int out_kib, long rows, noise_stream_t stream) {
  return hbm_stream_launch(src, in_kib, dst, out_kib, rows, static_cast<hipStream_t>(stream));
}

int noise_adam_batch(const noise_adam_tensor_t* tensors, int n, float beta1, float beta2, float eps,
                     noise_stream_t stream) {
  if (n <= 0 || !tensors) return NOISE_EINVAL;
  std::vector<AdamTensor> t(n);
  for (int k = 0; k < n; ++k)
    t[k] = AdamTensor{tensors[k].param, tensors[k].grad, tensors[k].exp_avg, tensors[k].exp_avg_sq, tensors[k].n,
                      tensors[k].step_size, tensors[k].bc2_sqrt, 0};
  return adam_batch_launch(t.data(), n, beta1, beta2, eps, static_cast<hipStream_t>(stream));
}

int noise_adam(float* param, const float* grad, float* exp_avg, float* exp_avg_sq, long n, float step_size,
               float beta1, float beta2, float eps, float bc2_sqrt, noise_stream_t stream) {
  AdamArgs g{param, grad, exp_avg, exp_avg_sq, n, step_size, beta1, beta2, eps, bc2_sqrt};
  return adam_launch(g, static_cast<hipStream_t>(stream));
}

}  // extern "C"
