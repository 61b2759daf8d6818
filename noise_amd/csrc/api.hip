// extern "C" entry points of libnoise_hip.so (declared in include/noise_hip.h).
#include "../../include/noise_hip.h"
#include "common.h"
#include "gemm.h"

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

constexpr int EPI_STORE = 0, EPI_RELU2 = 1, EPI_RESID = 2;

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
  g.ra = a;
  g.ra_ld = out;
  return g;
}

}  // namespace

extern "C" {

int noise_version(void) { return 100; }

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
  g.out_f32 = y_f32;
  g.out_bf16 = static_cast<bf16*>(y_bf16);
  g.ldo = out;
  return lowrank_gemm_launch(accumulate ? EPI_RESID : EPI_STORE, g, s);
}

int noise_lowrank_mlp_workspace_size(int members, int T, int d, int f, size_t* bytes) {
  if (members <= 0 || T <= 0 || d <= 0 || f <= 0 || !bytes) return NOISE_EINVAL;
  const size_t M = (size_t)members * T;
  Carve c(nullptr);
  c.take<float>(M);                                    // u_fc
  c.take<float>(M * lowrank_gemm_parts(f));            // partial dots h.b_proj
  c.take<bf16>(M * f);                                  // hidden h
  *bytes = c.used;
  return NOISE_OK;
}

int noise_lowrank_mlp(const void* x, long x_ld, long x_mstride, const void* w_fc, const void* w_proj, int d, int f,
                      const float* a_fc, const float* b_fc, const float* a_proj, const float* b_proj,
                      const float* sign, int members, int T, int pair_shift, float* y_f32, void* y_bf16,
                      int accumulate, void* workspace, size_t workspace_bytes, noise_stream_t stream) {
  size_t need = 0;
  if (int rc = noise_lowrank_mlp_workspace_size(members, T, d, f, &need)) return rc;
  if (!workspace || workspace_bytes < need) return NOISE_ENOSPC;
  if (!lowrank_gemm_parts(f) || (accumulate && (!y_f32 || y_bf16))) return NOISE_EINVAL;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t M = (size_t)members * T;
  Carve c(workspace);
  float* u_fc = c.take<float>(M);
  const int parts = lowrank_gemm_parts(f);
  float* upart = c.take<float>(M * parts);
  bf16* hid = c.take<bf16>(M * f);
  if (int rc = rowdot_launch(static_cast<const bf16*>(x), x_ld, x_mstride, (int)M, d, T, pair_shift, b_fc, d, u_fc, s))
    return rc;
  LowrankGemmArgs g1 = base_args(x, x_ld, x_mstride, w_fc, d, f, a_fc, sign, members, T, pair_shift);
  g1.u = u_fc;
  g1.u_parts = 1;
  g1.out_bf16 = hid;
  g1.ldo = f;
  g1.rb_next = b_proj;
  g1.rb_next_ld = f;
  g1.upart_out = upart;
  g1.upart_ld = parts;
  if (int rc = lowrank_gemm_launch(EPI_RELU2, g1, s)) return rc;
  LowrankGemmArgs g2 = base_args(hid, f, (long)T * f, w_proj, f, d, a_proj, sign, members, T, pair_shift);
  g2.u = upart;
  g2.u_parts = parts;
  g2.out_f32 = y_f32;
  g2.out_bf16 = static_cast<bf16*>(y_bf16);
  g2.ldo = d;
  return lowrank_gemm_launch(accumulate ? EPI_RESID : EPI_STORE, g2, s);
}

}  // extern "C"
