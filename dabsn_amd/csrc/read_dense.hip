// Dense-mask three-way admitted read: the registered op pair
// dabsn::admitted_three_way_read_native / dabsn::_admitted_three_way_read_backward
// (reference src/dabsn/kernels/admitted.py:16-65 forward, :126-236 backward, :383-622 the
// op pair; src/dabsn/kernels/cpu_runtime.cpp three_way_read_cpu / three_way_read_bwd).
//
// Unlike the compact read (read3.hip), whose masks follow from slot positions, the masks
// here are arbitrary [B, T, N] byte tensors, so the read is evaluated in three stages:
//
//   S = Q K^T                      batched MFMA GEMM (fp32), [B, T, N]
//   rows: three masked softmaxes   one workgroup per (b, t) row, three passes over N
//   out = W1 V + W2 Vn             one GEMM with two products; W1 = g_s P_s + g_p P_p and
//                                  W2 = g_i P_i are written by the row pass
//
// and the backward recomputes S and the softmaxes (the op saves its inputs only), forms
// G = dO V^T and Gn = dO Vn^T, and a row pass writes the score gradient D (all three
// pathways) and Dp (the permanent pathway alone) plus per-row partial sums of the scalar
// gradients; a column pass sums D and Dp over queries for the per-slot gradients, and
// four more GEMMs give the query, key and write gradients. Everything computes in fp32,
// the reference's compute dtype for fp32 and bf16 inputs. Scalar gradients are summed
// per row and then over rows in a fixed order (deterministic).
//
// Softmax semantics follow the reference's masked_fill / softmax / where sequence: a row
// that is not eligible has zero weights; an eligible row with no allowed slot has NaN
// weights (softmax over all -inf); disallowed slots of other rows have weight 0.
#include <math.h>

#include "../../include/dabsn_hip.h"
#include "capi.hpp"
#include "common.hpp"
#include "gemm.hpp"
#include "transpose.hpp"

namespace dabsn {
namespace dense {

constexpr int NT = 256;  // threads per row workgroup (4 waves)

// Scalars in the op's schema order.
enum { kScale = 0, kShort = 1, kPad = 2, kInduct = 3, kCocktail = 4, kNumScalars = 5 };

struct RowArgs {
  int T, N;
  const float* S;        // [B, T, N] raw query-key products
  const float* ck;       // [B, T, 4] query cocktails
  const float* cb;       // [B, N, 4] slot cocktails
  const float* kb;       // [B, N] key bias
  const float* adm;      // [B, N] admission
  const uint8_t* allow;  // [B, T, N]
  const uint8_t* iallow;
  const uint8_t* elig;   // [B, T]
  const uint8_t* ielig;
  const float* sc;       // [5] scalars
};

// Element-wise reductions over the 4 waves of a row workgroup; every thread receives the
// results. `sh` holds K x 4 floats.
template <int K, typename Op>
__device__ __forceinline__ void block_reduce(float (&v)[K], float identity, Op op, float* sh) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int k = 0; k < K; ++k) v[k] = wave_reduce(v[k], identity, op);
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < K; ++k) sh[k * 4 + wave] = v[k];
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < K; ++k)
    v[k] = op(op(sh[k * 4 + 0], sh[k * 4 + 1]), op(sh[k * 4 + 2], sh[k * 4 + 3]));
  __syncthreads();
}

// The three softmaxes of one row: scores of slot n, the row maxima and normalisers.
struct Row {
  const float* s;
  const uint8_t* al;
  const uint8_t* ial;
  const float* kb;
  const float* adm;
  const float* cb;
  float q[4];
  float scale, cg;
  bool el, iel;
  float m_s, m_p, m_i, z_s, z_p, z_i;

  __device__ Row(const RowArgs& a, int row) {
    const int b = row / a.T;
    const size_t ro = static_cast<size_t>(row) * a.N;
    s = a.S + ro;
    al = a.allow + ro;
    ial = a.iallow + ro;
    kb = a.kb + static_cast<size_t>(b) * a.N;
    adm = a.adm + static_cast<size_t>(b) * a.N;
    cb = a.cb + static_cast<size_t>(b) * a.N * 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) q[k] = a.ck[static_cast<size_t>(row) * 4 + k];
    scale = a.sc[kScale];
    cg = a.sc[kCocktail];
    el = a.elig[row] != 0;
    iel = a.ielig[row] != 0;
  }

  // Unscaled cocktail compatibility of slot n (bmm(cocktail, bank_cocktail^T)).
  __device__ float raw_cocktail(int n) const {
    float d = q[0] * cb[n * 4 + 0];
    d += q[1] * cb[n * 4 + 1];
    d += q[2] * cb[n * 4 + 2];
    d += q[3] * cb[n * 4 + 3];
    return d;
  }
  // short = compat * scale + key_bias + admission; permanent adds the scaled cocktail
  // compatibility before the admission (admitted.py:47-50).
  __device__ void scores(int n, float& sh, float& pe) const {
    const float content = s[n] * scale + kb[n];
    sh = content + adm[n];
    pe = (content + raw_cocktail(n) * cg) + adm[n];
  }

};

__device__ __forceinline__ float softmax_weight(bool row_ok, bool slot_ok, float x, float m, float z) {
  if (!row_ok) return 0.0f;
  if (m == -INFINITY) return NAN;  // softmax over an all -inf row
  return slot_ok ? expf(x - m) / z : 0.0f;
}

// Passes 1 and 2 of both row kernels: maxima then normalisers of the three softmaxes.
__device__ __forceinline__ void row_stats(Row& r, int N, float* shm) {
  float m[3] = {-INFINITY, -INFINITY, -INFINITY};
  for (int n = threadIdx.x; n < N; n += NT) {
    float sh, pe;
    r.scores(n, sh, pe);
    if (r.al[n]) {
      m[0] = fmaxf(m[0], sh);
      m[1] = fmaxf(m[1], pe);
    }
    if (r.ial[n]) m[2] = fmaxf(m[2], sh);
  }
  block_reduce<3>(m, -INFINITY, [](float x, float y) { return fmaxf(x, y); }, shm);
  float z[3] = {0.f, 0.f, 0.f};
  for (int n = threadIdx.x; n < N; n += NT) {
    float sh, pe;
    r.scores(n, sh, pe);
    if (r.al[n]) {
      z[0] += expf(sh - m[0]);
      z[1] += expf(pe - m[1]);
    }
    if (r.ial[n]) z[2] += expf(sh - m[2]);
  }
  block_reduce<3>(z, 0.0f, [](float x, float y) { return x + y; }, shm);
  r.m_s = m[0];
  r.m_p = m[1];
  r.m_i = m[2];
  r.z_s = z[0];
  r.z_p = z[1];
  r.z_i = z[2];
}

__device__ __forceinline__ void weights(const Row& r, int n, float& ps, float& pp, float& pi) {
  float sh, pe;
  r.scores(n, sh, pe);
  const bool a = r.al[n] != 0, ia = r.ial[n] != 0;
  ps = softmax_weight(r.el, a, sh, r.m_s, r.z_s);
  pp = softmax_weight(r.el, a, pe, r.m_p, r.z_p);
  pi = softmax_weight(r.iel, ia, sh, r.m_i, r.z_i);
}

// Forward rows: W1 = g_s P_s + g_p P_p, W2 = g_i P_i; with Ps non-null also the three
// softmaxes themselves (the 4-output op returns them).
__global__ void __launch_bounds__(NT) rows_fwd_kernel(RowArgs a, float* W1, float* W2, float* Ps,
                                                      float* Pp, float* Pi) {
  __shared__ float shm[3 * 4];
  const int row = blockIdx.x;
  Row r(a, row);
  row_stats(r, a.N, shm);
  const float sg = a.sc[kShort], pg = a.sc[kPad], ig = a.sc[kInduct];
  const size_t ro = static_cast<size_t>(row) * a.N;
  for (int n = threadIdx.x; n < a.N; n += NT) {
    float ps, pp, pi;
    weights(r, n, ps, pp, pi);
    W1[ro + n] = sg * ps + pg * pp;
    W2[ro + n] = ig * pi;
    if (Ps) {
      Ps[ro + n] = ps;
      Pp[ro + n] = pp;
      Pi[ro + n] = pi;
    }
  }
}

// Backward rows. Inputs G = dO V^T and Gn = dO Vn^T. Writes the score gradient D (sum of
// the three pathways) and Dp (permanent pathway), W1 / W2 as in the forward (for the write
// gradients), the query cocktail gradient, and per-row partials
// [sum D*S, sum Dp*raw_cocktail, sum P_s*G, sum P_p*G, sum P_i*Gn].
__global__ void __launch_bounds__(NT) rows_bwd_kernel(RowArgs a, const float* G, const float* Gn,
                                                      float* D, float* Dp, float* W1, float* W2,
                                                      float* g_ck, float* partial) {
  __shared__ float shm[6 * 4];
  const int row = blockIdx.x;
  Row r(a, row);
  row_stats(r, a.N, shm);
  const float sg = a.sc[kShort], pg = a.sc[kPad], ig = a.sc[kInduct];
  const size_t ro = static_cast<size_t>(row) * a.N;
  // Pass 3: the softmax backward's row dots and the gains' partials.
  float acc[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int n = threadIdx.x; n < a.N; n += NT) {
    float ps, pp, pi;
    weights(r, n, ps, pp, pi);
    const float g = G[ro + n], gn = Gn[ro + n];
    acc[0] += (g * sg) * ps;
    acc[1] += (g * pg) * pp;
    acc[2] += (gn * ig) * pi;
    acc[3] += ps * g;
    acc[4] += pp * g;
    acc[5] += pi * gn;
  }
  block_reduce<6>(acc, 0.0f, [](float x, float y) { return x + y; }, shm);
  // Pass 4: score gradients (masked as admitted.py:116-123), then their products.
  float out[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int n = threadIdx.x; n < a.N; n += NT) {
    float ps, pp, pi;
    weights(r, n, ps, pp, pi);
    const float g = G[ro + n], gn = Gn[ro + n];
    const bool on = r.el && r.al[n], ion = r.iel && r.ial[n];
    const float ds = on ? ps * ((g * sg) - acc[0]) : 0.0f;
    const float dp = on ? pp * ((g * pg) - acc[1]) : 0.0f;
    const float di = ion ? pi * ((gn * ig) - acc[2]) : 0.0f;
    const float d = (ds + dp) + di;
    D[ro + n] = d;
    Dp[ro + n] = dp;
    W1[ro + n] = sg * ps + pg * pp;
    W2[ro + n] = ig * pi;
    out[0] += d * r.s[n];
    out[1] += dp * r.raw_cocktail(n);
#pragma unroll
    for (int k = 0; k < 4; ++k) out[2 + k] += dp * r.cb[n * 4 + k];
  }
  block_reduce<6>(out, 0.0f, [](float x, float y) { return x + y; }, shm);
  if (threadIdx.x == 0) {
    float* p = partial + static_cast<size_t>(row) * kNumScalars;
    p[0] = out[0];
    p[1] = out[1];
    p[2] = acc[3];
    p[3] = acc[4];
    p[4] = acc[5];
#pragma unroll
    for (int k = 0; k < 4; ++k) g_ck[static_cast<size_t>(row) * 4 + k] = out[2 + k] * r.cg;
  }
}

// Per-slot sums over queries: key-bias and admission gradients (sum_t D) and the slot
// cocktail gradient (cocktail_gain * sum_t Dp ck_t). One thread per (b, n).
__global__ void __launch_bounds__(NT) cols_kernel(int T, int N, const float* D, const float* Dp,
                                                  const float* ck, const float* sc, float* g_kb,
                                                  float* g_adm, float* g_cb) {
  const int b = blockIdx.y;
  const int n = blockIdx.x * NT + threadIdx.x;
  if (n >= N) return;
  float acc = 0.f, c[4] = {0.f, 0.f, 0.f, 0.f};
  const float* ckb = ck + static_cast<size_t>(b) * T * 4;
  for (int t = 0; t < T; ++t) {
    const size_t i = (static_cast<size_t>(b) * T + t) * N + n;
    acc += D[i];
    const float dp = Dp[i];
#pragma unroll
    for (int k = 0; k < 4; ++k) c[k] += dp * ckb[t * 4 + k];
  }
  const size_t o = static_cast<size_t>(b) * N + n;
  g_kb[o] = acc;
  g_adm[o] = acc;
  const float cg = sc[kCocktail];
#pragma unroll
  for (int k = 0; k < 4; ++k) g_cb[o * 4 + k] = c[k] * cg;
}

// Scalar gradients: per-row partials summed in a fixed order, in the op's scalar order
// (scale, short_gain, pad_gain, induct_gain, cocktail_gain).
__global__ void __launch_bounds__(NT) scalars_kernel(int rows, const float* partial, float* g) {
  __shared__ float shm[5 * 4];
  float v[5] = {0.f, 0.f, 0.f, 0.f, 0.f};
  for (int i = threadIdx.x; i < rows; i += NT) {
#pragma unroll
    for (int k = 0; k < 5; ++k) v[k] += partial[static_cast<size_t>(i) * 5 + k];
  }
  block_reduce<5>(v, 0.0f, [](float x, float y) { return x + y; }, shm);
  if (threadIdx.x == 0) {
    g[kScale] = v[0];
    g[kCocktail] = v[1];
    g[kShort] = v[2];
    g[kPad] = v[3];
    g[kInduct] = v[4];
  }
}

// x *= sc[kScale] (the reference multiplies the query and key products by scale after
// the bmm).
__global__ void __launch_bounds__(NT) scale_kernel(int64_t n, float* x, const float* sc) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x;
  if (i < n) x[i] = x[i] * sc[kScale];
}

}  // namespace dense
}  // namespace dabsn

using namespace dabsn;
using namespace dabsn::dense;

namespace {

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

struct Layout {
  size_t btn, bhn, bht, off[12], total;
};

// Forward: S, W1, W2 [B,T,N]; Vt, Vnt [B,H,N].
// Backward: S (later D^T), G (later W1^T), Gn (later W2^T), D, Dp, W1, W2 [B,T,N];
// K^T [B,H,N]; Q^T, dO^T [B,H,T]; row partials [B*T][5].
Layout layout(int64_t B, int64_t T, int64_t N, int64_t H, bool backward) {
  Layout l{};
  l.btn = align256(static_cast<size_t>(B * T * N) * 4);
  l.bhn = align256(static_cast<size_t>(B * H * N) * 4);
  l.bht = align256(static_cast<size_t>(B * H * T) * 4);
  size_t o = 0;
  int k = 0;
  auto put = [&](size_t bytes) {
    l.off[k++] = o;
    o += bytes;
  };
  if (!backward) {
    for (int i = 0; i < 3; ++i) put(l.btn);
    put(l.bhn);
    put(l.bhn);
  } else {
    for (int i = 0; i < 7; ++i) put(l.btn);
    put(l.bhn);
    put(l.bht);
    put(l.bht);
    put(align256(static_cast<size_t>(B * T) * 5 * 4));
  }
  l.total = o;
  return l;
}

int check_shape(int64_t B, int64_t T, int64_t N, int64_t H) {
  DABSN_REQUIRE(B > 0 && T > 0 && N > 0 && H > 0, "dense read: B, T, N, H must be positive");
  DABSN_REQUIRE(B * T < (1ll << 31) && N < (1ll << 30) && H < (1ll << 30) && T < (1ll << 30),
                "dense read: shape too large");
  return DABSN_OK;
}

// C[b] = A[b] B[b]^T (+ A2[b] B2[b]^T), fp32, all operands K-contiguous.
int gemm_nt(int batch, int M, int Ncols, int K, const float* A, int64_t lda, int64_t sA,
            const float* Bm, int64_t ldb, int64_t sB, const float* A2, const float* B2, float* C,
            int64_t ldc, int64_t sC, hipStream_t stream) {
  gemm::Args<float, float> g{};
  g.M = M;
  g.N = Ncols;
  g.K = K;
  g.A = A;
  g.lda = lda;
  g.sA = sA;
  g.B = Bm;
  g.ldb = ldb;
  g.sB = sB;
  g.A2 = A2;
  g.B2 = B2;
  g.C = C;
  g.ldc = ldc;
  g.sC = sC;
  g.alpha = 1.0f;
  const hipError_t e = gemm::launch<float, float>(g, batch, stream);
  if (e == hipErrorInvalidValue) {
    dabsn::set_error("dense read: a GEMM operand exceeds the 2 GiB buffer range");
    return DABSN_ERR_ARG;
  }
  DABSN_HIP_CHECK(e);
  return DABSN_OK;
}

#define DENSE_TRY(x)                \
  do {                              \
    const int rc_ = (x);            \
    if (rc_ != DABSN_OK) return rc_; \
  } while (0)

}  // namespace

extern "C" {

size_t dabsn_hip_read_dense_workspace_bytes(int64_t B, int64_t T, int64_t N, int64_t H,
                                            int backward) {
  if (B <= 0 || T <= 0 || N <= 0 || H <= 0) return 0;
  return layout(B, T, N, H, backward != 0).total;
}

int dabsn_hip_read_dense_fwd(int64_t B, int64_t T, int64_t N, int64_t H, const float* query,
                             const float* bank_keys, const float* bank_writes,
                             const float* next_writes, const float* cocktail,
                             const float* bank_cocktail, const float* bank_key_bias,
                             const float* bank_admission, const uint8_t* allow,
                             const uint8_t* induct_allow, const uint8_t* eligible,
                             const uint8_t* induct_eligible, const float* scalars, float* out,
                             void* workspace, size_t workspace_bytes, hipStream_t stream) {
  return dabsn_hip_read_dense_fwd_weights(B, T, N, H, query, bank_keys, bank_writes, next_writes,
                                          cocktail, bank_cocktail, bank_key_bias, bank_admission,
                                          allow, induct_allow, eligible, induct_eligible, scalars,
                                          out, nullptr, nullptr, nullptr, workspace,
                                          workspace_bytes, stream);
}

int dabsn_hip_read_dense_fwd_weights(int64_t B, int64_t T, int64_t N, int64_t H,
                                     const float* query, const float* bank_keys,
                                     const float* bank_writes, const float* next_writes,
                                     const float* cocktail, const float* bank_cocktail,
                                     const float* bank_key_bias, const float* bank_admission,
                                     const uint8_t* allow, const uint8_t* induct_allow,
                                     const uint8_t* eligible, const uint8_t* induct_eligible,
                                     const float* scalars, float* out, float* short_weights,
                                     float* permanent_weights, float* induct_weights,
                                     void* workspace, size_t workspace_bytes,
                                     hipStream_t stream) {
  DENSE_TRY(check_shape(B, T, N, H));
  DABSN_REQUIRE((short_weights == nullptr) == (permanent_weights == nullptr) &&
                    (short_weights == nullptr) == (induct_weights == nullptr),
                "dense read: the three weight outputs are given together or not at all");
  DABSN_REQUIRE(query && bank_keys && bank_writes && next_writes && cocktail && bank_cocktail &&
                    bank_key_bias && bank_admission && allow && induct_allow && eligible &&
                    induct_eligible && scalars && out && workspace,
                "dense read: null pointer");
  const Layout l = layout(B, T, N, H, false);
  DABSN_REQUIRE(workspace_bytes >= l.total, "dense read: workspace %zu < %zu bytes",
                workspace_bytes, l.total);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* S = reinterpret_cast<float*>(ws + l.off[0]);
  float* W1 = reinterpret_cast<float*>(ws + l.off[1]);
  float* W2 = reinterpret_cast<float*>(ws + l.off[2]);
  float* Vt = reinterpret_cast<float*>(ws + l.off[3]);
  float* Vnt = reinterpret_cast<float*>(ws + l.off[4]);
  const int b = static_cast<int>(B), t = static_cast<int>(T), n = static_cast<int>(N),
            h = static_cast<int>(H);
  DENSE_TRY(gemm_nt(b, t, n, h, query, H, T * H, bank_keys, H, N * H, nullptr, nullptr, S, N,
                    T * N, stream));
  const RowArgs ra{t, n, S, cocktail, bank_cocktail, bank_key_bias, bank_admission, allow,
                   induct_allow, eligible, induct_eligible, scalars};
  hipLaunchKernelGGL(rows_fwd_kernel, dim3(static_cast<unsigned>(B * T)), dim3(NT), 0, stream, ra,
                     W1, W2, short_weights, permanent_weights, induct_weights);
  DABSN_HIP_CHECK(hipGetLastError());
  DABSN_HIP_CHECK(xpose::transpose(bank_writes, Vt, b, n, h, stream));
  DABSN_HIP_CHECK(xpose::transpose(next_writes, Vnt, b, n, h, stream));
  return gemm_nt(b, t, h, n, W1, N, T * N, Vt, N, H * N, W2, Vnt, out, H, T * H, stream);
}

int dabsn_hip_read_dense_bwd(int64_t B, int64_t T, int64_t N, int64_t H, const float* grad_out,
                             const float* query, const float* bank_keys, const float* bank_writes,
                             const float* next_writes, const float* cocktail,
                             const float* bank_cocktail, const float* bank_key_bias,
                             const float* bank_admission, const uint8_t* allow,
                             const uint8_t* induct_allow, const uint8_t* eligible,
                             const uint8_t* induct_eligible, const float* scalars, float* g_query,
                             float* g_keys, float* g_writes, float* g_next, float* g_cocktail,
                             float* g_bank_cocktail, float* g_key_bias, float* g_admission,
                             float* g_scalars, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
  DENSE_TRY(check_shape(B, T, N, H));
  DABSN_REQUIRE(grad_out && query && bank_keys && bank_writes && next_writes && cocktail &&
                    bank_cocktail && bank_key_bias && bank_admission && allow && induct_allow &&
                    eligible && induct_eligible && scalars && g_query && g_keys && g_writes &&
                    g_next && g_cocktail && g_bank_cocktail && g_key_bias && g_admission &&
                    g_scalars && workspace,
                "dense read backward: null pointer");
  const Layout l = layout(B, T, N, H, true);
  DABSN_REQUIRE(workspace_bytes >= l.total, "dense read backward: workspace %zu < %zu bytes",
                workspace_bytes, l.total);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  auto buf = [&](int i) { return reinterpret_cast<float*>(ws + l.off[i]); };
  float *S = buf(0), *G = buf(1), *Gn = buf(2), *D = buf(3), *Dp = buf(4), *W1 = buf(5),
        *W2 = buf(6), *Kt = buf(7), *Qt = buf(8), *dOt = buf(9), *part = buf(10);
  // Reused once the row pass has consumed S, G and Gn.
  float *Dt = S, *W1t = G, *W2t = Gn;
  const int b = static_cast<int>(B), t = static_cast<int>(T), n = static_cast<int>(N),
            h = static_cast<int>(H);
  DENSE_TRY(gemm_nt(b, t, n, h, query, H, T * H, bank_keys, H, N * H, nullptr, nullptr, S, N,
                    T * N, stream));
  DENSE_TRY(gemm_nt(b, t, n, h, grad_out, H, T * H, bank_writes, H, N * H, nullptr, nullptr, G, N,
                    T * N, stream));
  DENSE_TRY(gemm_nt(b, t, n, h, grad_out, H, T * H, next_writes, H, N * H, nullptr, nullptr, Gn,
                    N, T * N, stream));
  const RowArgs ra{t, n, S, cocktail, bank_cocktail, bank_key_bias, bank_admission, allow,
                   induct_allow, eligible, induct_eligible, scalars};
  hipLaunchKernelGGL(rows_bwd_kernel, dim3(static_cast<unsigned>(B * T)), dim3(NT), 0, stream, ra,
                     G, Gn, D, Dp, W1, W2, g_cocktail, part);
  DABSN_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(cols_kernel, dim3(static_cast<unsigned>((N + NT - 1) / NT), b), dim3(NT), 0,
                     stream, t, n, D, Dp, cocktail, scalars, g_key_bias, g_admission,
                     g_bank_cocktail);
  DABSN_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(scalars_kernel, dim3(1), dim3(NT), 0, stream, static_cast<int>(B * T), part,
                     g_scalars);
  DABSN_HIP_CHECK(hipGetLastError());
  // Query and key gradients: (D K) * scale and (D^T Q) * scale.
  DABSN_HIP_CHECK(xpose::transpose(bank_keys, Kt, b, n, h, stream));
  DENSE_TRY(gemm_nt(b, t, h, n, D, N, T * N, Kt, N, H * N, nullptr, nullptr, g_query, H, T * H,
                    stream));
  DABSN_HIP_CHECK(xpose::transpose(D, Dt, b, t, n, stream));
  DABSN_HIP_CHECK(xpose::transpose(query, Qt, b, t, h, stream));
  DENSE_TRY(gemm_nt(b, n, h, t, Dt, T, N * T, Qt, T, H * T, nullptr, nullptr, g_keys, H, N * H,
                    stream));
  const int64_t nq = B * T * H, nk = B * N * H;
  hipLaunchKernelGGL(scale_kernel, dim3(static_cast<unsigned>((nq + NT - 1) / NT)), dim3(NT), 0,
                     stream, nq, g_query, scalars);
  hipLaunchKernelGGL(scale_kernel, dim3(static_cast<unsigned>((nk + NT - 1) / NT)), dim3(NT), 0,
                     stream, nk, g_keys, scalars);
  DABSN_HIP_CHECK(hipGetLastError());
  // Write gradients: W1^T dO and W2^T dO.
  DABSN_HIP_CHECK(xpose::transpose(W1, W1t, b, t, n, stream));
  DABSN_HIP_CHECK(xpose::transpose(W2, W2t, b, t, n, stream));
  DABSN_HIP_CHECK(xpose::transpose(grad_out, dOt, b, t, h, stream));
  DENSE_TRY(gemm_nt(b, n, h, t, W1t, T, N * T, dOt, T, H * T, nullptr, nullptr, g_writes, H,
                    N * H, stream));
  return gemm_nt(b, n, h, t, W2t, T, N * T, dOt, T, H * T, nullptr, nullptr, g_next, H, N * H,
                 stream);
}

}  // extern "C"
