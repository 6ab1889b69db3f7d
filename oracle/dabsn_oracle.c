/*
 * CPU oracle for the DABSN recurrent hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file is a plain-C restatement of the reference algorithms, used only by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.
 * No product code path links, loads or calls it.
 *
 * Precision and order follow the reference CPU backend: fp32 storage, fp32
 * arithmetic, serial row-loop dot products, compiled with -ffp-contract=off
 * (reference: src/dabsn/kernels/cpu.py:78,95-96). Parallelism is OpenMP over the
 * batch, as in the reference.
 *
 * Functions and the reference code they restate:
 *   oracle_core_scan_fwd   cpu_runtime.cpp:672-837 (training forward), plus the
 *                          gate tape that cpu.py:866-869 recomputes.
 *   oracle_core_scan_bwd   batched_runtime.py:299-466 (_backward_step), driven as
 *                          in _backward_chunk 501-589 / _prev_slices 592-622, and the
 *                          recurrent-weight gradient GEMM at 1475-1482. This is the
 *                          backward the registered op actually runs on CPU.
 *   oracle_read3_fwd       cpu_runtime.cpp:321-438 (three-pass masked softmax per
 *                          pathway), with masks built as compact_admitted.py:176-198.
 *   oracle_read3_bwd       cpu_runtime.cpp:479-662.
 *   oracle_linrec_fwd/bwd  cpu_runtime.cpp:92-143.
 *   oracle_long_fwd/bwd    long.py:492-579 (three linear recurrences plus glue);
 *                          the backward is the chain rule through those recurrences.
 *   oracle_tape_stats      read.py:58-72, 154-183 (means over H, norms, key bias,
 *                          admission, cocktail).
 *   oracle_bank_select     read.py:185-239 (cummax floor, member, stable partition).
 *   oracle_permanent_fwd/bwd  cpu_runtime.cpp:1075-1188 (delta scan and its reverse).
 *   oracle_field_gather/_bwd  cpu_runtime.cpp:1191-1237 (patch gather, scatter-add).
 *   oracle_ce_fwd/bwd      runtime/loss.py:83-93, 105-133 (cross-entropy rows).
 *
 * Deliberate deviation: cpu_runtime.cpp:381 and :571 skip a pathway whose gain is
 * exactly 0, which also zeroes that gain's gradient. The read's math oracle
 * (admitted.py:126-239) does not skip, so its gain gradient is the true one. This
 * restatement follows admitted.py for that case (identical whenever gain != 0).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }
static inline float softplus_(float x) { return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))); }
static inline float hardsig(float x) { return fminf(fmaxf(x + 3.0f, 0.0f), 6.0f) * (1.0f / 6.0f); }
static inline float clamp01(float x) { return fminf(fmaxf(x, 0.0f), 1.0f); }
static inline float signf_(float x) { return (float)((x > 0.0f) - (x < 0.0f)); }

int oracle_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* Per-unit parameter vectors, in the order of the registered op's inputs 4..19
 * (batched_runtime.py:1507-1535). */
enum {
  P_BETA = 0, P_LOG_KAPPA, P_LOGIT_RECOVER, P_KS, P_KY, P_KB, P_KN, P_KBIAS,
  P_RS, P_RY, P_RB, P_RN, P_RBIAS, P_LOGIT_CDECAY, P_KC, P_RC, P_COUNT
};

/* ---------------------------------------------------------------------------
 * Core scan forward. GA is [Ug; A] row-major (2H, H). Outputs follow the
 * registered op's 11-output order: U [B,T,2H], novelty, plasticity, expression,
 * write, energy (pre-update e), saturation (post-update c), gate, final b/e/c.
 * ------------------------------------------------------------------------- */
void oracle_core_scan_fwd(int64_t B, int64_t T, int64_t H,
                          const float* Wx, const float* Wgx, const float* GA,
                          const float* const* vec, float logit_alpha, float log_lambda,
                          float logit_c_suppress, const float* b0, const float* e0,
                          const float* c0, float* U, float* Nov, float* Pl, float* Ay,
                          float* Wr, float* Et, float* Ct, float* St, float* bF, float* eF,
                          float* cF) {
  const float gate_alpha = sigm(logit_alpha);
  const float lam = softplus_(log_lambda);
  const float c_suppress = sigm(logit_c_suppress);
  int64_t bi;
  /* Rows are independent: with a single row the matvec's output units are split over the
   * threads instead (each unit's dot product keeps its serial order). */
#pragma omp parallel for schedule(static) if (B > 1)
  for (bi = 0; bi < B; ++bi) {
    float* b = (float*)malloc(sizeof(float) * H * 6);
    float* e = b + H;
    float* c = e + H;
    float* y = c + H;
    float* ug = y + H;
    float* ay = ug + H;
    for (int64_t i = 0; i < H; ++i) {
      b[i] = b0[bi * H + i];
      e[i] = e0[bi * H + i];
      c[i] = c0[bi * H + i];
    }
    for (int64_t t = 0; t < T; ++t) {
      const float* wx = Wx + (bi * T + t) * H;
      const float* wgx = Wgx + (bi * T + t) * H;
      for (int64_t i = 0; i < H; ++i) y[i] = tanhf(wx[i] + b[i]);
      int64_t i;
#pragma omp parallel for schedule(static) if (B == 1)
      for (i = 0; i < H; ++i) {
        const float* gu = GA + i * H;
        const float* ga = GA + (H + i) * H;
        float su = 0.0f, sa = 0.0f;
        for (int64_t j = 0; j < H; ++j) {
          su += gu[j] * y[j];
          sa += ga[j] * y[j];
        }
        ug[i] = su;
        ay[i] = sa;
      }
      float* up = U + (bi * T + t) * 2 * H;
      const int64_t off = (bi * T + t) * H;
      for (int64_t i = 0; i < H; ++i) {
        const float b_0 = b[i], e_0 = e[i], c_0 = c[i];
        const float s = hardsig(wgx[i] + ug[i]);
        const float nov = tanhf(fabsf(ay[i] - b_0));
        const float decay = sigm(vec[P_LOGIT_CDECAY][i]);
        const float stress = nov * (1.0f - e_0);
        const float cpost = decay * c_0 + (1.0f - decay) * stress;
        const float nov_eff = nov * (1.0f - c_suppress * cpost);
        const float tb = tanhf(b_0);
        float k_sig = vec[P_KS][i] * s + vec[P_KY][i] * y[i] + vec[P_KB][i] * tb +
                      vec[P_KN][i] * nov_eff + vec[P_KBIAS][i];
        float r_sig = vec[P_RS][i] * s + vec[P_RY][i] * y[i] + vec[P_RB][i] * tb +
                      vec[P_RN][i] * nov_eff + vec[P_RBIAS][i];
        k_sig += vec[P_KC][i] * cpost;
        r_sig += vec[P_RC][i] * cpost;
        const float kappa = softplus_(vec[P_LOG_KAPPA][i]);
        const float recover = sigm(vec[P_LOGIT_RECOVER][i]);
        const float k_t = kappa * expf(0.5f * tanhf(k_sig));
        const float r_t = clamp01(recover * expf(0.5f * tanhf(r_sig)));
        const float p = s * e_0;
        const float write = p * ay[i];
        const float bn = (1.0f - gate_alpha) * b_0 + vec[P_BETA][i] + lam * (p * ay[i]);
        const float en = clamp01(e_0 + r_t * (1.0f - e_0) - k_t * p);
        up[i] = y[i];
        up[H + i] = bn;
        Nov[off + i] = nov;
        Pl[off + i] = p;
        Ay[off + i] = ay[i];
        Wr[off + i] = write;
        Et[off + i] = e_0;
        Ct[off + i] = cpost;
        St[off + i] = s;
        b[i] = bn;
        e[i] = en;
        c[i] = cpost;
      }
    }
    for (int64_t i = 0; i < H; ++i) {
      bF[bi * H + i] = b[i];
      eF[bi * H + i] = e[i];
      cF[bi * H + i] = c[i];
    }
    free(b);
  }
}

/* ---------------------------------------------------------------------------
 * Core scan backward (registered reverse recurrence). Any grad pointer may be
 * NULL (treated as zeros). Outputs: gWx, gWgx [B,T,H]; gGA [2H,H];
 * gvec [16][H]; gscal[3] = (logit_alpha, log_lambda, logit_c_suppress);
 * gb0, ge0, gc0 [B,H]. day_scratch is caller-provided [B,T,H] scratch.
 * ------------------------------------------------------------------------- */
void oracle_core_scan_bwd(int64_t B, int64_t T, int64_t H, const float* GA,
                          const float* const* vec, float logit_alpha, float log_lambda,
                          float logit_c_suppress, const float* b0, const float* c0,
                          const float* U, const float* Pl, const float* Ay, const float* Et,
                          const float* Ct, const float* St, const float* gU, const float* gNov,
                          const float* gP, const float* gAy, const float* gW, const float* gE,
                          const float* gC, const float* gbF, const float* geF, const float* gcF,
                          float* gWx, float* gWgx, float* day_scratch, float* gGA, float* gvec,
                          float* gscal, float* gb0, float* ge0, float* gc0) {
  const float alpha = sigm(logit_alpha);
  const float lam = softplus_(log_lambda);
  const float sig_lam = sigm(log_lambda);
  const float suppress = sigm(logit_c_suppress);
  float* part_vec = (float*)calloc((size_t)B * P_COUNT * H, sizeof(float));
  float* part_scal = (float*)calloc((size_t)B * 3, sizeof(float));
  /* [Ug; A] transposed once, so the recurrent adjoint below reads each unit's 2H weights
   * contiguously; its sums run over r in the same order as through GA's columns. */
  float* GAT = (float*)malloc(sizeof(float) * 2 * H * H);
  for (int64_t r0 = 0; r0 < 2 * H; ++r0)
    for (int64_t j = 0; j < H; ++j) GAT[j * 2 * H + r0] = GA[r0 * H + j];
  int64_t bi;
#pragma omp parallel for schedule(static) if (B > 1)
  for (bi = 0; bi < B; ++bi) {
    float* gbn = (float*)calloc((size_t)H * 6, sizeof(float));
    float* gen = gbn + H;
    float* gcn = gen + H;
    float* dg = gcn + H;  /* [2H]: dgate_pre then d_expression */
    float* gyx = dg + 2 * H; /* gy0 + gy_energy per unit */
    float* acc = part_vec + bi * P_COUNT * H;
    float* sacc = part_scal + bi * 3;
    /* per-unit values kept from the first pass to the second */
    float* keep = (float*)malloc(sizeof(float) * H * 4);
    for (int64_t i = 0; i < H; ++i) {
      gbn[i] = gbF ? gbF[bi * H + i] : 0.0f;
      gen[i] = geF ? geF[bi * H + i] : 0.0f;
      gcn[i] = gcF ? gcF[bi * H + i] : 0.0f;
    }
    for (int64_t t = T - 1; t >= 0; --t) {
      const int64_t off = (bi * T + t) * H;
      const float* u_t = U + (bi * T + t) * 2 * H;
      for (int64_t i = 0; i < H; ++i) {
        const float y = u_t[i];
        const float b_prev = t > 0 ? U[(bi * T + t - 1) * 2 * H + H + i] : b0[bi * H + i];
        const float e_prev = Et[off + i];
        const float c_prev = t > 0 ? Ct[off - H + i] : c0[bi * H + i];
        const float gate = St[off + i];
        const float p = Pl[off + i];
        const float ay = Ay[off + i];
        const float nov = tanhf(fabsf(ay - b_prev));
        const float c_t = Ct[off + i];
        const float gy0 = gU ? gU[(bi * T + t) * 2 * H + i] : 0.0f;
        const float gb_new = (gU ? gU[(bi * T + t) * 2 * H + H + i] : 0.0f) + gbn[i];
        const float gc_new = gcn[i] + (gC ? gC[off + i] : 0.0f);
        const float gnov0 = gNov ? gNov[off + i] : 0.0f;
        const float gp0 = gP ? gP[off + i] : 0.0f;
        const float gay0 = gAy ? gAy[off + i] : 0.0f;
        const float gwrite = gW ? gW[off + i] : 0.0f;

        const float kappa = softplus_(vec[P_LOG_KAPPA][i]);
        const float recover = sigm(vec[P_LOGIT_RECOVER][i]);
        const float decay = sigm(vec[P_LOGIT_CDECAY][i]);
        const float tanh_b = tanhf(b_prev);
        const float nov_eff = nov * (1.0f - suppress * c_t);
        const float k_signal = vec[P_KS][i] * gate + vec[P_KY][i] * y + vec[P_KB][i] * tanh_b +
                               vec[P_KN][i] * nov_eff + vec[P_KBIAS][i] + vec[P_KC][i] * c_t;
        const float r_signal = vec[P_RS][i] * gate + vec[P_RY][i] * y + vec[P_RB][i] * tanh_b +
                               vec[P_RN][i] * nov_eff + vec[P_RBIAS][i] + vec[P_RC][i] * c_t;
        const float tanh_k = tanhf(k_signal), tanh_r = tanhf(r_signal);
        const float exp_k = expf(0.5f * tanh_k), exp_r = expf(0.5f * tanh_r);
        const float write_cost = kappa * exp_k;
        const float recovery_pre = recover * exp_r;
        const float recovery = clamp01(recovery_pre);
        const float rclamp = (recovery_pre >= 0.0f && recovery_pre <= 1.0f) ? 1.0f : 0.0f;
        const float energy_pre = e_prev + recovery * (1.0f - e_prev) - write_cost * p;
        const float ge_pre = gen[i] * ((energy_pre >= 0.0f && energy_pre <= 1.0f) ? 1.0f : 0.0f);
        const float g_bprev_state = gb_new * (1.0f - alpha);
        const float g_eprev_state = ge_pre * (1.0f - recovery);
        float gp = gp0 + gb_new * lam * ay - ge_pre * write_cost;
        const float gay = gay0 + gb_new * lam * p;
        const float g_write_cost = -ge_pre * p;
        const float g_recovery = ge_pre * (1.0f - e_prev);
        const float d_expr_main = gay + gwrite * p;
        gp = gp + gwrite * ay;
        const float g_k = g_write_cost * write_cost * 0.5f * (1.0f - tanh_k * tanh_k);
        const float g_rpre = g_recovery * rclamp;
        const float g_r = g_rpre * recovery_pre * 0.5f * (1.0f - tanh_r * tanh_r);
        const float g_gate_energy = g_k * vec[P_KS][i] + g_r * vec[P_RS][i];
        const float gy_energy = g_k * vec[P_KY][i] + g_r * vec[P_RY][i];
        const float gb_energy = (g_k * vec[P_KB][i] + g_r * vec[P_RB][i]) * (1.0f - tanh_b * tanh_b);
        const float gnov_eff = g_k * vec[P_KN][i] + g_r * vec[P_RN][i];
        const float gc_energy = g_k * vec[P_KC][i] + g_r * vec[P_RC][i];
        const float dgate_pre =
            (gp * e_prev + g_gate_energy) * (((gate > 0.0f) && (gate < 1.0f)) ? (1.0f / 6.0f) : 0.0f);
        const float ge_gate = gp * gate;
        const float stress = nov * (1.0f - e_prev);
        const float c_new = decay * c_prev + (1.0f - decay) * stress;
        const float g_c_new = gc_new + gc_energy - gnov_eff * nov * suppress;
        const float g_stress = g_c_new * (1.0f - decay);
        const float g_nov = gnov_eff * (1.0f - suppress * c_new) + g_stress * (1.0f - e_prev);
        const float g_e_prev_cort = -g_stress * nov;
        const float g_c_prev = g_c_new * decay;
        const float diff = ay - b_prev;
        const float nov_check = tanhf(fabsf(diff));
        const float d_nov = (gnov0 + g_nov) * (1.0f - nov_check * nov_check) * signf_(diff);
        const float d_expr = d_expr_main + d_nov;

        dg[i] = dgate_pre;
        dg[H + i] = d_expr;
        gyx[i] = gy0 + gy_energy;
        keep[i] = g_bprev_state + gb_energy - d_nov;
        keep[H + i] = g_eprev_state + ge_gate + g_e_prev_cort + (gE ? gE[off + i] : 0.0f);
        keep[2 * H + i] = g_c_prev;

        acc[P_BETA * H + i] += gb_new;
        acc[P_LOG_KAPPA * H + i] += g_write_cost * exp_k * sigm(vec[P_LOG_KAPPA][i]);
        acc[P_LOGIT_RECOVER * H + i] += g_rpre * exp_r * recover * (1.0f - recover);
        acc[P_KS * H + i] += g_k * gate;
        acc[P_KY * H + i] += g_k * y;
        acc[P_KB * H + i] += g_k * tanh_b;
        acc[P_KN * H + i] += g_k * nov_eff;
        acc[P_KBIAS * H + i] += g_k;
        acc[P_RS * H + i] += g_r * gate;
        acc[P_RY * H + i] += g_r * y;
        acc[P_RB * H + i] += g_r * tanh_b;
        acc[P_RN * H + i] += g_r * nov_eff;
        acc[P_RBIAS * H + i] += g_r;
        acc[P_LOGIT_CDECAY * H + i] += g_c_new * (c_prev - stress) * decay * (1.0f - decay);
        acc[P_KC * H + i] += g_k * c_t;
        acc[P_RC * H + i] += g_r * c_t;
        sacc[0] += gb_new * (-b_prev) * alpha * (1.0f - alpha);
        sacc[1] += gb_new * (p * ay) * sig_lam;
        sacc[2] += gnov_eff * nov * (-c_new) * suppress * (1.0f - suppress);
      }
      /* recurrent adjoint: [dgate_pre; d_expr] @ [Ug; A] -> [H] (a single row splits the
       * units over the threads) */
      int64_t j;
#pragma omp parallel for schedule(static) if (B == 1)
      for (j = 0; j < H; ++j) {
        float s = 0.0f;
        const float* gat = GAT + j * 2 * H;
        for (int64_t r = 0; r < 2 * H; ++r) s += dg[r] * gat[r];
        const float y = u_t[j];
        const float gy = gyx[j] + s;
        const float gpre = gy * (1.0f - y * y);
        gWx[off + j] = gpre;
        gWgx[off + j] = dg[j];
        day_scratch[off + j] = dg[H + j];
        gbn[j] = keep[j] + gpre;
        gen[j] = keep[H + j];
        gcn[j] = keep[2 * H + j];
      }
    }
    for (int64_t i = 0; i < H; ++i) {
      gb0[bi * H + i] = gbn[i];
      ge0[bi * H + i] = gen[i];
      gc0[bi * H + i] = gcn[i];
    }
    free(keep);
    free(gbn);
  }
  /* reduce per-batch partials in batch order */
  for (int64_t k = 0; k < P_COUNT * H; ++k) {
    float s = 0.0f;
    for (int64_t b = 0; b < B; ++b) s += part_vec[b * P_COUNT * H + k];
    gvec[k] = s;
  }
  for (int k = 0; k < 3; ++k) {
    float s = 0.0f;
    for (int64_t b = 0; b < B; ++b) s += part_scal[b * 3 + k];
    gscal[k] = s;
  }
  free(part_vec);
  free(part_scal);
  free(GAT);
  /* grad [Ug; A] = [gWgx; day]^T @ y over all (b, t) */
  int64_t r;
#pragma omp parallel for schedule(static)
  for (r = 0; r < 2 * H; ++r) {
    const float* src = r < H ? gWgx : day_scratch;
    const int64_t rr = r < H ? r : r - H;
    float* out = gGA + r * H;
    for (int64_t j = 0; j < H; ++j) out[j] = 0.0f;
    for (int64_t bt = 0; bt < B * T; ++bt) {
      const float d = src[bt * H + rr];
      const float* y = U + bt * 2 * H;
      for (int64_t j = 0; j < H; ++j) out[j] += d * y[j];
    }
  }
}

/* ---------------------------------------------------------------------------
 * Three-way admitted read (compact ABI). idx/valid [B,N]; mode 0 = seq
 * (allow idx<=t, induct idx<t), mode 1 = field (allow valid, induct idx<T-1).
 * Query positions are query_offset + t; total_steps is the field-mode T.
 * ------------------------------------------------------------------------- */
static inline int allow_at(int mode, int64_t idx, uint8_t valid, int64_t pos, int64_t total) {
  (void)total;
  if (!valid) return 0;
  return mode == 0 ? (idx <= pos) : 1;
}
static inline int induct_at(int mode, int64_t idx, uint8_t valid, int64_t pos, int64_t total) {
  if (!valid) return 0;
  return mode == 0 ? (idx < pos) : (idx < total - 1);
}

static float score_of(const float* q, const float* k, int64_t H, float scale, float kbj,
                      float admj, int perm, const float* ct, const float* cbj, int64_t C,
                      float cgain) {
  float dot = 0.0f;
  for (int64_t h = 0; h < H; ++h) dot += q[h] * k[h];
  float s = dot * scale + kbj + admj;
  if (perm) {
    float cd = 0.0f;
    for (int64_t c = 0; c < C; ++c) cd += ct[c] * cbj[c];
    s += cd * cgain;
  }
  return s;
}

void oracle_read3_fwd(int64_t B, int64_t T, int64_t N, int64_t H, int64_t C, const float* q,
                      const float* K, const float* V, const float* Vn, const float* ck,
                      const float* cb, const float* kb, const float* adm, float scale,
                      const int64_t* idx, const uint8_t* valid, int mode, int64_t query_offset,
                      int64_t total_steps, float sg, float pg, float ig, float cg, float* out) {
  int64_t bt;
#pragma omp parallel for schedule(static)
  for (bt = 0; bt < B * T; ++bt) {
    const int64_t bi = bt / T, ti = bt % T;
    const int64_t pos = query_offset + ti;
    const float* qt = q + bt * H;
    const float* ct = ck + bt * C;
    float* o = out + bt * H;
    for (int64_t h = 0; h < H; ++h) o[h] = 0.0f;
    for (int path = 0; path < 3; ++path) {
      const int perm = path == 1;
      const float gain = path == 0 ? sg : (path == 1 ? pg : ig);
      const float* vals = path == 2 ? Vn : V;
      float mx = -INFINITY;
      for (int64_t j = 0; j < N; ++j) {
        const int ok = path == 2 ? induct_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps)
                                 : allow_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps);
        if (!ok) continue;
        const float s = score_of(qt, K + (bi * N + j) * H, H, scale, kb[bi * N + j], adm[bi * N + j],
                                 perm, ct, cb + (bi * N + j) * C, C, cg);
        mx = fmaxf(mx, s);
      }
      if (mx == -INFINITY) continue;
      float den = 0.0f;
      for (int64_t j = 0; j < N; ++j) {
        const int ok = path == 2 ? induct_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps)
                                 : allow_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps);
        if (!ok) continue;
        den += expf(score_of(qt, K + (bi * N + j) * H, H, scale, kb[bi * N + j], adm[bi * N + j],
                             perm, ct, cb + (bi * N + j) * C, C, cg) - mx);
      }
      if (den <= 0.0f) continue;
      for (int64_t j = 0; j < N; ++j) {
        const int ok = path == 2 ? induct_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps)
                                 : allow_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps);
        if (!ok) continue;
        const float s = score_of(qt, K + (bi * N + j) * H, H, scale, kb[bi * N + j], adm[bi * N + j],
                                 perm, ct, cb + (bi * N + j) * C, C, cg);
        const float wgt = gain * expf(s - mx) / den;
        const float* v = vals + (bi * N + j) * H;
        for (int64_t h = 0; h < H; ++h) o[h] += wgt * v[h];
      }
    }
  }
}

/* Backward of oracle_read3_fwd. Outputs (all zero-initialised here):
 * gq [B,T,H], gK, gV, gVn [B,N,H], gck [B,T,C], gcb [B,N,C], gkb, gadm [B,N],
 * gsc[5] = (scale, short_gain, pad_gain, induct_gain, cocktail_gain). */
void oracle_read3_bwd(int64_t B, int64_t T, int64_t N, int64_t H, int64_t C, const float* go,
                      const float* q, const float* K, const float* V, const float* Vn,
                      const float* ck, const float* cb, const float* kb, const float* adm,
                      float scale, const int64_t* idx, const uint8_t* valid, int mode,
                      int64_t query_offset, int64_t total_steps, float sg, float pg, float ig,
                      float cg, float* gq, float* gK, float* gV, float* gVn, float* gck,
                      float* gcb, float* gkb, float* gadm, float* gsc) {
  memset(gq, 0, sizeof(float) * B * T * H);
  memset(gK, 0, sizeof(float) * B * N * H);
  memset(gV, 0, sizeof(float) * B * N * H);
  memset(gVn, 0, sizeof(float) * B * N * H);
  memset(gck, 0, sizeof(float) * B * T * C);
  memset(gcb, 0, sizeof(float) * B * N * C);
  memset(gkb, 0, sizeof(float) * B * N);
  memset(gadm, 0, sizeof(float) * B * N);
  float* part = (float*)calloc((size_t)B * 5, sizeof(float));
  int64_t bi;
#pragma omp parallel for schedule(static)
  for (bi = 0; bi < B; ++bi) {
    float* w = (float*)malloc(sizeof(float) * N * 2);
    float* gdv = w + N;
    float* pb = part + bi * 5;
    for (int64_t ti = 0; ti < T; ++ti) {
      const int64_t bt = bi * T + ti;
      const int64_t pos = query_offset + ti;
      const float* qt = q + bt * H;
      const float* ct = ck + bt * C;
      const float* g = go + bt * H;
      for (int path = 0; path < 3; ++path) {
        const int perm = path == 1;
        const float gain = path == 0 ? sg : (path == 1 ? pg : ig);
        const float* vals = path == 2 ? Vn : V;
        float* gvals = path == 2 ? gVn : gV;
        float mx = -INFINITY;
        for (int64_t j = 0; j < N; ++j) {
          w[j] = 0.0f;
          gdv[j] = 0.0f;
          const int ok = path == 2 ? induct_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps)
                                   : allow_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps);
          if (!ok) continue;
          const float s = score_of(qt, K + (bi * N + j) * H, H, scale, kb[bi * N + j],
                                   adm[bi * N + j], perm, ct, cb + (bi * N + j) * C, C, cg);
          mx = fmaxf(mx, s);
        }
        if (mx == -INFINITY) continue;
        float den = 0.0f;
        for (int64_t j = 0; j < N; ++j) {
          const int ok = path == 2 ? induct_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps)
                                   : allow_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps);
          if (!ok) continue;
          const float ex = expf(score_of(qt, K + (bi * N + j) * H, H, scale, kb[bi * N + j],
                                         adm[bi * N + j], perm, ct, cb + (bi * N + j) * C, C, cg) -
                                mx);
          w[j] = ex;
          den += ex;
        }
        if (den <= 0.0f) continue;
        float dot_go_read = 0.0f;
        for (int64_t j = 0; j < N; ++j) {
          const int ok = path == 2 ? induct_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps)
                                   : allow_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps);
          if (!ok) continue;
          w[j] /= den;
          const float* v = vals + (bi * N + j) * H;
          float d = 0.0f;
          for (int64_t h = 0; h < H; ++h) {
            d += g[h] * v[h];
            gvals[(bi * N + j) * H + h] += gain * w[j] * g[h];
          }
          gdv[j] = d;
          dot_go_read += w[j] * d;
        }
        pb[1 + path] += dot_go_read;
        for (int64_t j = 0; j < N; ++j) {
          const int ok = path == 2 ? induct_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps)
                                   : allow_at(mode, idx[bi * N + j], valid[bi * N + j], pos, total_steps);
          if (!ok) continue;
          const float dz = gain * w[j] * (gdv[j] - dot_go_read);
          const float* kv = K + (bi * N + j) * H;
          float kd = 0.0f;
          for (int64_t h = 0; h < H; ++h) {
            kd += qt[h] * kv[h];
            gq[bt * H + h] += dz * scale * kv[h];
            gK[(bi * N + j) * H + h] += dz * scale * qt[h];
          }
          gkb[bi * N + j] += dz;
          gadm[bi * N + j] += dz;
          pb[0] += dz * kd;
          if (perm) {
            const float* cbj = cb + (bi * N + j) * C;
            float cd = 0.0f;
            for (int64_t c = 0; c < C; ++c) {
              cd += ct[c] * cbj[c];
              gck[bt * C + c] += dz * cg * cbj[c];
              gcb[(bi * N + j) * C + c] += dz * cg * ct[c];
            }
            pb[4] += dz * cd;
          }
        }
      }
    }
    free(w);
  }
  for (int k = 0; k < 5; ++k) {
    float s = 0.0f;
    for (int64_t b = 0; b < B; ++b) s += part[b * 5 + k];
    gsc[k] = s;
  }
  free(part);
}

/* ---------------------------------------------------------------------------
 * Diagonal linear recurrence y_t = a_t y_{t-1} + g_t (cpu_runtime.cpp:92-143).
 * ------------------------------------------------------------------------- */
void oracle_linrec_fwd(int64_t B, int64_t T, int64_t H, const float* a, const float* g,
                       const float* y0, float* out) {
  int64_t bi;
#pragma omp parallel for schedule(static)
  for (bi = 0; bi < B; ++bi) {
    for (int64_t h = 0; h < H; ++h) {
      float carry = y0[bi * H + h];
      for (int64_t t = 0; t < T; ++t) {
        const int64_t off = (bi * T + t) * H + h;
        carry = a[off] * carry + g[off];
        out[off] = carry;
      }
    }
  }
}

void oracle_linrec_bwd(int64_t B, int64_t T, int64_t H, const float* a, const float* g,
                       const float* y0, const float* gy, float* da, float* dg, float* dy0) {
  int64_t bi;
#pragma omp parallel for schedule(static)
  for (bi = 0; bi < B; ++bi) {
    float* yprev = (float*)malloc(sizeof(float) * T);
    for (int64_t h = 0; h < H; ++h) {
      float carry = y0[bi * H + h];
      for (int64_t t = 0; t < T; ++t) {
        const int64_t off = (bi * T + t) * H + h;
        yprev[t] = carry;
        carry = a[off] * carry + g[off];
      }
      float c = 0.0f;
      for (int64_t t = T - 1; t >= 0; --t) {
        const int64_t off = (bi * T + t) * H + h;
        const float a_next = (t + 1 < T) ? a[off + H] : 0.0f;
        c = gy[off] + a_next * c;
        dg[off] = c;
        da[off] = c * yprev[t];
      }
      dy0[bi * H + h] = a[(bi * T) * H + h] * c;
    }
    free(yprev);
  }
}

/* ---------------------------------------------------------------------------
 * Recurrent long-memory scan (long.py:492-579 / read.py:625-636). coef[4] =
 * (expect_retain, retention_decay, retain, retention_strength), already passed
 * through sigmoid. State (L, E, R) enters as L0, E0, R0 and leaves as LF, EF, RF.
 * ------------------------------------------------------------------------- */
void oracle_long_fwd(int64_t B, int64_t T, int64_t H, const float* w, const float* p,
                     const float* coef, const float* L0, const float* E0, const float* R0,
                     float* out, float* LF, float* EF, float* RF) {
  const float er = coef[0], rd = coef[1], ret = coef[2], rs = coef[3];
  int64_t bi;
#pragma omp parallel for schedule(static)
  for (bi = 0; bi < B; ++bi) {
    for (int64_t h = 0; h < H; ++h) {
      float L = L0[bi * H + h], E = E0[bi * H + h], R = R0[bi * H + h];
      for (int64_t t = 0; t < T; ++t) {
        const int64_t off = (bi * T + t) * H + h;
        const float wt = w[off];
        const float pe = tanhf(fabsf(wt - E));
        const float sal = p[off] * pe;
        E = er * E + (1.0f - er) * wt;
        R = rd * R + (1.0f - rd) * (1.0f - pe);
        const float eff = ret + (1.0f - ret) * rs * R;
        L = eff * L + (1.0f - eff) * (sal * wt);
        out[off] = L;
      }
      LF[bi * H + h] = L;
      EF[bi * H + h] = E;
      RF[bi * H + h] = R;
    }
  }
}

/* Backward of oracle_long_fwd. gout [B,T,H]; gLF/gEF/gRF may be NULL. Outputs
 * gw, gp [B,T,H], gL0, gE0, gR0 [B,H], gcoef[4] (w.r.t. the sigmoid outputs). */
void oracle_long_bwd(int64_t B, int64_t T, int64_t H, const float* w, const float* p,
                     const float* coef, const float* L0, const float* E0, const float* R0,
                     const float* gout, const float* gLF, const float* gEF, const float* gRF,
                     float* gw, float* gp, float* gL0, float* gE0, float* gR0, float* gcoef) {
  const float er = coef[0], rd = coef[1], ret = coef[2], rs = coef[3];
  float* part = (float*)calloc((size_t)B * 4, sizeof(float));
  int64_t bi;
#pragma omp parallel for schedule(static)
  for (bi = 0; bi < B; ++bi) {
    float* Ls = (float*)malloc(sizeof(float) * (T + 1) * 3);
    float* Es = Ls + (T + 1);
    float* Rs = Es + (T + 1);
    float* pa = part + bi * 4;
    for (int64_t h = 0; h < H; ++h) {
      Ls[0] = L0[bi * H + h];
      Es[0] = E0[bi * H + h];
      Rs[0] = R0[bi * H + h];
      for (int64_t t = 0; t < T; ++t) {
        const int64_t off = (bi * T + t) * H + h;
        const float wt = w[off];
        const float pe = tanhf(fabsf(wt - Es[t]));
        const float sal = p[off] * pe;
        Es[t + 1] = er * Es[t] + (1.0f - er) * wt;
        Rs[t + 1] = rd * Rs[t] + (1.0f - rd) * (1.0f - pe);
        const float eff = ret + (1.0f - ret) * rs * Rs[t + 1];
        Ls[t + 1] = eff * Ls[t] + (1.0f - eff) * (sal * wt);
      }
      float gLc = gLF ? gLF[bi * H + h] : 0.0f;
      float gEc = gEF ? gEF[bi * H + h] : 0.0f;
      float gRc = gRF ? gRF[bi * H + h] : 0.0f;
      for (int64_t t = T - 1; t >= 0; --t) {
        const int64_t off = (bi * T + t) * H + h;
        const float wt = w[off], pt = p[off];
        const float Eprev = Es[t], Rcur = Rs[t + 1], Rprev = Rs[t], Lprev = Ls[t];
        const float diff = wt - Eprev;
        const float pe = tanhf(fabsf(diff));
        const float sal = pt * pe;
        const float eff = ret + (1.0f - ret) * rs * Rcur;
        const float gL = gout[off] + gLc;
        const float deff = gL * (Lprev - sal * wt);
        const float dsal = gL * (1.0f - eff) * wt;
        float dw = gL * (1.0f - eff) * sal;
        gLc = gL * eff;
        const float dR = gRc + deff * (1.0f - ret) * rs;
        gRc = dR * rd;
        const float dpe = dsal * pt - dR * (1.0f - rd);
        gp[off] = dsal * pe;
        const float darg = dpe * (1.0f - pe * pe) * signf_(diff);
        dw += darg;
        const float dE = gEc;
        dw += (1.0f - er) * dE;
        gEc = er * dE - darg;
        gw[off] = dw;
        pa[0] += dE * (Eprev - wt);
        pa[1] += dR * (Rprev - (1.0f - pe));
        pa[2] += deff * (1.0f - rs * Rcur);
        pa[3] += deff * (1.0f - ret) * Rcur;
      }
      gL0[bi * H + h] = gLc;
      gE0[bi * H + h] = gEc;
      gR0[bi * H + h] = gRc;
    }
    free(Ls);
  }
  for (int k = 0; k < 4; ++k) {
    float s = 0.0f;
    for (int64_t b = 0; b < B; ++b) s += part[b * 4 + k];
    gcoef[k] = s;
  }
  free(part);
}

/* ---------------------------------------------------------------------------
 * Per-position read statistics (read.py:58-72, 154-183). gains[10] =
 * (p_gain, novelty_gain, null_bias, adm_p, adm_n, adm_s, adm_e, adm_bias, -, -).
 * Outputs per (b,t): means[4] = (e, c, n, p), norm_ay, norm_w, key_bias,
 * admission, cocktail[4].
 * ------------------------------------------------------------------------- */
void oracle_tape_stats(int64_t B, int64_t T, int64_t H, const float* nov, const float* pl,
                       const float* en, const float* sat, const float* ay, const float* wr,
                       const float* gains, float* means, float* norm_ay, float* norm_w,
                       float* key_bias, float* admission, float* cocktail) {
  int64_t bt;
#pragma omp parallel for schedule(static)
  for (bt = 0; bt < B * T; ++bt) {
    double sn = 0, sp = 0, se = 0, sc = 0, sa = 0, sw = 0;
    for (int64_t h = 0; h < H; ++h) {
      const int64_t off = bt * H + h;
      sn += nov[off];
      sp += pl[off];
      se += en[off];
      sc += sat[off];
      sa += (double)ay[off] * ay[off];
      sw += (double)wr[off] * wr[off];
    }
    const float mn = (float)(sn / H), mp = (float)(sp / H), me = (float)(se / H),
                mc = (float)(sc / H);
    means[bt * 4 + 0] = me;
    means[bt * 4 + 1] = mc;
    means[bt * 4 + 2] = mn;
    means[bt * 4 + 3] = mp;
    norm_ay[bt] = (float)sqrt(sa);
    norm_w[bt] = (float)sqrt(sw);
    const float lp = log1pf(mp * (float)H);
    key_bias[bt] = gains[0] * lp + gains[1] * mn + gains[2];
    admission[bt] = gains[3] * lp + gains[4] * mn + gains[5] * mc + gains[6] * me + gains[7];
    const float cn = fmaxf(sqrtf(me * me + mc * mc + mn * mn + mp * mp), 1e-12f);
    cocktail[bt * 4 + 0] = me / cn;
    cocktail[bt * 4 + 1] = mc / cn;
    cocktail[bt * 4 + 2] = mn / cn;
    cocktail[bt * 4 + 3] = mp / cn;
  }
}

/* ---------------------------------------------------------------------------
 * Admitted-slot selection (read.py:185-239), seq geometry. For each row:
 * floor_t = cummax_{tau<=t} adm - window; member = adm >= floor; order is the
 * stable descending argsort of member (members by ascending t, then the rest by
 * ascending t). Writes the full permutation order[B,T] and counts[B].
 * ------------------------------------------------------------------------- */
void oracle_bank_select(int64_t B, int64_t T, const float* adm, float window, int64_t* order,
                        int64_t* counts) {
  int64_t bi;
#pragma omp parallel for schedule(static)
  for (bi = 0; bi < B; ++bi) {
    const float* a = adm + bi * T;
    int64_t* o = order + bi * T;
    float run = -INFINITY;
    int64_t cnt = 0;
    for (int64_t t = 0; t < T; ++t) {
      run = (t == 0 || a[t] > run) ? a[t] : run;
      if (a[t] >= run - window) ++cnt;
    }
    counts[bi] = cnt;
    int64_t mpos = 0, npos = cnt;
    run = -INFINITY;
    for (int64_t t = 0; t < T; ++t) {
      run = (t == 0 || a[t] > run) ? a[t] : run;
      if (a[t] >= run - window) o[mpos++] = t;
      else o[npos++] = t;
    }
  }
}

/* ---------------------------------------------------------------------------
 * Permanent associative delta scan (cpu_runtime.cpp:1075-1109; definition
 * permanent.py:39-51). Per batch row: S [H][H] = 0; for each step the output row
 * is S k (serial dot over the key index), then every value row moves by
 * beta * (v - out) along k.
 * ------------------------------------------------------------------------- */
void oracle_permanent_fwd(int64_t B, int64_t T, int64_t H, const float* k, const float* v,
                          const float* beta, float* out) {
  int64_t bi;
#pragma omp parallel for schedule(static)
  for (bi = 0; bi < B; ++bi) {
    float* S = (float*)calloc((size_t)(H * H), sizeof(float));
    for (int64_t t = 0; t < T; ++t) {
      const float* kt = k + (bi * T + t) * H;
      const float* vt = v + (bi * T + t) * H;
      float* rt = out + (bi * T + t) * H;
      for (int64_t i = 0; i < H; ++i) {
        float acc = 0.0f;
        for (int64_t j = 0; j < H; ++j) acc += S[i * H + j] * kt[j];
        rt[i] = acc;
      }
      const float bt = beta[bi * T + t];
      for (int64_t i = 0; i < H; ++i) {
        const float step = bt * (vt[i] - rt[i]);
        for (int64_t j = 0; j < H; ++j) S[i * H + j] += step * kt[j];
      }
    }
    free(S);
  }
}

/* Reverse of the delta scan (cpu_runtime.cpp:1112-1188; permanent.py:70-119). The states
 * before each step are kept (T H^2 floats per batch row), then the adjoint A = dL/dS walks
 * back: Ak = A k, dv = beta Ak, dbeta = sum_i Ak_i (v_i - r_i), dk_j = sum_i (S_ij g_i +
 * beta A_ij v_i - beta S_ij Ak_i - beta A_ij r_i), A += g k^T - beta Ak k^T. */
void oracle_permanent_bwd(int64_t B, int64_t T, int64_t H, const float* k, const float* v,
                          const float* beta, const float* g, float* dk, float* dv, float* db) {
  int64_t bi;
#pragma omp parallel for schedule(static)
  for (bi = 0; bi < B; ++bi) {
    const size_t HH = (size_t)(H * H);
    float* tape = (float*)malloc(sizeof(float) * (size_t)T * HH);
    float* r = (float*)malloc(sizeof(float) * (size_t)(T * H));
    float* S = (float*)calloc(HH, sizeof(float));
    float* A = (float*)calloc(HH, sizeof(float));
    float* ak = (float*)malloc(sizeof(float) * (size_t)H);
    for (int64_t t = 0; t < T; ++t) {
      const float* kt = k + (bi * T + t) * H;
      const float* vt = v + (bi * T + t) * H;
      memcpy(tape + (size_t)t * HH, S, sizeof(float) * HH);
      for (int64_t i = 0; i < H; ++i) {
        float acc = 0.0f;
        for (int64_t j = 0; j < H; ++j) acc += S[i * H + j] * kt[j];
        r[t * H + i] = acc;
      }
      const float bt = beta[bi * T + t];
      for (int64_t i = 0; i < H; ++i) {
        const float step = bt * (vt[i] - r[t * H + i]);
        for (int64_t j = 0; j < H; ++j) S[i * H + j] += step * kt[j];
      }
    }
    for (int64_t t = T - 1; t >= 0; --t) {
      const float* kt = k + (bi * T + t) * H;
      const float* vt = v + (bi * T + t) * H;
      const float* gt = g + (bi * T + t) * H;
      const float* St = tape + (size_t)t * HH;
      const float* rt = r + t * H;
      const float bt = beta[bi * T + t];
      float dbt = 0.0f;
      for (int64_t i = 0; i < H; ++i) {
        float acc = 0.0f;
        for (int64_t j = 0; j < H; ++j) acc += A[i * H + j] * kt[j];
        ak[i] = acc;
        dv[(bi * T + t) * H + i] = bt * acc;
        dbt += acc * (vt[i] - rt[i]);
      }
      db[bi * T + t] = dbt;
      for (int64_t j = 0; j < H; ++j) {
        float acc = 0.0f;
        for (int64_t i = 0; i < H; ++i) {
          acc += St[i * H + j] * gt[i];
          acc += bt * A[i * H + j] * vt[i];
          acc -= bt * St[i * H + j] * ak[i];
          acc -= bt * A[i * H + j] * rt[i];
        }
        dk[(bi * T + t) * H + j] = acc;
      }
      for (int64_t i = 0; i < H; ++i)
        for (int64_t j = 0; j < H; ++j)
          A[i * H + j] = gt[i] * kt[j] + A[i * H + j] - bt * ak[i] * kt[j];
    }
    free(tape); free(r); free(S); free(A); free(ak);
  }
}

/* ---------------------------------------------------------------------------
 * Local field patch gather (cpu_runtime.cpp:1191-1237): out[b,p,j,:] = x[b,patch[p,j],:];
 * the backward adds grad rows back to their source cells, visiting (p, j) in order.
 * ------------------------------------------------------------------------- */
void oracle_field_gather(int64_t B, int64_t N, int64_t D, int64_t P, int64_t K, const float* x,
                         const int64_t* patch, float* out) {
  for (int64_t bi = 0; bi < B; ++bi)
    for (int64_t e = 0; e < P * K; ++e)
      memcpy(out + (bi * P * K + e) * D, x + (bi * N + patch[e]) * D, sizeof(float) * (size_t)D);
}

void oracle_field_gather_bwd(int64_t B, int64_t N, int64_t D, int64_t P, int64_t K,
                             const float* gout, const int64_t* patch, float* gx) {
  memset(gx, 0, sizeof(float) * (size_t)(B * N * D));
  for (int64_t bi = 0; bi < B; ++bi)
    for (int64_t e = 0; e < P * K; ++e) {
      float* dst = gx + (bi * N + patch[e]) * D;
      const float* src = gout + (bi * P * K + e) * D;
      for (int64_t d = 0; d < D; ++d) dst[d] += src[d];
    }
}

/* ---------------------------------------------------------------------------
 * Cross-entropy rows of the chunked readout loss (runtime/loss.py:83-93, 105-133): per
 * row, lse = max + log(sum exp(x - max)) (serial over the vocabulary), nll = lse - x[t]
 * (0 for ignored rows); backward d = (exp(x - lse) - [c == t]) * scale (0 rows ignored).
 * ------------------------------------------------------------------------- */
void oracle_ce_fwd(int64_t rows, int64_t V, const float* x, const int64_t* t, int64_t ignore,
                   float* lse, float* nll) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * V;
    float m = -INFINITY;
    for (int64_t c = 0; c < V; ++c) m = fmaxf(m, xr[c]);
    float s = 0.0f;
    for (int64_t c = 0; c < V; ++c) s += expf(xr[c] - m);
    lse[r] = m + logf(s);
    nll[r] = (t[r] == ignore) ? 0.0f : lse[r] - xr[t[r]];
  }
}

void oracle_ce_bwd(int64_t rows, int64_t V, const float* x, const int64_t* t, int64_t ignore,
                   const float* lse, float scale, float* d) {
  for (int64_t r = 0; r < rows; ++r) {
    const float sc = (t[r] == ignore) ? 0.0f : scale;
    for (int64_t c = 0; c < V; ++c)
      d[r * V + c] = (expf(x[r * V + c] - lse[r]) - (c == t[r] ? 1.0f : 0.0f)) * sc;
  }
}
