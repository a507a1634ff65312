/*
 * lthc_oracle.c — CPU restatement of the LTHC read / write / materialise
 * interface.  TEST INFRASTRUCTURE ONLY: called by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker
 * or the CPU baseline, never by the product path.
 *
 * Inputs and outputs are fp32; every sum is accumulated in fp64 and rounded
 * once.  Index map (local_thc_triton_kernels.py:355-363, local_thc.py:1220-1222):
 *   x[b, m, k, c] == X[b, (m / G) * S + k / S, (m % G) * S + k % S, c]
 * with X stored NHWC [B, G*S, G*S, C], cells m < G*G, taps k < S*S.
 * Weights are [C, S*S] row-major.  Pointer arrays hold L layer pointers.
 * OpenMP parallelises over cells (or channels for the reductions); results do
 * not depend on the thread count.
 */
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int64_t hi_off(int64_t b, int64_t m, int64_t k, int64_t G, int64_t S, int64_t C) {
  const int64_t H = G * S;
  const int64_t gy = m / G, gx = m % G, sy = k / S, sx = k % S;
  return ((b * H + gy * S + sy) * H + gx * S + sx) * C;
}

void oracle_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

int oracle_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* READ: z[b,m,c] = sum_k alpha[c,k] x[b,m,k,c]
 * Follows SharedLocalRead.read (local_thc.py:1211-1223) and the kernel
 * _write_fwd_kernel (local_thc_triton_kernels.py:27-60). */
void oracle_read(const float* x, const float* alpha, float* z, int64_t B, int64_t G, int64_t S, int64_t C) {
  const int64_t M = G * G, K = S * S;
#pragma omp parallel
  {
    double* acc = (double*)malloc(sizeof(double) * (size_t)C);
#pragma omp for schedule(static)
    for (int64_t bm = 0; bm < B * M; ++bm) {
      const int64_t b = bm / M, m = bm % M;
      for (int64_t c = 0; c < C; ++c) acc[c] = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const float* row = x + hi_off(b, m, k, G, S, C);
        for (int64_t c = 0; c < C; ++c) acc[c] += (double)alpha[c * K + k] * (double)row[c];
      }
      float* zr = z + bm * C;
      for (int64_t c = 0; c < C; ++c) zr[c] = (float)acc[c];
    }
    free(acc);
  }
}

/* WRITE / MATERIALISE: out[b,m,k,c] = base[b,m,k,c] + sum_l beta_l[c,k] dz_l[b,m,c]
 * base may be NULL.  Follows LayerLocalWrite.write/write_add
 * (local_thc.py:1261-1276), the final_accumulate_reference loop
 * (local_thc.py:1368-1372) and _final_accumulate_b4_12_fwd_kernel
 * (local_thc_triton_kernels.py:317-405). */
void oracle_write(const float* base, const float* const* dz, const float* const* beta, float* out, int64_t B,
                  int64_t G, int64_t S, int64_t C, int L) {
  const int64_t M = G * G, K = S * S;
#pragma omp parallel for schedule(static)
  for (int64_t bm = 0; bm < B * M; ++bm) {
    const int64_t b = bm / M, m = bm % M;
    for (int64_t k = 0; k < K; ++k) {
      const int64_t o = hi_off(b, m, k, G, S, C);
      for (int64_t c = 0; c < C; ++c) {
        double acc = base ? (double)base[o + c] : 0.0;
        for (int l = 0; l < L; ++l) acc += (double)beta[l][c * K + k] * (double)dz[l][bm * C + c];
        out[o + c] = (float)acc;
      }
    }
  }
}

/* MULTI-WEIGHT READ: out_l[b,m,c] = sum_k w_l[c,k] g[b,m,k,c]
 * The gradient of the materialisation with respect to dz_l
 * (_final_accumulate_b4_12_grad_dz_ptr_kernel, local_thc_triton_kernels.py:512-595). */
void oracle_read_multi(const float* g, const float* const* w, float* const* out, int64_t B, int64_t G, int64_t S,
                       int64_t C, int L) {
  for (int l = 0; l < L; ++l) oracle_read(g, w[l], out[l], B, G, S, C);
}

/* CELL WEIGHT GRADIENT: gw[l,c,k] = sum_{b,m} high[b,m,k,c] low_l[b,m,c]
 * (_cell_weight_grad_kernel :167-199, _final_accumulate_b4_12_grad_beta_ptr_kernel
 * :598-680).  Each thread owns a channel range; the sum runs over cells in
 * ascending order. */
void oracle_weight_grad(const float* high, const float* const* low, float* gw, int64_t B, int64_t G, int64_t S,
                        int64_t C, int L) {
  const int64_t M = G * G, K = S * S;
#pragma omp parallel
  {
    int nt = 1, tid = 0;
#ifdef _OPENMP
    nt = omp_get_num_threads();
    tid = omp_get_thread_num();
#endif
    const int64_t c_lo = C * tid / nt, c_hi = C * (tid + 1) / nt;
    const int64_t nc = c_hi - c_lo;
    if (nc > 0) {
      double* acc = (double*)calloc((size_t)(L * nc * K), sizeof(double));
      for (int64_t bm = 0; bm < B * M; ++bm) {
        const int64_t b = bm / M, m = bm % M;
        for (int64_t k = 0; k < K; ++k) {
          const float* row = high + hi_off(b, m, k, G, S, C);
          for (int l = 0; l < L; ++l) {
            const float* lo = low[l] + bm * C;
            double* a = acc + (int64_t)l * nc * K;
            for (int64_t c = c_lo; c < c_hi; ++c) a[(c - c_lo) * K + k] += (double)row[c] * (double)lo[c];
          }
        }
      }
      for (int l = 0; l < L; ++l)
        for (int64_t c = c_lo; c < c_hi; ++c)
          for (int64_t k = 0; k < K; ++k) gw[((int64_t)l * C + c) * K + k] = (float)acc[((int64_t)l * nc + (c - c_lo)) * K + k];
      free(acc);
    }
  }
}

/* GAMMA: gamma[l,c] = sum_k alpha[c,k] beta_l[c,k]  (local_thc.py:1278-1283) */
void oracle_gamma(const float* alpha, const float* const* beta, float* gamma, int64_t C, int64_t K, int L) {
  for (int l = 0; l < L; ++l)
    for (int64_t c = 0; c < C; ++c) {
      double s = 0.0;
      for (int64_t k = 0; k < K; ++k) s += (double)alpha[c * K + k] * (double)beta[l][c * K + k];
      gamma[(int64_t)l * C + c] = (float)s;
    }
}

/* RECURRENCE: z_next = z + gamma * dz  (lazy_workspace_update, local_thc.py:1325-1328) */
void oracle_recur(const float* z, const float* dz, const float* gamma, float* zn, int64_t rows, int64_t C) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < C; ++c)
      zn[r * C + c] = (float)((double)z[r * C + c] + (double)gamma[c] * (double)dz[r * C + c]);
}

/* RECURRENCE BACKWARD: gdz = gamma * g ; ggamma[c] = sum_r g[r,c] dz[r,c] */
void oracle_recur_bwd(const float* g, const float* dz, const float* gamma, float* gdz, float* ggamma, int64_t rows,
                      int64_t C) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < C; ++c) gdz[r * C + c] = (float)((double)gamma[c] * (double)g[r * C + c]);
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < C; ++c) {
    double s = 0.0;
    for (int64_t r = 0; r < rows; ++r) s += (double)g[r * C + c] * (double)dz[r * C + c];
    ggamma[c] = (float)s;
  }
}
