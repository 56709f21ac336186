/* fp32 GEMM on the CPU, restated from internal/sgemm/sgemm.go (GotoBLAS blocking: B packed in
 * panels of NR columns, A in panels of MR rows, an MR x NR register kernel over KC).
 * Test infrastructure only (see oracle.h). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* sgemm.go:17-23; mr is 6 on amd64 without AVX-512 (kernel_amd64.go) */
enum { MR = 6, NR = 16, KC = 256, MC = 96, NC = 2048 };

typedef struct {
  const float *data;
  int stride, trans;
} amat;

typedef struct {
  const float *data;
  int stride, n, trans; /* trans: given as its transpose (n x k), sgemm.go:60-84 */
} bmat;

/* sgemm.go:36-52 (Matrix.Pack) and :63-84 (Transposed.Pack): panel p at dst[p*kc*NR], row kk's
 * NR values at kk*NR, zeros past column n */
static void pack_b(const bmat *b, float *dst, int k0, int kc, int j0, int nc) {
  for (int p = 0; p * NR < nc; p++) {
    float *d = dst + (size_t)p * kc * NR;
    int c0 = j0 + p * NR;
    int w = b->n - c0 < NR ? b->n - c0 : NR;
    if (!b->trans) {
      for (int kk = 0; kk < kc; kk++) {
        const float *row = b->data + (size_t)(k0 + kk) * b->stride + c0;
        float *o = d + kk * NR;
        memcpy(o, row, sizeof(float) * w);
        memset(o + w, 0, sizeof(float) * (NR - w));
      }
    } else {
      for (int c = 0; c < w; c++) {
        const float *col = b->data + (size_t)(c0 + c) * b->stride + k0;
        for (int kk = 0; kk < kc; kk++) d[kk * NR + c] = col[kk];
      }
      if (w < NR)
        for (int kk = 0; kk < kc; kk++) memset(d + kk * NR + w, 0, sizeof(float) * (NR - w));
    }
  }
}

/* sgemm.go:99-123: panels of MR rows, column kk's MR values at kk*MR, zeros past row m */
static void pack_a(const amat *a, float *dst, int m, int i0, int mc, int k0, int kc) {
  for (int p = 0; p * MR < mc; p++) {
    float *d = dst + (size_t)p * kc * MR;
    int r0 = i0 + p * MR;
    int h = m - r0 < MR ? m - r0 : MR;
    if (!a->trans) {
      for (int r = 0; r < h; r++) {
        const float *row = a->data + (size_t)(r0 + r) * a->stride + k0;
        for (int kk = 0; kk < kc; kk++) d[kk * MR + r] = row[kk];
      }
    } else {
      for (int kk = 0; kk < kc; kk++) memcpy(d + kk * MR, a->data + (size_t)(k0 + kk) * a->stride + r0, sizeof(float) * h);
    }
    if (h < MR)
      for (int kk = 0; kk < kc; kk++) memset(d + kk * MR + h, 0, sizeof(float) * (MR - h));
  }
}

/* sgemm.go:214-230 (kernelGo; the AVX2 kernel fuses the multiply-add): c += a (kc x MR) b (kc x NR) */
static void kernel(int kc, const float *restrict a, const float *restrict b, float *restrict c, int ldc) {
  float acc[MR][NR];
  memset(acc, 0, sizeof(acc));
  for (int kk = 0; kk < kc; kk++) {
    const float *bp = b + kk * NR;
    const float *ap = a + kk * MR;
    for (int r = 0; r < MR; r++) {
      float av = ap[r];
      for (int j = 0; j < NR; j++) acc[r][j] = fmaf(av, bp[j], acc[r][j]);
    }
  }
  for (int r = 0; r < MR; r++)
    for (int j = 0; j < NR; j++) c[(size_t)r * ldc + j] += acc[r][j];
}

/* sgemm.go:172-211 */
static void block(int m, int k, const amat *a, const bmat *b, float *c, int ldc, int i0, int i1,
                  int j0, int j1) {
  float *bufa = malloc(sizeof(float) * (MC + MR) * KC);
  float *bufb = malloc(sizeof(float) * NC * KC);
  float edge[MR * NR];
  for (int jc = j0; jc < j1; jc += NC) {
    int nc = j1 - jc < NC ? j1 - jc : NC;
    for (int pc = 0; pc < k; pc += KC) {
      int kc = k - pc < KC ? k - pc : KC;
      pack_b(b, bufb, pc, kc, jc, nc);
      for (int ic = i0; ic < i1; ic += MC) {
        int mc = i1 - ic < MC ? i1 - ic : MC;
        pack_a(a, bufa, m, ic, mc, pc, kc);
        for (int jr = 0; jr < nc; jr += NR) {
          const float *bp = bufb + (size_t)(jr / NR) * kc * NR;
          int w = nc - jr < NR ? nc - jr : NR;
          for (int ir = 0; ir < mc; ir += MR) {
            const float *ap = bufa + (size_t)(ir / MR) * kc * MR;
            int h = mc - ir < MR ? mc - ir : MR;
            float *cp = c + (size_t)(ic + ir) * ldc + jc + jr;
            if (h == MR && w == NR) {
              kernel(kc, ap, bp, cp, ldc);
              continue;
            }
            memset(edge, 0, sizeof(edge));
            kernel(kc, ap, bp, edge, NR);
            for (int r = 0; r < h; r++)
              for (int j = 0; j < w; j++) cp[(size_t)r * ldc + j] += edge[r * NR + j];
          }
        }
      }
    }
  }
  free(bufa);
  free(bufb);
}

/* sgemm.go:127-163 (MulAdd): whole column panels per thread, or rows when the columns are few */
void or_sgemm(int m, int n, int k, const float *a, int lda, int transa, const float *b, int ldb,
              int transb, float *c, int ldc, int threads) {
  if (m == 0 || n == 0 || k == 0) return;
  if (threads <= 0) threads = or_max_threads();
  amat A = {a, lda, transa};
  bmat B = {b, ldb, n, transb};
  int panels = (n + NR - 1) / NR;
  if (threads > 1 && panels >= 2 * threads) {
    int per = (panels + threads - 1) / threads;
    int parts = (n + per * NR - 1) / (per * NR);
#pragma omp parallel for schedule(static, 1) num_threads(threads)
    for (int t = 0; t < parts; t++) {
      int j0 = t * per * NR, j1 = j0 + per * NR < n ? j0 + per * NR : n;
      block(m, k, &A, &B, c, ldc, 0, m, j0, j1);
    }
    return;
  }
  if (threads > 1 && m >= 2 * MR * threads) {
    int per = ((m + threads - 1) / threads + MR - 1) / MR * MR;
    int parts = (m + per - 1) / per;
#pragma omp parallel for schedule(static, 1) num_threads(threads)
    for (int t = 0; t < parts; t++) {
      int i0 = t * per, i1 = i0 + per < m ? i0 + per : m;
      block(m, k, &A, &B, c, ldc, i0, i1, 0, n);
    }
    return;
  }
  block(m, k, &A, &B, c, ldc, 0, m, 0, n);
}
