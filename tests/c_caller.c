/* A plain C99 caller of libfdattn: the header compiles as C, the library
 * links and answers without a GPU. Queries (ABI version, workspace size,
 * the planner's kernel choice), an argument error reported through
 * fd_last_error, and one real decode through the host-core entry point on
 * fp32 data, checked against a direct double-precision computation.
 * Exit status 0 = every check passed; otherwise the number of the check. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fdattn.h"

#ifndef EXPECTED_ABI
#error "compile with -DEXPECTED_ABI=<the library's ABI version>"
#endif

enum { N = 2, H = 4, KVH = 2, D = 16, BS = 4, C = 4, W = 3 };

static float q[N][H][D], kc[C][KVH][BS][D], vc[C][KVH][BS][D];
static float out[N][H][D], lse[H][N];

static float val(unsigned i) { /* a fixed pseudo-random value in [-1, 1) */
  i = i * 2654435761u + 12345u;
  i ^= i >> 13;
  i *= 2246822519u;
  i ^= i >> 16;
  return (float)(i & 0xffff) / 32768.0f - 1.0f;
}

int main(void) {
  if (fd_abi_version() != EXPECTED_ABI) return 1;

  size_t ws = 0;
  if (fd_paged_decode_workspace_size(128, 32, 8, 128, 16, 256, &ws) != FD_OK) return 2;

  FdDecodePlan plan;
  if (fd_decode_plan_info(128, 32, 8, 128, 16, 128, FD_BF16, 1, 0, &plan) != FD_OK) return 3;
  if (plan.kernel != FD_KERNEL_MM || plan.heads_per_task != 16 || plan.passes != 1) return 4;

  /* q == NULL: rejected on the host, with a message, nothing launched */
  int32_t bt[N][W] = {{2, 0, 3}, {0, 0, 0}};
  int32_t lens[N] = {9, 0};
  if (fd_paged_decode_partial(NULL, H * D, D, kc, vc, KVH * BS * D, BS * D, D, C, &bt[0][0], W,
                              W, lens, NULL, N, H, KVH, D, BS, 0.25f, FD_F32, out, H * D, D,
                              FD_F32, &lse[0][0], N, NULL, 0, NULL) != FD_ERR_INVALID)
    return 5;
  if (strlen(fd_last_error()) == 0) return 6;

  /* one decode on the host cores: row 0 over blocks 2, 0, 3 (9 tokens), row 1 empty */
  unsigned s = 0;
  for (int i = 0; i < N; ++i)
    for (int h = 0; h < H; ++h)
      for (int d = 0; d < D; ++d) q[i][h][d] = val(s++);
  for (int b = 0; b < C; ++b)
    for (int kh = 0; kh < KVH; ++kh)
      for (int t = 0; t < BS; ++t)
        for (int d = 0; d < D; ++d) {
          kc[b][kh][t][d] = val(s++);
          vc[b][kh][t][d] = val(s++);
        }
  const float scale = 0.25f;
  if (fd_host_decode_partial(q, H * D, D, kc, vc, KVH * BS * D, BS * D, D, C, &bt[0][0], W, W,
                             lens, N, H, KVH, D, BS, scale, FD_F32, out, H * D, D, FD_F32,
                             &lse[0][0], N, 2) != FD_OK)
    return 7;
  for (int h = 0; h < H; ++h) {
    const int kh = h / (H / KVH);
    double sc[9], m = -INFINITY, l = 0.0, o[D];
    for (int t = 0; t < lens[0]; ++t) {
      const float* k = kc[bt[0][t / BS]][kh][t % BS];
      double dot = 0.0;
      for (int d = 0; d < D; ++d) dot += (double)q[0][h][d] * k[d];
      sc[t] = dot * scale;
      if (sc[t] > m) m = sc[t];
    }
    for (int d = 0; d < D; ++d) o[d] = 0.0;
    for (int t = 0; t < lens[0]; ++t) {
      const double p = exp(sc[t] - m);
      const float* v = vc[bt[0][t / BS]][kh][t % BS];
      l += p;
      for (int d = 0; d < D; ++d) o[d] += p * v[d];
    }
    for (int d = 0; d < D; ++d)
      if (fabs(out[0][h][d] - o[d] / l) > 1e-5) return 8;
    if (fabs(lse[h][0] - (m + log(l))) > 1e-5 * fmax(1.0, fabs(m + log(l)))) return 9;
    for (int d = 0; d < D; ++d)
      if (out[1][h][d] != 0.0f) return 10;
    if (!(isinf(lse[h][1]) && lse[h][1] < 0)) return 11;
  }
  printf("c caller ok (workspace for the query: %zu bytes)\n", ws);
  return 0;
}
