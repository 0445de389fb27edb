/* A plain C99 caller of libfdattn: the header compiles as C, the library
 * links and answers without a GPU. Queries (ABI version, workspace size,
 * the planner's kernel choice), an argument error reported through
 * fd_last_error, and one real decode through the host-core entry point on
 * fp32 data, checked against a direct double-precision computation. Built
 * with -DWITH_GPU (and the HIP runtime API, which is C), it also runs the
 * GPU entry point on device copies of a larger fp32 case (16-token blocks:
 * the tiled fp32 kernel), with and without the rows' token total, and checks
 * it the same way.
 * Exit status 0 = every check passed; otherwise the number of the check. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "fdattn.h"
#ifdef WITH_GPU
#include <hip/hip_runtime_api.h>
#endif

#ifndef EXPECTED_ABI
#error "compile with -DEXPECTED_ABI=<the library's ABI version>"
#endif

enum { N = 2, H = 4, KVH = 2, D = 16, BS = 4, C = 4, W = 3 };

static float q[N][H][D], kc[C][KVH][BS][D], vc[C][KVH][BS][D];
static float out[N][H][D], lse[H][N];

/* Double-precision attention of row i, head h over its table; 0 = matches
 * out / lse within 1e-5 (out absolute, lse relative to max(1, |lse|)). */
static int check_row(const float* qr, const float* k, const float* v, const int32_t* row_bt,
                     int32_t len, int kvh, int KVH_, int BS_, int D_, float scale,
                     const float* out_r, float lse_r) {
  double m = -INFINITY, l = 0.0, o[256], sc[4096];
  if (len > 4096 || D_ > 256) return 1;
  for (int t = 0; t < len; ++t) {
    const float* kt = k + (((int64_t)row_bt[t / BS_] * KVH_ + kvh) * BS_ + t % BS_) * D_;
    double dot = 0.0;
    for (int d = 0; d < D_; ++d) dot += (double)qr[d] * kt[d];
    sc[t] = dot * scale;
    if (sc[t] > m) m = sc[t];
  }
  for (int d = 0; d < D_; ++d) o[d] = 0.0;
  for (int t = 0; t < len; ++t) {
    const double p = exp(sc[t] - m);
    const float* vt = v + (((int64_t)row_bt[t / BS_] * KVH_ + kvh) * BS_ + t % BS_) * D_;
    l += p;
    for (int d = 0; d < D_; ++d) o[d] += p * vt[d];
  }
  for (int d = 0; d < D_; ++d)
    if (fabs(out_r[d] - o[d] / l) > 1e-5) return 1;
  return fabs(lse_r - (m + log(l))) > 1e-5 * fmax(1.0, fabs(m + log(l)));
}

static float val(unsigned i) { /* a fixed pseudo-random value in [-1, 1) */
  i = i * 2654435761u + 12345u;
  i ^= i >> 13;
  i *= 2246822519u;
  i ^= i >> 16;
  return (float)(i & 0xffff) / 32768.0f - 1.0f;
}

#ifdef WITH_GPU
enum { GN = 3, GH = 8, GKVH = 2, GD = 64, GBS = 16, GC = 10, GW = 4 };
static float gq[GN][GH][GD], gk[GC][GKVH][GBS][GD], gv[GC][GKVH][GBS][GD];
static float gout[GN][GH][GD], glse[GH][GN];

/* The GPU entry point on device copies: rows of 50, 0 and 64 tokens. */
static int gpu_case(void) {
  int32_t bt[GN][GW] = {{7, 2, 9, 0}, {0, 0, 0, 0}, {1, 4, 3, 8}};
  int32_t lens[GN] = {50, 0, 64};
  unsigned s = 777;
  for (int i = 0; i < GN; ++i)
    for (int h = 0; h < GH; ++h)
      for (int d = 0; d < GD; ++d) gq[i][h][d] = val(s++);
  for (int b = 0; b < GC; ++b)
    for (int kh = 0; kh < GKVH; ++kh)
      for (int t = 0; t < GBS; ++t)
        for (int d = 0; d < GD; ++d) {
          gk[b][kh][t][d] = val(s++);
          gv[b][kh][t][d] = val(s++);
        }
  void *dq, *dk, *dv, *dbt, *dlens, *dout, *dlse, *dws = NULL;
  size_t ws = 0;
  if (fd_paged_decode_workspace_size(GN, GH, GKVH, GD, GBS, GW, &ws) != FD_OK) return 1;
  if (hipMalloc(&dq, sizeof gq) || hipMalloc(&dk, sizeof gk) || hipMalloc(&dv, sizeof gv) ||
      hipMalloc(&dbt, sizeof bt) || hipMalloc(&dlens, sizeof lens) ||
      hipMalloc(&dout, sizeof gout) || hipMalloc(&dlse, sizeof glse) ||
      (ws > 0 && hipMalloc(&dws, ws)))
    return 2;
  if (hipMemcpy(dq, gq, sizeof gq, hipMemcpyHostToDevice) ||
      hipMemcpy(dk, gk, sizeof gk, hipMemcpyHostToDevice) ||
      hipMemcpy(dv, gv, sizeof gv, hipMemcpyHostToDevice) ||
      hipMemcpy(dbt, bt, sizeof bt, hipMemcpyHostToDevice) ||
      hipMemcpy(dlens, lens, sizeof lens, hipMemcpyHostToDevice))
    return 3;
  const float scale = 0.125f;
  if (fd_paged_decode_partial(dq, GH * GD, GD, dk, dv, GKVH * GBS * GD, GBS * GD, GD, GC,
                              (const int32_t*)dbt, GW, GW, (const int32_t*)dlens, NULL, GN, GH,
                              GKVH, GD, GBS, scale, FD_F32, dout, GH * GD, GD, FD_F32,
                              (float*)dlse, GN, dws, ws, NULL) != FD_OK) {
    fprintf(stderr, "%s\n", fd_last_error());
    return 4;
  }
  if (hipDeviceSynchronize() || hipMemcpy(gout, dout, sizeof gout, hipMemcpyDeviceToHost) ||
      hipMemcpy(glse, dlse, sizeof glse, hipMemcpyDeviceToHost))
    return 5;
  for (int pass = 0; pass < 2; ++pass) {
    for (int i = 0; i < GN; ++i)
      for (int h = 0; h < GH; ++h) {
        if (lens[i] == 0) {
          for (int d = 0; d < GD; ++d)
            if (gout[i][h][d] != 0.0f) return 6;
          if (!(isinf(glse[h][i]) && glse[h][i] < 0)) return 7;
        } else if (check_row(gq[i][h], &gk[0][0][0][0], &gv[0][0][0][0], bt[i], lens[i],
                             h / (GH / GKVH), GKVH, GBS, GD, scale, gout[i][h], glse[h][i])) {
          return 8;
        }
      }
    if (pass == 1) break;
    /* again through the entry point that takes the rows' token total */
    memset(gout, 0, sizeof gout);
    if (hipMemcpy(dout, gout, sizeof gout, hipMemcpyHostToDevice)) return 3;
    if (fd_paged_decode_partial_hint(dq, GH * GD, GD, dk, dv, GKVH * GBS * GD, GBS * GD, GD, GC,
                                     (const int32_t*)dbt, GW, GW, (const int32_t*)dlens, NULL,
                                     GN, GH, GKVH, GD, GBS, scale, FD_F32, dout, GH * GD, GD,
                                     FD_F32, (float*)dlse, GN, dws, ws, NULL,
                                     (int64_t)lens[0] + lens[1] + lens[2]) != FD_OK) {
      fprintf(stderr, "%s\n", fd_last_error());
      return 9;
    }
    if (hipDeviceSynchronize() || hipMemcpy(gout, dout, sizeof gout, hipMemcpyDeviceToHost) ||
        hipMemcpy(glse, dlse, sizeof glse, hipMemcpyDeviceToHost))
      return 5;
  }
  hipFree(dq); hipFree(dk); hipFree(dv); hipFree(dbt); hipFree(dlens); hipFree(dout);
  hipFree(dlse);
  if (dws) hipFree(dws);
  return 0;
}
#endif

int main(void) {
  if (fd_abi_version() != EXPECTED_ABI) return 1;

  size_t ws = 0;
  if (fd_paged_decode_workspace_size(128, 32, 8, 128, 16, 256, &ws) != FD_OK) return 2;

  FdDecodePlan plan;
  if (fd_decode_plan_info(128, 32, 8, 128, 16, 128, FD_BF16, 1, 0, 0, &plan) != FD_OK) return 3;
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
    if (check_row(q[0][h], &kc[0][0][0][0], &vc[0][0][0][0], bt[0], lens[0], h / (H / KVH), KVH,
                  BS, D, scale, out[0][h], lse[h][0]))
      return 8;
    for (int d = 0; d < D; ++d)
      if (out[1][h][d] != 0.0f) return 10;
    if (!(isinf(lse[h][1]) && lse[h][1] < 0)) return 11;
  }
  /* the same call queued on the library's runner thread: the same bits */
  static float out2[N][H][D], lse2[H][N];
  int64_t call = -1;
  double secs = -1.0;
  if (fd_host_decode_partial_start(NULL, q, H * D, D, kc, vc, KVH * BS * D, BS * D, D, C,
                                   &bt[0][0], W, W, lens, N, H, KVH, D, BS, scale, FD_F32, out2,
                                   H * D, D, FD_F32, &lse2[0][0], N, 2, &call) != FD_OK)
    return 13;
  if (fd_host_decode_wait(call, &secs) != FD_OK || secs < 0.0) return 14;
  if (memcmp(out, out2, sizeof out2) != 0 || memcmp(lse, lse2, sizeof lse2) != 0) return 15;
  if (fd_host_decode_wait(call, NULL) != FD_ERR_INVALID) return 16;
#ifdef WITH_GPU
  if (gpu_case()) return 12;
#endif
  printf("c caller ok (workspace for the query: %zu bytes)\n", ws);
  return 0;
}
