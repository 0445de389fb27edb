/* A plain C99 caller of libfdattn: the header compiles as C, the library
 * links and answers without a GPU. Queries (ABI version, workspace size,
 * the planner's kernel choice), an argument error reported through
 * fd_last_error, and one real decode through the host-core entry point on
 * fp32 data, checked against a direct double-precision computation. Built
 * with -DWITH_GPU (and the HIP runtime API, which is C), it also runs the
 * GPU entry point on device copies of a larger fp32 case (16-token blocks:
 * the tiled fp32 kernel), with and without the rows' token total, and checks
 * it the same way, and a whole hybrid split step (host cores and GPU on the
 * host tier, merged on the GPU).
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

/* The hybrid split step from C: an HBM tier in device memory and a host tier
 * in pinned memory (fd_host_alloc); the host cores' share queued behind the
 * copy of q to the host (fd_host_decode_partial_start), the GPU's fused launch
 * over the HBM tier and the leading host blocks (fd_split_decode), then
 * fd_host_decode_wait and the merge reading the host partial in place. Rows
 * of 50 (32 in HBM + 18 on the host), 0 and 56 (16 + 40) tokens, half of each
 * row's host blocks to the host cores; checked against double-precision
 * attention over each row's blocks of both tiers. */
enum { HG = 6, HC = 8 }; /* HBM blocks, host blocks */
static float hk_all[HG + HC][GKVH][GBS][GD], hv_all[HG + HC][GKVH][GBS][GD];
static float hq[GN][GH][GD], hout[GN][GH][GD], hlse[GH][GN];

/* one_call: steps 1-2 below as the single fd_hybrid_share_start call */
static int hybrid_case(int one_call) {
  int32_t hbm_bt[GN][GW] = {{4, 1, 0, 0}, {0, 0, 0, 0}, {5, 0, 0, 0}};
  int32_t host_bt[GN][GW] = {{6, 2, 0, 0}, {0, 0, 0, 0}, {0, 7, 3, 0}};
  int32_t hbm_lens[GN] = {32, 0, 16}, host_lens[GN] = {18, 0, 40};
  unsigned s = 4242;
  for (int i = 0; i < GN; ++i)
    for (int h = 0; h < GH; ++h)
      for (int d = 0; d < GD; ++d) hq[i][h][d] = val(s++);
  for (int b = 0; b < HG + HC; ++b)
    for (int kh = 0; kh < GKVH; ++kh)
      for (int t = 0; t < GBS; ++t)
        for (int d = 0; d < GD; ++d) {
          hk_all[b][kh][t][d] = val(s++);
          hv_all[b][kh][t][d] = val(s++);
        }
  const size_t blk = sizeof hk_all[0];
  const int64_t sb = GKVH * GBS * GD, sh = GBS * GD, st = GD;
  /* pinned host tier, q staging and host partial */
  void *hk, *hv, *q_host, *o_host, *l_host, *hk_d, *hv_d, *o_host_d, *l_host_d;
  if (fd_host_alloc(HC * blk, &hk) || fd_host_alloc(HC * blk, &hv) ||
      fd_host_alloc(sizeof hq, &q_host) || fd_host_alloc(sizeof hout, &o_host) ||
      fd_host_alloc(sizeof hlse, &l_host))
    return 20;
  if (fd_host_device_pointer(hk, &hk_d) || fd_host_device_pointer(hv, &hv_d) ||
      fd_host_device_pointer(o_host, &o_host_d) || fd_host_device_pointer(l_host, &l_host_d))
    return 21;
  memcpy(hk, hk_all[HG], HC * blk);
  memcpy(hv, hv_all[HG], HC * blk);
  /* device side: q, the HBM tier, the tables, the GPU partial and the output */
  void *dq, *dk, *dv, *dhbt, *dhl, *dhost_bt, *dgl, *dog, *dlg, *dout, *dlse, *dws = NULL;
  size_t ws = 0;
  if (fd_paged_decode_workspace_size(GN, GH, GKVH, GD, GBS, 2 * GW, &ws) != FD_OK) return 22;
  if (hipMalloc(&dq, sizeof hq) || hipMalloc(&dk, HG * blk) || hipMalloc(&dv, HG * blk) ||
      hipMalloc(&dhbt, sizeof hbm_bt) || hipMalloc(&dhl, sizeof hbm_lens) ||
      hipMalloc(&dhost_bt, sizeof host_bt) || hipMalloc(&dgl, sizeof host_lens) ||
      hipMalloc(&dog, sizeof hout) || hipMalloc(&dlg, sizeof hlse) ||
      hipMalloc(&dout, sizeof hout) || hipMalloc(&dlse, sizeof hlse) ||
      (ws > 0 && hipMalloc(&dws, ws)))
    return 23;
  if (hipMemcpy(dq, hq, sizeof hq, hipMemcpyHostToDevice) ||
      hipMemcpy(dk, hk_all, HG * blk, hipMemcpyHostToDevice) ||
      hipMemcpy(dv, hv_all, HG * blk, hipMemcpyHostToDevice) ||
      hipMemcpy(dhbt, hbm_bt, sizeof hbm_bt, hipMemcpyHostToDevice) ||
      hipMemcpy(dhl, hbm_lens, sizeof hbm_lens, hipMemcpyHostToDevice) ||
      hipMemcpy(dhost_bt, host_bt, sizeof host_bt, hipMemcpyHostToDevice))
    return 24;
  /* 1. divide each row's host blocks: half to the host cores */
  int32_t gpu_lens[GN], cpu_lens[GN], cpu_bt[GN][GW], wc = 0;
  hipEvent_t q_ready;
  if (hipEventCreate(&q_ready)) return 26;
  const float scale = 0.125f;
  int64_t call = -1;
  if (one_call) {
    /* 1-2 in one call: q to the host, the division, the share queued */
    if (fd_hybrid_share_start(NULL, q_ready, dq, q_host, &host_bt[0][0], GW, GW, host_lens, 0.5,
                              gpu_lens, &cpu_bt[0][0], GW, cpu_lens, hk, hv, sb, sh, st, HC, GN,
                              GH, GKVH, GD, GBS, scale, FD_F32, (float*)o_host, (float*)l_host, 2,
                              &call) != FD_OK) {
      fprintf(stderr, "%s\n", fd_last_error());
      return 27;
    }
  } else {
    if (fd_share_host_blocks(&host_bt[0][0], GW, GW, host_lens, GN, GBS, 0.5, gpu_lens,
                             &cpu_bt[0][0], GW, cpu_lens, &wc) != FD_OK)
      return 25;
    /* 2. q to the host and the host cores' share queued behind it */
    if (hipMemcpyAsync(q_host, dq, sizeof hq, hipMemcpyDeviceToHost, NULL) ||
        hipEventRecord(q_ready, NULL))
      return 26;
    if (fd_host_decode_partial_start(q_ready, q_host, GH * GD, GD, hk, hv, sb, sh, st, HC,
                                     &cpu_bt[0][0], GW, GW, cpu_lens, GN, GH, GKVH, GD, GBS,
                                     scale, FD_F32, o_host, GH * GD, GD, FD_F32, (float*)l_host,
                                     GN, 2, &call) != FD_OK) {
      fprintf(stderr, "%s\n", fd_last_error());
      return 27;
    }
  }
  if (hipMemcpy(dgl, gpu_lens, sizeof gpu_lens, hipMemcpyHostToDevice)) return 24;
  /* 3. the GPU's share: the HBM tier and the leading host blocks, zero-copy */
  fd_kv_tier hbm = {dk, dv, sb, sh, st, HG, (const int32_t*)dhbt, GW, GW, (const int32_t*)dhl};
  fd_kv_tier host = {hk_d, hv_d, sb, sh, st, HC, (const int32_t*)dhost_bt, GW, GW,
                     (const int32_t*)dgl};
  if (fd_split_decode(dq, GH * GD, GD, &hbm, &host, NULL, GN, GH, GKVH, GD, GBS, scale, FD_F32,
                      dog, GH * GD, GD, FD_F32, (float*)dlg, GN, dws, ws, NULL) != FD_OK) {
    fprintf(stderr, "%s\n", fd_last_error());
    fd_host_decode_wait(call, NULL);
    return 28;
  }
  /* 4. wait for the host cores, then merge reading their partial in place */
  double secs = -1.0;
  if (fd_host_decode_wait(call, &secs) != FD_OK || secs < 0.0) return 29;
  if (fd_merge_attn_states(dout, GH * GD, GD, FD_F32, dog, GH * GD, GD, FD_F32, (const float*)dlg,
                           GN, o_host_d, GH * GD, GD, FD_F32, (const float*)l_host_d, GN,
                           (float*)dlse, GN, GN, GH, GD, NULL) != FD_OK) {
    fprintf(stderr, "%s\n", fd_last_error());
    return 30;
  }
  if (hipDeviceSynchronize() || hipMemcpy(hout, dout, sizeof hout, hipMemcpyDeviceToHost) ||
      hipMemcpy(hlse, dlse, sizeof hlse, hipMemcpyDeviceToHost))
    return 31;
  /* each row's blocks of both tiers as one table over hk_all / hv_all */
  for (int i = 0; i < GN; ++i) {
    int32_t both[2 * GW];
    const int nh = (hbm_lens[i] + GBS - 1) / GBS, nc = (host_lens[i] + GBS - 1) / GBS;
    for (int b = 0; b < nh; ++b) both[b] = hbm_bt[i][b];
    for (int b = 0; b < nc; ++b) both[nh + b] = HG + host_bt[i][b];
    const int32_t len = hbm_lens[i] + host_lens[i];
    for (int h = 0; h < GH; ++h) {
      if (len == 0) {
        for (int d = 0; d < GD; ++d)
          if (hout[i][h][d] != 0.0f) return 32;
        if (!(isinf(hlse[h][i]) && hlse[h][i] < 0)) return 33;
      } else if (check_row(hq[i][h], &hk_all[0][0][0][0], &hv_all[0][0][0][0], both, len,
                           h / (GH / GKVH), GKVH, GBS, GD, scale, hout[i][h], hlse[h][i])) {
        return 34;
      }
    }
  }
  hipEventDestroy(q_ready);
  hipFree(dq); hipFree(dk); hipFree(dv); hipFree(dhbt); hipFree(dhl); hipFree(dhost_bt);
  hipFree(dgl); hipFree(dog); hipFree(dlg); hipFree(dout); hipFree(dlse);
  if (dws) hipFree(dws);
  if (fd_host_free(hk) || fd_host_free(hv) || fd_host_free(q_host) || fd_host_free(o_host) ||
      fd_host_free(l_host))
    return 35;
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
  const int hyb = hybrid_case(0);
  if (hyb) return hyb;
  static float first_out[GN][GH][GD], first_lse[GH][GN];
  memcpy(first_out, hout, sizeof hout);
  memcpy(first_lse, hlse, sizeof hlse);
  const int hyb1 = hybrid_case(1);
  if (hyb1) return hyb1;
  /* the one-call start divides and computes exactly as the separate calls */
  if (memcmp(first_out, hout, sizeof hout) || memcmp(first_lse, hlse, sizeof hlse)) return 36;
#endif
  printf("c caller ok (workspace for the query: %zu bytes)\n", ws);
  return 0;
}
