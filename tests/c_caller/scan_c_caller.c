/*
 * A plain C caller of the scan's C ABI (include/mvm_scan.h): device buffers
 * from hipMalloc, a non-default HIP stream, validation, checkpoint and
 * workspace sizing, forward with checkpoints, then the VJP from them.
 *
 *   scan_c_caller OUT.bin
 *
 * Shape B=2, L=100, D=96, N=16, fp32, automatic chunking (4 chunks of 32
 * positions; 96 channels are one full and one partial 64-channel block).
 * Inputs are deterministic functions of the element index.  OUT.bin holds
 * int64 B, L, D, N, then float32 u, delta, A, B, C, D, dy (the inputs as
 * passed) and y, du, ddelta, dA, dB, dC, dD (the outputs), each row-major:
 * (B,L,D), (B,L,D), (D,N), (B,L,N), (B,L,N), (D), (B,L,D) and the outputs
 * shaped like their primals.  The Python test compares the outputs with the
 * float64 oracle on those inputs.  Exit status 0 on success; a library or
 * HIP error prints its message and exits 1.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <hip/hip_runtime_api.h>

#include "mvm_scan.h"

enum { NB = 2, NL = 100, ND = 96, NN = 16 };

static int hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fprintf(stderr, "scan_c_caller: %s: %s\n", what, hipGetErrorString(e));
    return 0;
  }
  return 1;
}

static int mvm_ok(int rc, const char* what) {
  if (rc != MVM_OK) {
    fprintf(stderr, "scan_c_caller: %s: %d %s\n", what, rc, mvm_last_error());
    return 0;
  }
  return 1;
}

/* one host array and its device copy */
typedef struct {
  float* h;
  void* d;
  size_t n;
} buf_t;

static int buf_new(buf_t* b, size_t n) {
  b->n = n;
  b->h = (float*)calloc(n ? n : 1, sizeof(float));
  b->d = NULL;
  if (b->h == NULL) return 0;
  return hip_ok(hipMalloc(&b->d, (n ? n : 1) * sizeof(float)), "hipMalloc");
}

static int upload(buf_t* b) {
  return hip_ok(hipMemcpy(b->d, b->h, b->n * sizeof(float), hipMemcpyHostToDevice), "upload");
}

static int download(buf_t* b) {
  return hip_ok(hipMemcpy(b->h, b->d, b->n * sizeof(float), hipMemcpyDeviceToHost), "download");
}

int main(int argc, char** argv) {
  if (argc != 2) {
    fprintf(stderr, "usage: scan_c_caller OUT.bin\n");
    return 2;
  }
  const size_t nx = (size_t)NB * NL * ND, nbc = (size_t)NB * NL * NN, na = (size_t)ND * NN;
  buf_t u, dl, A, Bm, Cm, Dv, dy, y, du, ddl, dA, dB, dC, dD;
  buf_t* ins[] = {&u, &dl, &A, &Bm, &Cm, &Dv, &dy};
  buf_t* outs[] = {&y, &du, &ddl, &dA, &dB, &dC, &dD};
  const size_t in_n[] = {nx, nx, na, nbc, nbc, ND, nx};
  const size_t out_n[] = {nx, nx, nx, na, nbc, nbc, ND};
  for (int i = 0; i < 7; ++i)
    if (!buf_new(ins[i], in_n[i]) || !buf_new(outs[i], out_n[i])) return 1;

  for (size_t i = 0; i < nx; ++i) {
    u.h[i] = (float)sin(0.37 * (double)i + 0.1);
    dl.h[i] = (float)(0.01 + 0.04 * (0.5 + 0.5 * sin(0.13 * (double)i)));
    dy.h[i] = (float)cos(0.31 * (double)i + 0.2);
  }
  for (size_t i = 0; i < na; ++i) {
    const size_t d = i / NN, n = i % NN;
    A.h[i] = (float)(-(double)(n + 1) * (1.0 + 0.1 * sin((double)d)));
  }
  for (size_t i = 0; i < nbc; ++i) {
    Bm.h[i] = (float)cos(0.23 * (double)i);
    Cm.h[i] = (float)sin(0.19 * (double)i + 0.5);
  }
  for (size_t d = 0; d < ND; ++d) Dv.h[d] = (float)(1.0 + 0.1 * cos((double)d));
  for (int i = 0; i < 7; ++i)
    if (!upload(ins[i])) return 1;

  mvm_scan_desc desc = {0};
  desc.batch = NB;
  desc.seqlen = NL;
  desc.dim = ND;
  desc.dstate = NN;
  desc.ndir = 1;
  desc.x_stride_b = (int64_t)NL * ND;
  desc.x_stride_k = 0;
  desc.x_stride_t = ND;
  desc.bc_stride_b = (int64_t)NL * NN;
  desc.bc_stride_k = 0;
  desc.bc_stride_t = NN;
  desc.seq_to_tok = NULL;
  desc.in_dtype = MVM_F32;
  desc.out_dtype = MVM_F32;
  desc.chunk_len = 0;
  if (mvm_abi_version() != MVM_ABI_VERSION) {
    fprintf(stderr, "scan_c_caller: ABI %d, header %d\n", mvm_abi_version(), MVM_ABI_VERSION);
    return 1;
  }
  if (!mvm_ok(mvm_scan_validate(&desc), "validate")) return 1;

  const int64_t ck_elems = mvm_scan_ckpt_elems(&desc);
  const int64_t ws_f = mvm_scan_workspace_bytes(&desc, 0);
  const int64_t ws_b = mvm_scan_workspace_bytes(&desc, 1);
  if (ck_elems < 0 || ws_f < 0 || ws_b < 0) {
    fprintf(stderr, "scan_c_caller: sizing failed: %s\n", mvm_last_error());
    return 1;
  }
  void *ckpt = NULL, *ws = NULL;
  const size_t ws_n = (size_t)(ws_f > ws_b ? ws_f : ws_b);
  if (!hip_ok(hipMalloc(&ckpt, (size_t)ck_elems * sizeof(float)), "hipMalloc ckpt")) return 1;
  if (!hip_ok(hipMalloc(&ws, ws_n ? ws_n : 1), "hipMalloc workspace")) return 1;
  hipStream_t stream;
  if (!hip_ok(hipStreamCreate(&stream), "hipStreamCreate")) return 1;

  if (!mvm_ok(mvm_scan_fwd(&desc, u.d, (const float*)dl.d, (const float*)A.d, Bm.d, Cm.d,
                           (const float*)Dv.d, y.d, (float*)ckpt, ws, (size_t)ws_f, stream),
              "mvm_scan_fwd"))
    return 1;
  if (!mvm_ok(mvm_scan_bwd(&desc, u.d, (const float*)dl.d, (const float*)A.d, Bm.d, Cm.d,
                           (const float*)Dv.d, (const float*)ckpt, dy.d, du.d, (float*)ddl.d,
                           (float*)dA.d, dB.d, dC.d, (float*)dD.d, ws, (size_t)ws_b, stream),
              "mvm_scan_bwd"))
    return 1;
  if (!hip_ok(hipStreamSynchronize(stream), "hipStreamSynchronize")) return 1;
  for (int i = 0; i < 7; ++i)
    if (!download(outs[i])) return 1;

  FILE* f = fopen(argv[1], "wb");
  if (f == NULL) {
    fprintf(stderr, "scan_c_caller: cannot write %s\n", argv[1]);
    return 1;
  }
  const int64_t dims[4] = {NB, NL, ND, NN};
  int okw = fwrite(dims, sizeof(dims), 1, f) == 1;
  for (int i = 0; i < 7; ++i) okw = okw && fwrite(ins[i]->h, sizeof(float), ins[i]->n, f) == ins[i]->n;
  for (int i = 0; i < 7; ++i) okw = okw && fwrite(outs[i]->h, sizeof(float), outs[i]->n, f) == outs[i]->n;
  okw = (fclose(f) == 0) && okw;
  if (!okw) {
    fprintf(stderr, "scan_c_caller: short write to %s\n", argv[1]);
    return 1;
  }

  hipStreamDestroy(stream);
  hipFree(ckpt);
  hipFree(ws);
  for (int i = 0; i < 7; ++i) {
    hipFree(ins[i]->d);
    hipFree(outs[i]->d);
    free(ins[i]->h);
    free(outs[i]->h);
  }
  printf("scan_c_caller: wrote %s\n", argv[1]);
  return 0;
}
