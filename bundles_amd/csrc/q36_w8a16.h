// The W8A16 GEMM shared by the lm_head (mode 0: per-row fp32 scales, argmax) and the DENSE8 linear
// (mode 1: per-(row, 128-group) fp16 scales, column segments); kernels in w8a16.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q36 {

struct W16Dev {
  int T, N, K;
  const uint16_t* x;      // bf16 [T, K]
  const int8_t* q;        // int8 [N, K], row-major or (tiled) in the tile order of q36_tile_w16
  int tiled;
  // mode 0
  const float* ws;        // fp32 [N]
  uint16_t* logits;       // bf16 [T, N] or null
  float* logits32;        // fp32 [T, N] (the bf16-rounded values) or null
  unsigned long long* keys;  // [T] argmax keys (zero on entry)
  // mode 1
  const uint16_t* s16;    // fp16 [K / 128][s_ld]
  int64_t s_ld;
  int nseg, nout;
  int c0[4], ld[4];
  uint16_t* ys[4];
};

// T <= 64, N % 32 == 0, K 2048 (mode 0) or 2048 / 4096 (mode 1), checked by the callers
int launch_w8a16(const W16Dev& d, int mode, hipStream_t st);

}  // namespace q36
