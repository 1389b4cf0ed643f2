// Split-K partial sums of the NF4 (+ LoRA) linear, and the reference
// epilogue that every consumer applies to them
// (src/triton_kernels/lora_forward.py:243-257):
//   acc = sum_s part[s][m][n]                  (slice order: deterministic)
//   v   = bf16(acc); v = bf16(v + bias[n])     (bias optional)
//   t   = bf16(sum_s tpart[s][seg][m][:])      (LoRA, r <= 16)
//   u   = bf16(bf16(t . B[n, :]) * bf16(scaling)); v = bf16(v + u)
#pragma once

#include "common.hpp"

namespace grpo {

constexpr int MAXSEG = GRPO_MAX_SEGMENTS;

// Device copy of grpo_linear_parts_t (passed to kernels by value).
struct LinParts {
  const float* part;   // [S][M][N]
  const float* tpart;  // [S][nseg][M][16]
  int S, M, N, K, nseg, r;
  int seg_end[MAXSEG];
  const uint16_t* bias[MAXSEG];
  const uint16_t* lb[MAXSEG];
  float scaling;
  bool lb_vec;    // r == 16 and every lora_b 16-byte aligned: rows read as 2 x 16 bytes
  bool bias_vec;  // every bias 8-byte aligned: 4 columns read as 8 bytes
};

// Host: validates a descriptor and converts it.  Returns GRPO_OK or einval.
int make_parts(const grpo_linear_parts_t* h, LinParts* d);

__device__ __forceinline__ int lin_seg(const LinParts& o, int n) {
  int s = 0;
  while (s + 1 < o.nseg && n >= o.seg_end[s]) ++s;
  return s;
}

// Sum over the S slices of float4 partials at p (slice stride `stride` float4s),
// in slice order.  Loads are issued 8 slices at a time so that they are in
// flight together (the kernels consuming partials are latency-bound).
__device__ __forceinline__ float4 slice_sum4(const float4* p, int S, int64_t stride) {
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int k0 = 0; k0 < S; k0 += 8) {
    float4 v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (k0 + j < S) v[j] = p[(k0 + j) * stride];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (k0 + j < S) {
        acc.x += v[j].x;
        acc.y += v[j].y;
        acc.z += v[j].z;
        acc.w += v[j].w;
      }
  }
  return acc;
}

// LoRA t of row m rounded to bf16, ts[seg*16 + j], computed by the whole
// workgroup (the caller synchronises before reading ts).
__device__ __forceinline__ void lin_load_t(const LinParts& o, int m, float* ts) {
  if (o.r <= 0) return;
  for (int i = threadIdx.x; i < o.nseg * 4; i += blockDim.x) {
    const int seg = i >> 2, q = i & 3;
    const float4* p = reinterpret_cast<const float4*>(o.tpart + ((int64_t)seg * o.M + m) * 16) + q;
    const float4 s = slice_sum4(p, o.S, (int64_t)o.nseg * o.M * 4);
    float* t = ts + seg * 16 + 4 * q;
    t[0] = round_bf(s.x);
    t[1] = round_bf(s.y);
    t[2] = round_bf(s.z);
    t[3] = round_bf(s.w);
  }
}

// Outputs (m, n..n+3) of the linear as the reference's bf16 values (as floats);
// n % 4 == 0, so the four columns lie in one segment.
__device__ __forceinline__ void lin_values4(const LinParts& o, const float* ts, int m, int n,
                                            float v[4]) {
  const float4 acc = slice_sum4(
      reinterpret_cast<const float4*>(o.part + (int64_t)m * o.N + n), o.S, (int64_t)o.M * o.N / 4);
  v[0] = round_bf(acc.x);
  v[1] = round_bf(acc.y);
  v[2] = round_bf(acc.z);
  v[3] = round_bf(acc.w);
  const int seg = lin_seg(o, n);
  const int nl = n - (seg > 0 ? o.seg_end[seg - 1] : 0);
  if (o.bias[seg]) {
    float b[4];
    if (o.bias_vec) {
      const uint2 bb = *reinterpret_cast<const uint2*>(o.bias[seg] + nl);
      b[0] = bf_lo(bb.x);
      b[1] = bf_hi(bb.x);
      b[2] = bf_lo(bb.y);
      b[3] = bf_hi(bb.y);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) b[c] = bf2f(o.bias[seg][nl + c]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = round_bf(v[c] + b[c]);
  }
  if (o.r > 0) {
    const float* t = ts + seg * 16;
    const float sc = round_bf(o.scaling);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint16_t* br = o.lb[seg] + (int64_t)(nl + c) * o.r;
      float u = 0.f;
      if (o.lb_vec) {
        const uint4 b0 = reinterpret_cast<const uint4*>(br)[0];
        const uint4 b1 = reinterpret_cast<const uint4*>(br)[1];
        const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          u += t[2 * j] * bf_lo(bw[j]);
          u += t[2 * j + 1] * bf_hi(bw[j]);
        }
      } else {
        for (int j = 0; j < o.r; ++j) u += t[j] * bf2f(br[j]);
      }
      u = round_bf(round_bf(u) * sc);
      v[c] = round_bf(v[c] + u);
    }
  }
}

}  // namespace grpo
