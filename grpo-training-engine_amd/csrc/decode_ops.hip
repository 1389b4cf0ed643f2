// Per-step ops of the model-level decode around the two hot-path kernels
// (src/triton_kernels/paged_kv.py:690-820 and fused_ops.py:34-251):
// embedding gather, residual add + RMSNorm, RoPE fused with the KV append,
// SiLU*mul, and greedy argmax.  All bf16 in / bf16 out with the reference's
// rounding points; memory-bound, one workgroup per row.  The *_parts forms
// take the split-K partial sums of the NF4 linear that feeds them and first
// rebuild its bf16 output (reduction over K slices + LoRA epilogue,
// linear_parts.hpp), so that linear needs no epilogue launch of its own.
#include <math.h>

#include "linear_parts.hpp"

using namespace grpo;

namespace {

constexpr int ROW_T = 256;

constexpr int PARTS_T = 512;  // consumers of partial sums: more loads in flight per row

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// Sum over a wave: DPP within each row of 16 lanes (xor 1, xor 2, half-row
// mirror, row mirror), then the permlane swaps across rows; every lane gets
// the total.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return pair32_sum(pair16_sum(v));
}

// Sum over the workgroup, every thread gets the total.  Uses red[] once:
// call it once per kernel (there is no trailing barrier).
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += red[w];
  return t;
}

// out[b, :] = table[ids[b], :]; ids outside [0, V) give a zero row.
__global__ void __launch_bounds__(ROW_T) embedding_kernel(const int64_t* __restrict__ ids,
                                                          const uint16_t* __restrict__ table,
                                                          int64_t V, int H,
                                                          uint16_t* __restrict__ out) {
  const int b = blockIdx.x;
  const int64_t id = ids[b];
  const bool ok = id >= 0 && id < V;
  const uint16_t* src = table + (ok ? id : 0) * (int64_t)H;
  for (int i = threadIdx.x; i < H; i += ROW_T) out[(int64_t)b * H + i] = ok ? src[i] : 0;
}

// embedding_kernel that also writes the RMSNorm statistic of each row:
// sumsq[b, t] = sum of out[b, i]^2 over i = t, t + ROW_T, ... (ROW_T groups per
// row), which the first q|k|v kernel stages the input norm from.
__global__ void __launch_bounds__(ROW_T) embedding_sumsq_kernel(const int64_t* __restrict__ ids,
                                                                const uint16_t* __restrict__ table,
                                                                int64_t V, int H,
                                                                uint16_t* __restrict__ out,
                                                                float* __restrict__ sumsq) {
  const int b = blockIdx.x;
  const int64_t id = ids[b];
  const bool ok = id >= 0 && id < V;
  const uint16_t* src = table + (ok ? id : 0) * (int64_t)H;
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += ROW_T) {
    const uint16_t v = ok ? src[i] : 0;
    out[(int64_t)b * H + i] = v;
    ss += bf2f(v) * bf2f(v);
  }
  sumsq[(int64_t)b * ROW_T + threadIdx.x] = ss;
}

// h = residual ? bf16(x + residual) : x; y = bf16(bf16(h * rsqrt(mean(h^2) + eps)) * w)
// (fused_ops.py:34-77; transformers' Qwen2RMSNorm).  h is written to h_out when given.
__global__ void __launch_bounds__(ROW_T) add_rmsnorm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* residual, uint16_t* h_out,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ y, int H, float eps) {
  __shared__ float red[ROW_T / 64];
  extern __shared__ float hs[];  // H floats
  const int64_t row = (int64_t)blockIdx.x * H;
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += ROW_T) {
    float h = bf2f(x[row + i]);
    if (residual) h = round_bf(h + bf2f(residual[row + i]));
    hs[i] = h;
    ss += h * h;
  }
  const float total = block_sum(ss, red);
  const float inv = 1.f / sqrtf(total / (float)H + eps);
  for (int i = threadIdx.x; i < H; i += ROW_T) {
    const float h = hs[i];
    if (residual && h_out) h_out[row + i] = f2bf(h);
    y[row + i] = f2bf(round_bf(h * inv) * bf2f(w[i]));
  }
}

// RoPE (x*cos + rotate_half(x)*sin in bf16 arithmetic, transformers'
// apply_rotary_pos_emb) on q and k of one token per sequence, then the KV
// append of paged_kv.py:253-319 at slot context_lens[b].
//   qkv row: [q (Hq*D) | k (Hkv*D) | v (Hkv*D)], row stride ld
__global__ void __launch_bounds__(ROW_T) rope_append_kernel(
    const uint16_t* __restrict__ qkv, int64_t ld, int Hq, int Hkv, int D,
    const uint16_t* __restrict__ cos_t, const uint16_t* __restrict__ sin_t, int max_pos,
    const int32_t* __restrict__ context_lens, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t num_blocks,
    const int32_t* __restrict__ bt, int64_t bts, int BS, int max_blocks) {
  const int b = blockIdx.x;
  const int pos = context_lens[b];
  const int cpos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const uint16_t* row = qkv + (int64_t)b * ld;
  const uint16_t* cr = cos_t + (int64_t)cpos * D;
  const uint16_t* sr = sin_t + (int64_t)cpos * D;
  const int half = D / 2;
  bool slot_ok = pos >= 0 && pos < max_blocks * BS;
  int64_t slot_base = 0;
  if (slot_ok) {
    const int phys = bt[(int64_t)b * bts + pos / BS];
    slot_ok = phys >= 0 && phys < num_blocks;
    slot_base = ((int64_t)phys * Hkv * BS + (pos % BS)) * D;  // + h * BS * D + d
  }
  const int nrot = (Hq + Hkv) * D;
  for (int i = threadIdx.x; i < nrot + Hkv * D; i += ROW_T) {
    if (i < nrot) {
      const int h = i / D, d = i - h * D;
      const uint16_t* xh = row + (int64_t)h * D;  // q heads then k heads (contiguous)
      const float xv = bf2f(xh[d]);
      const float rv = d < half ? -bf2f(xh[d + half]) : bf2f(xh[d - half]);
      const float o = round_bf(round_bf(xv * bf2f(cr[d])) + round_bf(rv * bf2f(sr[d])));
      if (h < Hq) {
        q_out[((int64_t)b * Hq + h) * D + d] = f2bf(o);
      } else if (slot_ok) {
        kc[slot_base + (int64_t)(h - Hq) * BS * D + d] = f2bf(o);
      }
    } else if (slot_ok) {
      const int j = i - nrot, h = j / D, d = j - h * D;
      vc[slot_base + (int64_t)h * BS * D + d] = row[nrot + j];
    }
  }
}

// out = bf16(bf16(silu(gate)) * up), gate = row[0:N], up = row[N:2N] (fused_ops.py:79-112).
__global__ void __launch_bounds__(ROW_T) silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                         int64_t ld, int N,
                                                         uint16_t* __restrict__ out,
                                                         int64_t ldo) {
  const int64_t m = blockIdx.y;
  const int i = blockIdx.x * ROW_T + threadIdx.x;
  if (i >= N) return;
  const float g = bf2f(gu[m * ld + i]);
  const float u = bf2f(gu[m * ld + N + i]);
  const float s = round_bf(g * (1.f / (1.f + expf(-g))));
  out[m * ldo + i] = f2bf(s * u);
}

// Greedy argmax over a bf16 row (first index of the maximum, NaNs ignored).
constexpr int AMAX_T = 1024;
__global__ void __launch_bounds__(AMAX_T) argmax_kernel(const uint16_t* __restrict__ logits,
                                                        int64_t ld, int V,
                                                        int64_t* __restrict__ out) {
  __shared__ float sv[AMAX_T / 64];
  __shared__ int si[AMAX_T / 64];
  const uint16_t* row = logits + (int64_t)blockIdx.x * ld;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  // 16-byte loads of 8 logits, four in flight per thread before any compare
  // (one dependent 2-byte load per iteration left the row latency-bound); a
  // thread's indexes rise through its chunks, so strictly-greater keeps the
  // first index of a maximum.  Misaligned rows and the tail take 2-byte loads.
  const bool vec = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
  const int nv = vec ? V / 8 : 0;
  constexpr int AMAX_U = 4;
  for (int c0 = 0; c0 < nv; c0 += AMAX_U * AMAX_T) {
    uint4 w[AMAX_U];
#pragma unroll
    for (int u = 0; u < AMAX_U; ++u) {
      const int c = c0 + u * AMAX_T + threadIdx.x;
      w[u] = c < nv ? reinterpret_cast<const uint4*>(row)[c] : make_uint4(0xFF80FF80u, 0xFF80FF80u,
                                                                          0xFF80FF80u, 0xFF80FF80u);
    }
#pragma unroll
    for (int u = 0; u < AMAX_U; ++u) {
      const int c = c0 + u * AMAX_T + threadIdx.x;
      const uint32_t ww[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = (j & 1) ? bf_hi(ww[j >> 1]) : bf_lo(ww[j >> 1]);
        if (v > best) {
          best = v;
          bi = 8 * c + j;
        }
      }
    }
  }
  for (int i = 8 * nv + threadIdx.x; i < V; i += AMAX_T) {
    const float v = bf2f(row[i]);
    if (v > best) {  // strictly greater keeps the first index per thread
      best = v;
      bi = i;
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o);
    const int oi = __shfl_xor(bi, o);
    if (ov > best || (ov == best && oi < bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < AMAX_T / 64; ++w)
      if (sv[w] > best || (sv[w] == best && si[w] < bi)) {
        best = sv[w];
        bi = si[w];
      }
    out[blockIdx.x] = bi == 0x7fffffff ? 0 : bi;
  }
}

// add_rmsnorm_kernel with x = the finished linear output of row m (a thread
// finishes four columns at a time; the first four columns of every thread are
// fetched before the LoRA-t barrier, so most rows need one memory round trip).
// T threads per row, MS the most K slices it fetches (S <= MS): rows of up to
// 4 * T columns are finished from the loads issued before the LoRA-t barrier.
// LORA false: the host guarantees r == 0 (no registers for LoRA B rows).
template <int T, int MS, bool LORA>
__global__ void __launch_bounds__(T) add_rmsnorm_parts_kernel(
    LinParts op, const uint16_t* residual, uint16_t* h_out, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ y, float eps, bool vec) {
  constexpr int PARTS_T = T;
  LinParts o = op;
  if (!LORA) o.r = 0;
  touch_kernargs<sizeof(LinParts) + 4 * sizeof(void*) + 8>();
  __shared__ float red[PARTS_T / 64];
  __shared__ float ts[MAXSEG * 16];
  // Dynamic LDS: max(H, 4 * PARTS_T) floats with LoRA, else H (512 threads)
  // or none.  hs holds the columns past 4 * PARTS_T; lu, the LoRA sums of
  // each wave's 256 columns, the first 4 * PARTS_T floats (disjoint from
  // every hs entry used).
  extern __shared__ float hs[];
  float* lu = hs;
  const int m = blockIdx.x, H = o.N;
  const int64_t row = (int64_t)m * H;
  const int tid = threadIdx.x;
  // Rank-16 LoRA of one aligned segment: each wave reads the B rows of its
  // 256 columns in 1 KiB loads (lin_fetch_lb_wave) instead of 128 bytes per
  // lane.  o1 serves the first pass (other LoRA shapes read B per element
  // there), o the wide rows.
  const int c0 = 4 * (tid & ~63);
  const bool wave_lb = LORA && o.r == 16 && o.lb_vec && o.nseg == 1 && c0 < H;
  LinParts o1 = o;
  o1.lb_vec = false;
  // Thread tid owns columns 4*tid .. 4*tid+3 from the loads to the final
  // stores, so its h stays in registers; the norm weight is fetched with the
  // partial sums (a load after the row reduction would be one more memory
  // round trip at the end of the kernel).  Wider rows (> 4 * PARTS_T) put the
  // rest through LDS.
  const bool first = tid < H / 4;
  Fetch4<MS> f;
  uint2 res0 = make_uint2(0, 0), w0 = make_uint2(0, 0);
  uint4 lbw[8];
  if (wave_lb) lin_fetch_lb_wave(o, c0, lbw);
  if (first) {
    lin_fetch4(o1, m, 4 * tid, f);
    if (residual) res0 = *reinterpret_cast<const uint2*>(residual + row + 4 * tid);
    if (vec) {
      w0 = *reinterpret_cast<const uint2*>(w + 4 * tid);
    } else {
      w0.x = pack2(w[4 * tid], w[4 * tid + 1]);
      w0.y = pack2(w[4 * tid + 2], w[4 * tid + 3]);
    }
  }
  lin_load_t<MS>(o, m, ts);
  __syncthreads();
  float4 lora_u = make_float4(0.f, 0.f, 0.f, 0.f);
  if (wave_lb) lora_u = lin_lora_wave(ts, lbw, lu + c0);
  float ss = 0.f;
  float h0[4] = {0.f, 0.f, 0.f, 0.f};
  auto add_res = [&](const float (&v)[4], uint2 rr, float (&h)[4]) {
    const float rv[4] = {bf_lo(rr.x), bf_hi(rr.x), bf_lo(rr.y), bf_hi(rr.y)};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      h[c] = residual ? round_bf(v[c] + rv[c]) : v[c];
      ss += h[c] * h[c];
    }
  };
  if (first) {
    float v[4];
    lin_finish4(o1, ts, f, v, wave_lb, lora_u);
    add_res(v, res0, h0);
  }
  // rows wider than 4 * PARTS_T (the 1024-thread forms take at most 4096 columns)
  for (int i4 = tid + PARTS_T; T < 1024 && i4 < H / 4; i4 += PARTS_T) {
    float v[4], h[4];
    lin_values4(o, ts, m, 4 * i4, v);
    add_res(v, residual ? *reinterpret_cast<const uint2*>(residual + row + 4 * i4)
                        : make_uint2(0, 0), h);
#pragma unroll
    for (int c = 0; c < 4; ++c) hs[4 * i4 + c] = h[c];
  }
  const float total = block_sum(ss, red);
  const float inv = 1.f / sqrtf(total / (float)H + eps);
  if (first) {
    const float wv[4] = {bf_lo(w0.x), bf_hi(w0.x), bf_lo(w0.y), bf_hi(w0.y)};
    float yv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) yv[c] = round_bf(h0[c] * inv) * wv[c];
    const uint2 yo = make_uint2(pack_bf2(yv[0], yv[1]), pack_bf2(yv[2], yv[3]));
    const uint2 ho = make_uint2(pack_bf2(h0[0], h0[1]), pack_bf2(h0[2], h0[3]));
    if (vec) {
      *reinterpret_cast<uint2*>(y + row + 4 * tid) = yo;
      if (residual && h_out) *reinterpret_cast<uint2*>(h_out + row + 4 * tid) = ho;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        y[row + 4 * tid + c] = f2bf(yv[c]);
        if (residual && h_out) h_out[row + 4 * tid + c] = f2bf(h0[c]);
      }
    }
  }
  for (int i = 4 * PARTS_T + tid; T < 1024 && i < H; i += PARTS_T) {
    const float h = hs[i];
    if (residual && h_out) h_out[row + i] = f2bf(h);
    y[row + i] = f2bf(round_bf(h * inv) * bf2f(w[i]));
  }
}

// h = bf16(residual + y) for the finished linear output y (the epilogue of
// linear_parts.hpp) and, for the RMSNorm its consumer stages, sumsq[m, g] = sum
// of h^2 over the 64 columns of group g.  One wave per (256 columns, row), so a
// row's partial sums, LoRA B rows and residual are fetched by N / 256 CUs, not
// one: the per-row RMSNorm kernel above moved ~90 KB through a single CU per
// row for o_proj at hidden 1536.
constexpr int FRS_T = 64;
constexpr int FRS_COLS = 4 * FRS_T;
__global__ void __launch_bounds__(FRS_T) finish_residual_sumsq_kernel(
    LinParts o, const uint16_t* residual, uint16_t* h_out, int64_t ld, float* __restrict__ sumsq,
    int G) {
  touch_kernargs<sizeof(LinParts) + 5 * sizeof(void*)>();
  __shared__ float ts[MAXSEG * 16];
  const int g = blockIdx.x, m = blockIdx.y;
  const int n = g * FRS_COLS + 4 * threadIdx.x;
  const bool ok = n < o.N;
  Fetch4<> f;
  uint2 rr = make_uint2(0, 0);
  if (ok) {
    lin_fetch4(o, m, n, f);
    if (residual) rr = *reinterpret_cast<const uint2*>(residual + (int64_t)m * ld + n);
  }
  lin_load_t(o, m, ts);
  __syncthreads();
  float ss = 0.f;
  if (ok) {
    float v[4];
    lin_finish4(o, ts, f, v);
    const float r[4] = {bf_lo(rr.x), bf_hi(rr.x), bf_lo(rr.y), bf_hi(rr.y)};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (residual) v[c] = round_bf(v[c] + r[c]);
      ss += v[c] * v[c];
    }
    *reinterpret_cast<uint2*>(h_out + (int64_t)m * ld + n) =
        make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
  }
  // per 64 columns (16 lanes of 4): one sum per DPP row of the wave
  ss = sum16(ss);
  const int c64 = (g * FRS_COLS + 64 * (threadIdx.x >> 4)) / 64;
  if ((threadIdx.x & 15) == 0 && c64 < G) sumsq[(int64_t)m * G + c64] = ss;
}

// rope_append_kernel with qkv = the finished q|k|v output of row b; one
// workgroup per (row, head): q and k heads rotate column pairs (d, d + D/2),
// v heads are copied to the cache.
constexpr int ROPE_T = 64;
__global__ void __launch_bounds__(ROPE_T) qkv_rope_append_parts_kernel(
    LinParts o, int Hq, int Hkv, int D, const uint16_t* __restrict__ cos_t,
    const uint16_t* __restrict__ sin_t, int max_pos, const int32_t* __restrict__ context_lens,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    int64_t num_blocks, const int32_t* __restrict__ bt, int64_t bts, int BS, int max_blocks) {
  __shared__ float ts[MAXSEG * 16];
  const int b = blockIdx.x, h = blockIdx.y;
  lin_load_t(o, b, ts);
  __syncthreads();
  const int pos = context_lens[b];
  const int cpos = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
  const int half = D / 2;
  bool slot_ok = pos >= 0 && pos < max_blocks * BS;
  int64_t slot_base = 0;
  if (slot_ok) {
    const int phys = bt[(int64_t)b * bts + pos / BS];
    slot_ok = phys >= 0 && phys < num_blocks;
    slot_base = ((int64_t)phys * Hkv * BS + (pos % BS)) * D;  // + head * BS * D + d
  }
  if (h < Hq + Hkv) {
    uint16_t* dst = nullptr;
    if (h < Hq)
      dst = q_out + ((int64_t)b * Hq + h) * D;
    else if (slot_ok)
      dst = kc + slot_base + (int64_t)(h - Hq) * BS * D;
    if (!dst) return;
    const uint16_t* cr = cos_t + (int64_t)cpos * D;
    const uint16_t* sr = sin_t + (int64_t)cpos * D;
    for (int t = threadIdx.x; t < half / 4; t += ROPE_T) {
      const int d = 4 * t;
      float x1[4], x2[4];
      lin_values4(o, ts, b, h * D + d, x1);
      lin_values4(o, ts, b, h * D + d + half, x2);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int dd = d + c;
        const float o1 =
            round_bf(round_bf(x1[c] * bf2f(cr[dd])) + round_bf(-x2[c] * bf2f(sr[dd])));
        const float o2 = round_bf(round_bf(x2[c] * bf2f(cr[dd + half])) +
                                  round_bf(x1[c] * bf2f(sr[dd + half])));
        dst[dd] = f2bf(o1);
        dst[dd + half] = f2bf(o2);
      }
    }
  } else if (slot_ok) {
    const int hv = h - Hq - Hkv;
    uint16_t* dst = vc + slot_base + (int64_t)hv * BS * D;
    for (int t = threadIdx.x; t < D / 4; t += ROPE_T) {
      float v[4];
      lin_values4(o, ts, b, (Hq + Hkv + hv) * D + 4 * t, v);
#pragma unroll
      for (int c = 0; c < 4; ++c) dst[4 * t + c] = f2bf(v[c]);
    }
  }
}

// silu_mul_kernel with gate|up = the finished linear output of row m (four
// columns per thread).
__global__ void __launch_bounds__(ROW_T) silu_mul_parts_kernel(LinParts o,
                                                               uint16_t* __restrict__ out,
                                                               int64_t ldo) {
  __shared__ float ts[MAXSEG * 16];
  const int m = blockIdx.y, I = o.N / 2;
  lin_load_t(o, m, ts);
  __syncthreads();
  const int i = (blockIdx.x * ROW_T + threadIdx.x) * 4;
  if (i >= I) return;
  float g[4], u[4];
  lin_values4(o, ts, m, i, g);
  lin_values4(o, ts, m, I + i, u);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float s = round_bf(g[c] * (1.f / (1.f + expf(-g[c]))));
    out[(int64_t)m * ldo + i + c] = f2bf(s * u[c]);
  }
}

}  // namespace

extern "C" int grpo_embedding(const int64_t* ids, const void* table, int64_t V, int H, void* out,
                              int B, grpo_stream_t stream) {
  if (B < 0 || H <= 0 || V <= 0) return einval("bad embedding dimensions");
  if (B == 0) return GRPO_OK;
  if (!ids || !table || !out) return einval("null pointer");
  embedding_kernel<<<dim3(B), ROW_T, 0, as_stream(stream)>>>(
      ids, static_cast<const uint16_t*>(table), V, H, static_cast<uint16_t*>(out));
  return launch_check("embedding");
}

extern "C" int grpo_embedding_sumsq(const int64_t* ids, const void* table, int64_t V, int H,
                                    void* out, int B, float* sumsq, grpo_stream_t stream) {
  if (B < 0 || H <= 0 || V <= 0) return einval("bad embedding dimensions");
  if (B == 0) return GRPO_OK;
  if (!ids || !table || !out || !sumsq) return einval("null pointer");
  embedding_sumsq_kernel<<<dim3(B), ROW_T, 0, as_stream(stream)>>>(
      ids, static_cast<const uint16_t*>(table), V, H, static_cast<uint16_t*>(out), sumsq);
  return launch_check("embedding_sumsq");
}

extern "C" int grpo_embedding_sumsq_groups(void) { return ROW_T; }

extern "C" int grpo_add_rmsnorm(const void* x, const void* residual, void* h_out,
                                const void* weight, void* y, int M, int H, float eps,
                                grpo_stream_t stream) {
  if (M < 0 || H <= 0 || H > 16384) return einval("bad rmsnorm dimensions (H <= 16384)");
  if (M == 0) return GRPO_OK;
  if (!x || !weight || !y) return einval("null pointer");
  add_rmsnorm_kernel<<<dim3(M), ROW_T, H * sizeof(float), as_stream(stream)>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(residual),
      static_cast<uint16_t*>(h_out), static_cast<const uint16_t*>(weight),
      static_cast<uint16_t*>(y), H, eps);
  return launch_check("add_rmsnorm");
}

extern "C" int grpo_rope_append(const void* qkv, int64_t ld, int Hq, int Hkv, int D,
                                const void* cos_table, const void* sin_table, int max_pos,
                                const int32_t* context_lens, void* q_out, void* k_cache,
                                void* v_cache, int64_t num_blocks, const int32_t* block_tables,
                                int64_t bt_stride, int block_size, int max_blocks, int B,
                                grpo_stream_t stream) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || D % 2 || block_size <= 0 || max_pos <= 0)
    return einval("bad rope/append dimensions");
  if (ld < (int64_t)(Hq + 2 * Hkv) * D) return einval("qkv row stride too small");
  if (B == 0) return GRPO_OK;
  if (!qkv || !cos_table || !sin_table || !context_lens || !q_out || !k_cache || !v_cache ||
      !block_tables)
    return einval("null pointer");
  rope_append_kernel<<<dim3(B), ROW_T, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(qkv), ld, Hq, Hkv, D, static_cast<const uint16_t*>(cos_table),
      static_cast<const uint16_t*>(sin_table), max_pos, context_lens,
      static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache),
      static_cast<uint16_t*>(v_cache), num_blocks, block_tables, bt_stride, block_size,
      max_blocks);
  return launch_check("rope_append");
}

extern "C" int grpo_silu_mul(const void* gate_up, int64_t ld, int N, void* out, int64_t ldo,
                             int M, grpo_stream_t stream) {
  if (M < 0 || N <= 0 || ld < 2 * (int64_t)N || ldo < N) return einval("bad silu_mul dimensions");
  if (M == 0) return GRPO_OK;
  if (!gate_up || !out) return einval("null pointer");
  silu_mul_kernel<<<dim3((unsigned)cdiv(N, ROW_T), M), ROW_T, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(gate_up), ld, N, static_cast<uint16_t*>(out), ldo);
  return launch_check("silu_mul");
}

extern "C" int grpo_argmax_bf16(const void* logits, int64_t ld, int V, int M, int64_t* out,
                                grpo_stream_t stream) {
  if (M < 0 || V <= 0 || ld < V) return einval("bad argmax dimensions");
  if (M == 0) return GRPO_OK;
  if (!logits || !out) return einval("null pointer");
  argmax_kernel<<<dim3(M), AMAX_T, 0, as_stream(stream)>>>(static_cast<const uint16_t*>(logits),
                                                           ld, V, out);
  return launch_check("argmax");
}

extern "C" int grpo_add_rmsnorm_parts(const grpo_linear_parts_t* x, const void* residual,
                                      void* h_out, const void* weight, void* y, float eps,
                                      grpo_stream_t stream) {
  LinParts o;
  if (int rc = make_parts(x, &o)) return rc;
  if (o.N > 16384) return einval("rmsnorm width must be <= 16384");
  if (!weight || !y) return einval("null pointer");
  if (residual && (reinterpret_cast<uintptr_t>(residual) & 7u) != 0)
    return einval("residual must be 8-byte aligned");
  auto a8 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 7u) == 0; };
  const bool vec = a8(weight) && a8(y) && (!h_out || a8(h_out));  // rows: N % 16 == 0
  const uint16_t* res = static_cast<const uint16_t*>(residual);
  uint16_t* ho = static_cast<uint16_t*>(h_out);
  const uint16_t* wt = static_cast<const uint16_t*>(weight);
  uint16_t* yo = static_cast<uint16_t*>(y);
  // Rows wider than 4 * PARTS_T (Qwen2-7B's 3584) take 1024 threads when the
  // slices fit their registers (8 with LoRA, 16 without), so no column waits
  // for a second round trip after the LoRA-t barrier (64 x 3584 from 7 slices
  // with LoRA: 11.8 us with 512 threads).
  const bool one_pass = o.N > 4 * PARTS_T && o.N <= 4 * 1024;
  const size_t lds512 = std::max(o.N, 4 * PARTS_T) * sizeof(float);
  if (one_pass && o.S <= 8)
    add_rmsnorm_parts_kernel<1024, 8, true>
        <<<dim3(o.M), 1024, 4 * 1024 * sizeof(float), as_stream(stream)>>>(o, res, ho, wt, yo,
                                                                           eps, vec);
  else if (one_pass && o.S <= 16 && o.r == 0)
    add_rmsnorm_parts_kernel<1024, 16, false><<<dim3(o.M), 1024, 0, as_stream(stream)>>>(
        o, res, ho, wt, yo, eps, vec);
  else if (o.S <= 8)
    add_rmsnorm_parts_kernel<PARTS_T, 8, true>
        <<<dim3(o.M), PARTS_T, lds512, as_stream(stream)>>>(o, res, ho, wt, yo, eps, vec);
  else
    add_rmsnorm_parts_kernel<PARTS_T, MAX_SLICES, true>
        <<<dim3(o.M), PARTS_T, lds512, as_stream(stream)>>>(o, res, ho, wt, yo, eps, vec);
  return launch_check("add_rmsnorm_parts");
}

extern "C" int grpo_linear_finish_residual(const grpo_linear_parts_t* x, const void* residual,
                                           void* h_out, int64_t ld, float* sumsq,
                                           grpo_stream_t stream) {
  LinParts o;
  if (int rc = make_parts(x, &o)) return rc;
  if (!h_out || !sumsq) return einval("null pointer");
  if (ld < o.N || ld % 4) return einval("ld must be >= N and a multiple of 4");
  auto a8 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 7u) == 0; };
  if (!a8(h_out) || (residual && !a8(residual)))
    return einval("residual and h_out must be 8-byte aligned");
  if (o.N % 64) return einval("N must be a multiple of 64");
  const int G = o.N / 64;  // sums of squares per row, one per 64 columns
  finish_residual_sumsq_kernel<<<dim3((unsigned)cdiv(o.N, FRS_COLS), (unsigned)o.M), FRS_T, 0,
                                 as_stream(stream)>>>(
      o, static_cast<const uint16_t*>(residual), static_cast<uint16_t*>(h_out), ld, sumsq, G);
  return launch_check("finish_residual_sumsq");
}

extern "C" int grpo_qkv_rope_append_parts(const grpo_linear_parts_t* qkv, int Hq, int Hkv, int D,
                                          const void* cos_table, const void* sin_table,
                                          int max_pos, const int32_t* context_lens, void* q_out,
                                          void* k_cache, void* v_cache, int64_t num_blocks,
                                          const int32_t* block_tables, int64_t bt_stride,
                                          int block_size, int max_blocks, grpo_stream_t stream) {
  LinParts o;
  if (int rc = make_parts(qkv, &o)) return rc;
  if (Hq <= 0 || Hkv <= 0 || D <= 0 || D % 8 || block_size <= 0 || max_pos <= 0)
    return einval("bad rope/append dimensions (head_dim must be a multiple of 8)");
  if (o.N != (Hq + 2 * Hkv) * D) return einval("qkv width must be (Hq + 2 Hkv) * D");
  if (!cos_table || !sin_table || !context_lens || !q_out || !k_cache || !v_cache ||
      !block_tables)
    return einval("null pointer");
  qkv_rope_append_parts_kernel<<<dim3(o.M, Hq + 2 * Hkv), ROPE_T, 0, as_stream(stream)>>>(
      o, Hq, Hkv, D, static_cast<const uint16_t*>(cos_table),
      static_cast<const uint16_t*>(sin_table), max_pos, context_lens,
      static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_cache),
      static_cast<uint16_t*>(v_cache), num_blocks, block_tables, bt_stride, block_size,
      max_blocks);
  return launch_check("qkv_rope_append_parts");
}

extern "C" int grpo_silu_mul_parts(const grpo_linear_parts_t* gate_up, void* out, int64_t ldo,
                                   grpo_stream_t stream) {
  LinParts o;
  if (int rc = make_parts(gate_up, &o)) return rc;
  if (o.N % 2 || ldo < o.N / 2) return einval("bad silu_mul dimensions");
  if (!out) return einval("null pointer");
  silu_mul_parts_kernel<<<dim3((unsigned)cdiv(o.N / 8, ROW_T), o.M), ROW_T, 0,
                          as_stream(stream)>>>(o, static_cast<uint16_t*>(out), ldo);
  return launch_check("silu_mul_parts");
}
