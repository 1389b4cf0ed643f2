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
constexpr int ATTN_MAX_SPLITS = 8;  // context splits of the decode attention

// Host: bps (blocks per split) and number of splits of the split decode
// attention for this shape; GRPO_EUNSUPPORTED outside its fast path.
int attn_plan_geometry(int B, int Hq, int Hkv, int D, int block_size, int max_blocks, int* bps,
                       int* splits);

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

// Host: the NF4 GEMM (nf4_gemm.hip) for batches of more than 64 rows: y[M, N]
// = the reference epilogue of x W^T with W rows wrow0 .. wrow0 + N - 1 of a
// stacked NF4 weight, one bias / LoRA pair per output segment.  nf4_gemm_ok:
// the shapes it takes (per segment).
// With split (S > 1) the launch writes float32 partial sums over S K slices
// of kst stages (part[s][m][n] at slice stride psl, row stride ldp; LoRA t
// partials tpart[s][m][16] at slice stride tsl, r <= 16) for nf4_finish.
// nf4_gemm_plan: slices for this shape (S = 1: no split) and the partial-sum
// bytes of the whole (grouped) linear in the LinParts layout.
struct GemmSplit {
  int S, kst;
  float* part;    // column 0 of the whole linear
  int64_t ldp, psl;
  float* tpart;   // segment s at tpart + s * tseg
  int64_t tsl, tseg;
};
// The output segments of one launch (consecutive column ranges of a stacked
// weight and of y, each with its own bias and LoRA pair).
struct GemmSegs {
  int nseg;
  int seg_end[MAXSEG];
  const uint16_t* bias[MAXSEG];
  const uint16_t* la[MAXSEG];
  const uint16_t* lb[MAXSEG];
};
struct GemmPlan {
  int S, kst;
  size_t part_bytes, tpart_bytes;
};
bool nf4_gemm_ok(int M, int N, int K, int r, int blocksize);
GemmPlan nf4_gemm_plan(int M, int K, int r, int nseg, const int* seg_end);
// The MLP's gate|up projection + SiLU*up on the NF4 GEMM (more than 64 rows):
// act[M, I] = bf16(bf16(silu(x Wg^T)) * bf16(x Wu^T)), W = [2I, K] stacked.
bool nf4_gemm_silu_ok(int M, int I, int K, int blocksize);
int nf4_gemm_silu_launch(const uint16_t* x, int64_t ldx, const uint8_t* w, const float* absmax,
                         const float* code16, int blocksize, int I, int K, int M, uint16_t* act,
                         int64_t lda, hipStream_t st);
// The finish of a K-split GEMM (16 rows per workgroup).
int nf4_gemm_finish(const grpo_linear_parts_t* h, uint16_t* y, int64_t ldy, hipStream_t st);
int nf4_gemm_launch(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t wrow0,
                    const float* absmax, const float* code16, int blocksize,
                    const GemmSegs& segs, int r, float scaling, uint16_t* y, int64_t ldy, int M,
                    int K, hipStream_t st, const GemmSplit* split, bool f16 = false);

// Segment of column n, branch-free: the segment ends are increasing (checked by
// make_parts) and n < N = the last end.  (A loop over seg_end made the compiler
// load one argument per iteration and wait for each in turn.)
__device__ __forceinline__ int lin_seg(const LinParts& o, int n) {
  const int e0 = o.seg_end[0], e1 = o.seg_end[1], e2 = o.seg_end[2];
  return (o.nseg > 1 && n >= e0 ? 1 : 0) + (o.nseg > 2 && n >= e1 ? 1 : 0) +
         (o.nseg > 3 && n >= e2 ? 1 : 0);
}

// a[i] of a kernel-argument array for a per-lane i < MAXSEG, by selects over
// the four uniform entries: indexing the argument array with a per-lane index
// would read it with a dependent vector load instead of scalar loads.
template <typename T>
__device__ __forceinline__ T sel4(T a0, T a1, T a2, T a3, int i) {
  return i == 0 ? a0 : (i == 1 ? a1 : (i == 2 ? a2 : a3));
}
static_assert(MAXSEG == 4, "sel_seg selects among four entries");
#define sel_seg(a, i) sel4((a)[0], (a)[1], (a)[2], (a)[3], (i))

constexpr int MAX_SLICES = 20;  // K slices of a split-K linear (the plan keeps S <= 20)

// LoRA t of row m rounded to bf16, ts[seg*16 + j], computed by the whole
// workgroup (the caller synchronises before reading ts).  The S slices of a
// float4 are loaded together (predicated, no loop), so this is one round trip.
// MS: the most slices (S <= MS).
template <int MS = MAX_SLICES>
__device__ __forceinline__ void lin_load_t(const LinParts& o, int m, float* ts) {
  if (o.r <= 0) return;
  for (int i = threadIdx.x; i < o.nseg * 4; i += blockDim.x) {
    const int seg = i >> 2, q = i & 3;
    const float4* p = reinterpret_cast<const float4*>(o.tpart + ((int64_t)seg * o.M + m) * 16) + q;
    const int64_t stride = (int64_t)o.nseg * o.M * 4;
    // Every load unconditional (slices >= S re-read the last one): predicated
    // loads in this divergent loop were issued one round trip apart.
    float4 v[MS];
#pragma unroll
    for (int k = 0; k < MS; ++k) v[k] = p[min(k, o.S - 1) * stride];
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < MS; ++k)
      if (k < o.S) {
        acc.x += v[k].x;
        acc.y += v[k].y;
        acc.z += v[k].z;
        acc.w += v[k].w;
      }
    float* t = ts + seg * 16 + 4 * q;
    t[0] = round_bf(acc.x);
    t[1] = round_bf(acc.y);
    t[2] = round_bf(acc.z);
    t[3] = round_bf(acc.w);
  }
}

// Inputs of four consecutive outputs (m, n..n+3) of a linear, loaded by
// lin_fetch4 (all loads issued at once) and combined by lin_finish4, so a
// consumer can put a barrier (e.g. for lin_load_t) between the two without a
// second memory round trip.  n % 4 == 0: the four columns lie in one segment.
template <int MS = MAX_SLICES>
struct Fetch4 {
  float4 part[MS];  // requires S <= MS
  uint4 lb[8];  // LoRA B rows (r == 16, aligned): two 16-byte halves per column
  uint2 bias;   // four bf16 biases (aligned)
  int seg, nl;
};

template <int MS>
__device__ __forceinline__ void lin_fetch4(const LinParts& o, int m, int n, Fetch4<MS>& f) {
  const float4* p = reinterpret_cast<const float4*>(o.part + (int64_t)m * o.N + n);
  const int64_t stride = (int64_t)o.M * o.N / 4;
#pragma unroll
  for (int k = 0; k < MS; ++k)
    if (k < o.S) f.part[k] = p[k * stride];
  f.seg = lin_seg(o, n);
  f.nl = n - (f.seg > 0 ? sel_seg(o.seg_end, f.seg - 1) : 0);
  const uint16_t* bias = sel_seg(o.bias, f.seg);
  if (bias && o.bias_vec) f.bias = *reinterpret_cast<const uint2*>(bias + f.nl);
  if (o.r > 0 && o.lb_vec) {
    const uint4* br = reinterpret_cast<const uint4*>(sel_seg(o.lb, f.seg) + (int64_t)f.nl * 16);
#pragma unroll
    for (int j = 0; j < 8; ++j) f.lb[j] = br[j];
  }
}

// LoRA t of row m in two steps, so a caller can issue other loads between
// them: lin_fetch_t loads item i (one float4 of ranks of one segment, all
// slices; i is clamped into range and slices >= S re-read the last one),
// lin_store_t sums and stores the items i < nseg*4.
template <int MS>
__device__ __forceinline__ void lin_fetch_t(const LinParts& o, int m, int i, float4 (&v)[MS]) {
  const int ic = max(0, min(i, o.nseg * 4 - 1));
  const float* base = o.r > 0 ? o.tpart + ((int64_t)(ic >> 2) * o.M + m) * 16 : o.part;
  const float4* p = reinterpret_cast<const float4*>(base) + (o.r > 0 ? (ic & 3) : 0);
  const int64_t stride = o.r > 0 ? (int64_t)o.nseg * o.M * 4 : 0;
#pragma unroll
  for (int k = 0; k < MS; ++k) v[k] = p[min(k, o.S - 1) * stride];
}

template <int MS>
__device__ __forceinline__ void lin_store_t(const LinParts& o, const float4 (&v)[MS], int i,
                                            float* ts) {
  if (o.r <= 0 || i >= o.nseg * 4) return;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < MS; ++k)
    if (k < o.S) {
      acc.x += v[k].x;
      acc.y += v[k].y;
      acc.z += v[k].z;
      acc.w += v[k].w;
    }
  float* t = ts + (i >> 2) * 16 + 4 * (i & 3);
  t[0] = round_bf(acc.x);
  t[1] = round_bf(acc.y);
  t[2] = round_bf(acc.z);
  t[3] = round_bf(acc.w);
}

// LoRA B rows of one wave's 256 consecutive output columns c0 .. c0 + 255
// (r == 16, one segment, 16-byte aligned B): load k of lane l is the 16 bytes
// of ranks 8 (l & 1) .. + 7 of column c0 + 32 k + l / 2, so every load
// instruction reads 1 KiB contiguous.  (Lane l's own four columns are 128
// contiguous bytes; read that way each instruction touches 64 cache lines,
// and the address unit takes a cycle per line.)  Columns past N re-read
// column N - 1.  Every lane of the wave calls it.
__device__ __forceinline__ void lin_fetch_lb_wave(const LinParts& o, int c0, uint4 (&lb)[8]) {
  const int l = threadIdx.x & 63;
  const uint16_t* b = o.lb[0] + 8 * (l & 1);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int col = min(c0 + 32 * k + (l >> 1), o.N - 1);
    lb[k] = *reinterpret_cast<const uint4*>(b + (int64_t)col * 16);
  }
}

// t . B[n, :] for lane l's four columns c0 + 4 l .. + 3 from the rows of
// lin_fetch_lb_wave: the two lanes of a column each sum eight ranks (in rank
// order) and add the other's sum; the column sums pass through lu (this
// wave's 256 floats of LDS) to the lane that owns the column.  Every lane of
// the wave calls it.
__device__ __forceinline__ float4 lin_lora_wave(const float* ts, const uint4 (&lb)[8],
                                                float* lu) {
  const int l = threadIdx.x & 63;
  const float* t = ts + 8 * (l & 1);
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t w[4] = {lb[k].x, lb[k].y, lb[k].z, lb[k].w};
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s += t[2 * j] * bf_lo(w[j]);
      s += t[2 * j + 1] * bf_hi(w[j]);
    }
    s += dpp_move<0xB1>(s);  // quad_perm [1,0,3,2]: the other half of the column
    if (!(l & 1)) lu[32 * k + (l >> 1)] = s;
  }
  // LDS serves one wave's instructions in order: no barrier between the
  // writes and the reads of other lanes' sums
  __builtin_amdgcn_wave_barrier();
  return *reinterpret_cast<const float4*>(lu + 4 * l);
}

// The reference's bf16 values (as floats) of the four outputs; ts holds the
// row's LoRA t (lin_load_t) when r > 0.
// has_u: lora_u holds the four t . B[n, :] sums (lin_lora_wave); else they
// are computed here from f.lb or B.
template <int MS>
__device__ __forceinline__ void lin_finish4(const LinParts& o, const float* ts,
                                            const Fetch4<MS>& f, float v[4], bool has_u = false,
                                            float4 lora_u = float4{0.f, 0.f, 0.f, 0.f}) {
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < MS; ++k)
    if (k < o.S) {
      acc.x += f.part[k].x;
      acc.y += f.part[k].y;
      acc.z += f.part[k].z;
      acc.w += f.part[k].w;
    }
  v[0] = round_bf(acc.x);
  v[1] = round_bf(acc.y);
  v[2] = round_bf(acc.z);
  v[3] = round_bf(acc.w);
  const uint16_t* bias = sel_seg(o.bias, f.seg);
  if (bias) {
    float b[4];
    if (o.bias_vec) {
      b[0] = bf_lo(f.bias.x);
      b[1] = bf_hi(f.bias.x);
      b[2] = bf_lo(f.bias.y);
      b[3] = bf_hi(f.bias.y);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) b[c] = bf2f(bias[f.nl + c]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = round_bf(v[c] + b[c]);
  }
  if (o.r > 0) {
    const float* t = ts + f.seg * 16;
    const float sc = round_bf(o.scaling);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float u = 0.f;
      if (has_u) {
        u = c == 0 ? lora_u.x : (c == 1 ? lora_u.y : (c == 2 ? lora_u.z : lora_u.w));
      } else if (o.lb_vec) {
        const uint4 b0 = f.lb[2 * c], b1 = f.lb[2 * c + 1];
        const uint32_t bw[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          u += t[2 * j] * bf_lo(bw[j]);
          u += t[2 * j + 1] * bf_hi(bw[j]);
        }
      } else {
        const uint16_t* br = sel_seg(o.lb, f.seg) + (int64_t)(f.nl + c) * o.r;
        for (int j = 0; j < o.r; ++j) u += t[j] * bf2f(br[j]);
      }
      u = round_bf(round_bf(u) * sc);
      v[c] = round_bf(v[c] + u);
    }
  }
}

// Outputs (m, n..n+3) as the reference's bf16 values (fetch + finish).
__device__ __forceinline__ void lin_values4(const LinParts& o, const float* ts, int m, int n,
                                            float v[4]) {
  Fetch4<> f;
  lin_fetch4(o, m, n, f);
  lin_finish4(o, ts, f, v);
}

}  // namespace grpo
