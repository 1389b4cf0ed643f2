// NF4 dequantization and the split-K NF4 + LoRA linear for gfx950.
//
// Weight format (bitsandbytes Params4bit, read by the reference in
// src/triton_kernels/lora_forward.py:171-206): W[N,K] flattened row-major,
// element e = n*K + k, byte e/2, even e = high nibble; one float32 absmax per
// `blocksize` flat elements; value = bf16_rne(code[q] * absmax).
//
// Split-K linear (M <= 64, K % 256 == 0, N % 16 == 0, r <= 16, power-of-two
// blocksize >= 64): D = A*B on v_mfma_f32_16x16x32_bf16 with A = x (rows m)
// and B = W^T (columns n).
//
//  * Work unit: one wave = one 16-row n-tile x one slice of KPW k-steps of
//    256.  A workgroup is 4 waves = 4 consecutive n-tiles of one slice; the
//    grid is (tile groups, slices), sized for >= ~2048 waves when the shape
//    allows it.  Decode shapes have only 96..1120 n-tiles: without the K split
//    most CUs would idle while a few run the VALU-heavy nibble decode.
//  * Lane (n = lane%16, group g = lane/16) owns the 64-element chunk
//    [kstep*256 + 64g, +64) of row n: two 16-byte loads per k-step.  A wave
//    issues all its weight and absmax loads before it decodes anything.
//  * Decode: per chunk a 16-entry bf16 codebook bf16(code[j] * absmax) is built
//    in registers and nibbles are expanded with v_perm byte lookups, so every
//    product is exactly the reference's bf16(code*absmax) * x.  decode8 emits a
//    dword's eight elements in the order [0,2,4,6,1,3,5,7]; the workgroup
//    stages its slice of x in LDS permuted the same way.
//  * x rows >= M: those lanes read row M-1 instead (no masking); the MFMA
//    output rows they produce are never stored.
//  * LoRA: x A_s^T is one more 16-column tile per segment (A is bf16: no
//    decode), computed by extra waves of every slice.
//  * Output: float32 partial sums part[slice][m][n] and tpart[slice][seg][m][16].
//    There is no cross-workgroup synchronisation; the sum over slices (fixed
//    order) and the reference epilogue run in the consuming kernel
//    (linear_parts.hpp): nf4_finish here, or a fused decode-step op.
#include <algorithm>
#include <type_traits>

#include "linear_parts.hpp"
#include "nf4_decode.hpp"

using namespace grpo;

namespace {

constexpr int PART_WAVES = 4;       // n-tiles (waves) per workgroup, x given in bf16
constexpr int PART_LDS_MAX = 65536; // bytes of the staged x slice per workgroup (M <= 16)
// Wide batches (M > 16) may stage up to all of gfx950's 160 KiB per workgroup:
// x of 64 rows then covers 4 k-steps, so K slices stay few (fewer partial sums)
// and long-K linears need no row chunks (each of which re-read the weights).
constexpr int PART_LDS_BIG = 163840;
constexpr int KPW_MAX = 8;          // k-steps per wave (all loads in flight at once)
// x slices of 5 k-steps (only planned for more than 16 rows) are staged
// chunk-major in LDS (nf4_part_mfma's xs_offset).
__host__ __device__ constexpr bool xs_chunk_major(int MT, int kpw) { return MT > 1 && kpw == 5; }
#ifndef GRPO_TARGET_WAVES
#define GRPO_TARGET_WAVES 2048
#endif
int g_target_waves = GRPO_TARGET_WAVES;  // launch-shape target: 8 waves per CU on 256 CUs

// ------------------------------------------------------------- dequant --

// F16: float16_rne(code * absmax) instead of bf16 (the weight cast to a float16
// grad / LoRA dtype in the reference's backward and forward).
template <bool F16>
__global__ void __launch_bounds__(256) nf4_dequant_vec(const uint2* __restrict__ w,
                                                       const float* __restrict__ absmax,
                                                       const float* __restrict__ code16,
                                                       uint4* __restrict__ out, int64_t nvec,
                                                       int blocksize) {
  __shared__ float code[16];
  if (threadIdx.x < 16) code[threadIdx.x] = code16[threadIdx.x];
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nvec; i += stride) {
    const uint2 p = w[i];
    const float a = absmax[(i * 16) / blocksize];
    uint32_t o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t byte = ((j < 4 ? p.x : p.y) >> (8 * (j & 3))) & 0xFFu;
      const float hi = code[byte >> 4] * a;   // element 2j (even): high nibble
      const float lo = code[byte & 15u] * a;  // element 2j+1 (odd): low nibble
      o[j] = pack_e2<F16>(hi, lo);
    }
    out[2 * i] = make_uint4(o[0], o[1], o[2], o[3]);
    out[2 * i + 1] = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

template <bool F16>
__global__ void __launch_bounds__(256) nf4_dequant_scalar(const uint8_t* __restrict__ w,
                                                          const float* __restrict__ absmax,
                                                          const float* __restrict__ code16,
                                                          uint16_t* __restrict__ out,
                                                          int64_t numel, int blocksize) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < numel; e += stride) {
    const uint32_t byte = w[e >> 1];
    const uint32_t q = (e & 1) ? (byte & 15u) : (byte >> 4);
    out[e] = f2e<F16>(code16[q] * absmax[e / blocksize]);
  }
}

// ---------------------------------------------------- split-K linear --

struct PartArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  const float* absmax;
  const float* code16;
  int bs_shift;  // log2(blocksize)
  const uint16_t* la[MAXSEG];
  float* part;   // rows of this launch: part[slice][m][n] at slice stride Mp*N
  float* tpart;  // tpart[slice][seg][m][16] at seg stride Mp*16
  int M, N, K, NT, ntiles, nseg, r;
  int Mp;       // rows of the partial-sum layout (M, or more when rows are launched in chunks)
  int xstride;  // LDS row stride of the staged x slice (elements)
  // x = decode attention output given as split partials (o_proj of the decode step)
  const float* att_o;    // [M][Hq][S][128] unnormalised O
  const float* att_ml;   // [M][Hq][S][2]: max (log2 domain), sum
  const int32_t* att_len;
  int att_S, att_bps, att_Hq, att_cap;
  // x = SiLU(gate) * up from the gate|up projection's partial sums (down_proj)
  const float* gu_part;  // [gu_S][M][2 * K]
  int gu_S;
  // x = RMSNorm(h) with the statistic given as per-group sums of squares
  // (q|k|v of the decode step after nf4_fold_residual)
  const uint16_t* nh;  // h [M][ldnh] bf16
  int64_t ldnh;
  const float* nss;    // [M][nG]: sums of h^2 over column groups
  int nG;
  const uint16_t* nw;  // RMSNorm weight [K] bf16
  float neps;
  // Finish in the kernel (FIN): the K slice of a tile group that arrives last
  // sums the group's partials and writes h = residual + y for its columns.
  float* fin_tpart;         // [groups][S][M][16]: LoRA t partials of each group's slices
  int* fin_cnt;             // [groups * FIN_CNT_STRIDE] arrival counters: zero, left zero
  int* fin_err;             // set to 1 when a group's slices ran on two XCDs (xcd_arrive)
  const uint16_t* fin_res;  // residual [M][fin_ld] bf16 (may alias fin_h)
  uint16_t* fin_h;          // h [M][fin_ld] bf16
  int64_t fin_ld;
  float* fin_ss;            // [M][groups]: sums of h^2 over each group's columns
  const uint16_t* fin_bias; // [N] bf16 or null
  const uint16_t* fin_lb;   // LoRA B [N][r] bf16 (r > 0)
  float fin_scaling;
  int fin_lb_vec;           // r == 16 and lora_b 16-byte aligned
};

// X_WIDE: bf16, 16 waves; X_NORM: RMSNorm of h from per-group sums of squares;
// X_WIDE8: X_WIDE on 8 waves (launches whose 16-wave grid fills at most half
// the CUs)
enum XSource { X_BF16 = 0, X_ATTN = 1, X_SILU = 2, X_WIDE = 3, X_NORM = 4, X_WIDE8 = 5 };
// One arrival counter per 128-byte line: a tile group's counter line is only
// ever touched by the workgroups of that group, which share one XCD's L2.
constexpr int FIN_CNT_STRIDE = 32;
constexpr int FIN_MAX_SLICES = 8;
constexpr int NORM_MAX_GROUPS = 256;  // sums of squares per row the X_NORM source reads

// n-tiles (waves) per workgroup.  Every workgroup of a K slice rebuilds the x
// slice it stages; the SiLU source reads 16 bytes of partial sums per element,
// so its workgroups are larger (fewer rebuilds).  Measured at decode shapes:
// the attention-merge source is fastest with the default 4.  Wide batches whose
// x slice takes more than 64 KiB of LDS (X_WIDE) run one workgroup per CU, so
// it has 16 waves: four per SIMD keep enough weight loads in flight, and 16
// tiles share each staged copy of x (a quarter of the L2 -> LDS traffic of 4).
// When 16-wave workgroups would leave more than half of the CUs idle and two
// workgroups fit a CU, X_WIDE8 takes twice as many 8-wave workgroups
// (Qwen2-7B's o_proj at 64 rows: 112 -> 224 workgroups, 11.9 -> 9.0 us).
#ifndef GRPO_ATTN_WAVES
#define GRPO_ATTN_WAVES PART_WAVES
#endif
__host__ __device__ constexpr int waves_per_group(int xsrc) {
  return xsrc == X_SILU || xsrc == X_WIDE8
             ? 8
             : (xsrc == X_ATTN ? GRPO_ATTN_WAVES : (xsrc == X_WIDE ? 16 : PART_WAVES));
}
__host__ __device__ constexpr bool wide_source(int xsrc) { return xsrc == X_WIDE || xsrc == X_WIDE8; }
__host__ __device__ constexpr bool bf16_source(int xsrc) {
  return xsrc == X_BF16 || wide_source(xsrc);
}
constexpr int GU_MAX_SLICES = 2;  // K slices of the gate|up partial sums read while staging

// Columns k..k+7 of row m of bf16(bf16(silu(g)) * u), with g = bf16(sum of the
// gate partials), u = bf16(sum of the up partials) (fused_ops.py:79-112 applied
// to the finished gate|up output).  silu_fetch issues the loads, silu_finish
// combines them, so the loads can go out before the kernel's weight loads.
struct SiluFetch {
  float4 g[GU_MAX_SLICES][2], u[GU_MAX_SLICES][2];
};

__device__ __forceinline__ void silu_fetch(const PartArgs& p, int m, int k, SiluFetch& f) {
  const int64_t row = (int64_t)m * 2 * p.K;
  const int64_t stride = (int64_t)p.M * 2 * p.K / 4;
  const float4* pg = reinterpret_cast<const float4*>(p.gu_part + row + k);
  const float4* pu = reinterpret_cast<const float4*>(p.gu_part + row + p.K + k);
#pragma unroll
  for (int s = 0; s < GU_MAX_SLICES; ++s)
    if (s < p.gu_S) {
      f.g[s][0] = pg[s * stride];
      f.g[s][1] = pg[s * stride + 1];
      f.u[s][0] = pu[s * stride];
      f.u[s][1] = pu[s * stride + 1];
    }
}

__device__ __forceinline__ uint4 silu_finish(const PartArgs& p, const SiluFetch& f) {
  float gs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float us[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < GU_MAX_SLICES; ++s)
    if (s < p.gu_S) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        gs[4 * h + 0] += f.g[s][h].x;
        gs[4 * h + 1] += f.g[s][h].y;
        gs[4 * h + 2] += f.g[s][h].z;
        gs[4 * h + 3] += f.g[s][h].w;
        us[4 * h + 0] += f.u[s][h].x;
        us[4 * h + 1] += f.u[s][h].y;
        us[4 * h + 2] += f.u[s][h].z;
        us[4 * h + 3] += f.u[s][h].w;
      }
    }
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float gv = round_bf(gs[j]);
    o[j] = round_bf(gv * (1.f / (1.f + expf(-gv)))) * round_bf(us[j]);
  }
  return make_uint4(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]), pack_bf2(o[4], o[5]),
                    pack_bf2(o[6], o[7]));
}

__device__ __forceinline__ uint4 silu_chunk(const PartArgs& p, int m, int k) {
  SiluFetch f;
  silu_fetch(p, m, k, f);
  return silu_finish(p, f);
}

// Eight consecutive columns k..k+7 (one head, d0 = k % 128) of row m of the
// attention output, merged over its context splits:
// O = sum_s 2^(m_s - M) O_s / max(sum_s 2^(m_s - M) l_s, 1e-6), rounded to bf16
// (the reference's float32 attention output cast to the model dtype).
// attn_fetch loads every allocated split slot (only the row's ns <= att_S used
// splits are merged): the addresses do not depend on the context length, so
// these loads can be issued before the weights.
struct AttnFetch {
  float4 o0[ATTN_MAX_SPLITS], o1[ATTN_MAX_SPLITS];
  float2 ml[ATTN_MAX_SPLITS];
  int len;
};

__device__ __forceinline__ void attn_fetch(const PartArgs& p, int m, int k, AttnFetch& f) {
  const int hq = k >> 7, d0 = k & 127;
  f.len = p.att_len[m];
  const int64_t base = ((int64_t)m * p.att_Hq + hq) * p.att_S;
#pragma unroll
  for (int s = 0; s < ATTN_MAX_SPLITS; ++s)
    if (s < p.att_S) {
      const int64_t sl = base + s;
      f.ml[s] = *reinterpret_cast<const float2*>(p.att_ml + sl * 2);
      const float4* op = reinterpret_cast<const float4*>(p.att_o + sl * 128 + d0);
      f.o0[s] = op[0];
      f.o1[s] = op[1];
    }
}

__device__ __forceinline__ uint4 attn_finish(const PartArgs& p, const AttnFetch& f) {
  int ctx = f.len;
  ctx = ctx < 0 ? 0 : (ctx > p.att_cap ? p.att_cap : ctx);
  const int nblk = (ctx + 15) / 16;
  const int ns = nblk > 0 ? (nblk + p.att_bps - 1) / p.att_bps : 1;
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < ATTN_MAX_SPLITS; ++s)
    if (s < ns) M = fmaxf(M, f.ml[s].x);
  float L = 0.f, O[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (M != -INFINITY) {
#pragma unroll
    for (int s = 0; s < ATTN_MAX_SPLITS; ++s)
      if (s < ns) {
        const float w = exp2f(f.ml[s].x - M);
        L += w * f.ml[s].y;
        O[0] += w * f.o0[s].x;
        O[1] += w * f.o0[s].y;
        O[2] += w * f.o0[s].z;
        O[3] += w * f.o0[s].w;
        O[4] += w * f.o1[s].x;
        O[5] += w * f.o1[s].y;
        O[6] += w * f.o1[s].z;
        O[7] += w * f.o1[s].w;
      }
  }
  const float den = fmaxf(L, 1e-6f);
  return make_uint4(pack_bf2(O[0] / den, O[1] / den), pack_bf2(O[2] / den, O[3] / den),
                    pack_bf2(O[4] / den, O[5] / den), pack_bf2(O[6] / den, O[7] / den));
}

__device__ __forceinline__ uint4 attn_chunk(const PartArgs& p, int m, int k) {
  AttnFetch f;
  attn_fetch(p, m, k, f);
  return attn_finish(p, f);
}

// Last-arriver finish of tile group g (FIN): columns n0 .. n0 + 16 * WPG - 1 of
// every row, n0 = g * 16 * WPG, from the partial sums and LoRA t partials that
// the group's S workgroups (one per K slice) stored.  Wave w finishes the
// group's n-tile w in the MFMA layout of the linear itself: lane (n = lane %
// 16, lg = lane / 16) owns rows m = 4 lg + r (r < 4) of column n0 + 16 w + n.
// The reference epilogue (lora_forward.py:243-257) in the order and roundings
// of lin_finish4 (linear_parts.hpp), except that the LoRA product
// u = t . B[n, :] is one 16x16x16 bf16 MFMA (bf16 t and B, float32
// accumulation, as the reference's tl.dot), then h = bf16(residual + y) and
// fin_ss[m][g] = sum over the group's columns of h^2.  The finish code is short
// on purpose: the last arriver runs it once per launch with a cold instruction
// cache, and one wave's serial VALU chain is its critical path.
struct FinPre {
  uint32_t res[2];  // residual of rows 4 lg .. 4 lg + 3 at this lane's column (bf16 pairs)
  uint32_t lb[2];   // LoRA B[column][4 lg .. 4 lg + 3] (bf16, zero past r)
  float bias;
};

__device__ __forceinline__ int fin_col(int g, int wpg) {
  return g * 16 * wpg + 16 * (threadIdx.x >> 6) + (threadIdx.x & 15);
}

template <int WPG>
__device__ __forceinline__ void fin_prefetch(const PartArgs& p, int g, FinPre& f) {
  const int lg = (threadIdx.x & 63) >> 4;
  const int col = fin_col(g, WPG);
  uint32_t rv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) rv[r] = p.fin_res[(int64_t)min(4 * lg + r, p.M - 1) * p.fin_ld + col];
  f.res[0] = rv[0] | (rv[1] << 16);
  f.res[1] = rv[2] | (rv[3] << 16);
  f.bias = p.fin_bias ? bf2f(p.fin_bias[col]) : 0.f;
  f.lb[0] = f.lb[1] = 0;
  if (p.r > 0) {
    if (p.fin_lb_vec) {
      const uint2 v = *reinterpret_cast<const uint2*>(p.fin_lb + (int64_t)col * 16 + 4 * lg);
      f.lb[0] = v.x;
      f.lb[1] = v.y;
    } else {
      uint32_t b[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = 4 * lg + j < p.r ? p.fin_lb[(int64_t)col * p.r + 4 * lg + j] : 0u;
      f.lb[0] = b[0] | (b[1] << 16);
      f.lb[1] = b[2] | (b[3] << 16);
    }
  }
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));

template <int WPG, int S>
__device__ __forceinline__ void fin_group_s(const PartArgs& p, int g, const FinPre& f) {
  __shared__ float red[WPG][16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int G = p.NT / WPG;
  const int col = fin_col(g, WPG);
  // every load goes out at once: buffer loads with the slice offset in a
  // scalar register (no per-load address arithmetic)
  constexpr int BUF_FLAGS = 0x00020000;
  const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(p.part), 0, 0x7fffffff, BUF_FLAGS);
  float pv[S][4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int vo = (min(4 * lg + r, p.M - 1) * p.N + col) * 4;
#pragma unroll
    for (int s = 0; s < S; ++s)
      pv[s][r] = __uint_as_float(
          __builtin_amdgcn_raw_buffer_load_b32(rp, vo, s * p.Mp * p.N * 4, 0));
  }
  u32x4_t tv[S];
  if (p.r > 0) {
    const __amdgpu_buffer_rsrc_t rt =
        __builtin_amdgcn_make_buffer_rsrc(p.fin_tpart, 0, 0x7fffffff, BUF_FLAGS);
    const int vo = (min(ln, p.M - 1) * 16 + 4 * lg) * 4;
#pragma unroll
    for (int s = 0; s < S; ++s)
      tv[s] = __builtin_amdgcn_raw_buffer_load_b128(rt, vo, (g * S + s) * p.M * 64, 0);
  }
  // u[m][n] = t[m, :] . B[n, :]: t = bf16(sum over slices), rows m = lane % 16
  f32x4_t u = {0.f, 0.f, 0.f, 0.f};
  if (p.r > 0) {
    float t[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] += __uint_as_float(tv[s][i]);
    const uint32_t a0 = pack_bf2(t[0], t[1]), a1 = pack_bf2(t[2], t[3]);
    const i16x4_t av = __builtin_bit_cast(i16x4_t, make_uint2(a0, a1));
    const i16x4_t bv = __builtin_bit_cast(i16x4_t, make_uint2(f.lb[0], f.lb[1]));
    u = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, u, 0, 0, 0);
  }
  const float sc = round_bf(p.fin_scaling);
  const float res[4] = {bf_lo(f.res[0]), bf_hi(f.res[0]), bf_lo(f.res[1]), bf_hi(f.res[1])};
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < S; ++s)
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] += pv[s][r];
  float sq[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v = round_bf(acc[r]);
    if (p.fin_bias) v = round_bf(v + f.bias);
    if (p.r > 0) v = round_bf(v + round_bf(round_bf(u[r]) * sc));
    const float h = round_bf(v + res[r]);
    const int m = 4 * lg + r;
    if (m < p.M) p.fin_h[(int64_t)m * p.fin_ld + col] = f2bf(h);
    sq[r] = m < p.M ? h * h : 0.f;
  }
  // sums of h^2 of each row: over this wave's 16 columns (one DPP row of
  // lanes), then over the group's WPG waves in wave order
#pragma unroll
  for (int r = 0; r < 4; ++r) sq[r] = sum16(sq[r]);
  if (ln == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[w][4 * lg + r] = sq[r];
  }
  __syncthreads();
  if (threadIdx.x < p.M) {
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < WPG; ++i) tot += red[i][threadIdx.x];
    p.fin_ss[(int64_t)threadIdx.x * G + g] = tot;
  }
}

// The slice count is a template argument, so the finish has no per-slice
// selects (gridDim.y = S <= FIN_MAX_SLICES, checked by the host).
template <int WPG>
__device__ __forceinline__ void fin_group(const PartArgs& p, int g, const FinPre& f) {
  switch (gridDim.y) {
    case 1: fin_group_s<WPG, 1>(p, g, f); break;
    case 2: fin_group_s<WPG, 2>(p, g, f); break;
    case 3: fin_group_s<WPG, 3>(p, g, f); break;
    case 4: fin_group_s<WPG, 4>(p, g, f); break;
    case 5: fin_group_s<WPG, 5>(p, g, f); break;
    case 6: fin_group_s<WPG, 6>(p, g, f); break;
    case 7: fin_group_s<WPG, 7>(p, g, f); break;
    default: fin_group_s<WPG, 8>(p, g, f); break;
  }
}

// Waves per SIMD the compiler plans registers for: the default range (enough
// for one workgroup, up to 8) except for the X_NORM source (the decode step's
// q|k|v, at most one workgroup per CU in practice), planned for at most two:
// the schedule then keeps more loads and decodes in flight (config 3 q|k|v
// 4.12 -> 3.91 us per launch).
template <int MT, int KPW, int XSRC, bool FIN = false>
__global__ void __launch_bounds__(64 * waves_per_group(XSRC))
__attribute__((amdgpu_waves_per_eu((waves_per_group(XSRC) + 3) / 4, XSRC == X_NORM ? 2 : 8)))
nf4_part_mfma(PartArgs p) {
  touch_kernargs<sizeof(PartArgs)>();
  constexpr int WPG = waves_per_group(XSRC), NT = 64 * WPG;
  extern __shared__ __align__(16) uint16_t xs[];  // x slice in decode8 order (xs_offset)
  // Padding workgroups of the XCD-aligned grid have no tile at all.
  if ((int)blockIdx.x * WPG >= p.ntiles) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  // FIN: wave 0 also takes the LoRA-A tile of this K slice for its group
  // (every group computes its own copy, so the group's finish reads nothing
  // written on another XCD).
  const bool lwave = FIN && wave == 0;
  const int tile = blockIdx.x * WPG + wave;
  const int slice = blockIdx.y;
  const int ks0 = slice * KPW;
  const int nk = min(KPW, p.K / KSTEP - ks0);  // >= 1: the host sizes the grid
  const int kbase = ks0 * KSTEP;
  const bool wtile = tile < p.NT;
  const int n_row = tile * 16 + ln;

  // Load order.  Vector loads retire in issue order and the compiler waits for
  // a load with s_waitcnt vmcnt(N), N = loads issued after it; after a
  // conditional load it can only assume the fewest loads, so a conditional
  // load makes the waits of the loads issued BEFORE it conservative, never of
  // those after it.  Hence: the codebook (scalar loads), then the first batch
  // of the x source (predicated: only the chunks that exist), then the weights
  // k-step by k-step, unconditional (indexes clamped into range, extra values
  // discarded).  The staging then waits only for x, and decoding k-step i only
  // for that step's weights while later steps are in flight.  (With the
  // weight loads conditional, the staging had to wait with vmcnt(0), i.e. for
  // the whole workgroup's weights.)
  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];

  // x chunk i (16 bytes: 8 K values of one row) -> (row m, chunk c of the
  // slice): row-major, or (CM) in groups of 64 chunks of 8 rows x 8
  // consecutive chunks, 8 consecutive threads on one row, so every 8 threads
  // load one 128-byte line (a row-fastest order, which writes LDS without
  // bank conflicts, measured 1.4 us slower on Qwen2-7B's down_proj: its loads
  // touch 4x the lines per quad); rows past M repeat row M - 1.
  constexpr bool CM = xs_chunk_major(MT, KPW);
  constexpr int XROWS = MT * 16;  // CM: LDS rows of each chunk
  const int chunks = nk * (KSTEP / 8);
  const int total = CM ? ((p.M + 7) & ~7) * chunks : p.M * chunks;
  auto chunk_mc = [&](int i, int& m, int& c) __attribute__((always_inline)) {
    if (CM) {
      const int blk = i >> 6, l = i & 63, nbc = chunks >> 3;
      const int mb = blk / nbc;
      m = min(8 * mb + (l >> 3), p.M - 1);
      c = 8 * (blk - mb * nbc) + (l & 7);
    } else {
      m = i / chunks;
      c = i - m * chunks;
    }
  };
  // LDS element offset of chunk c of row m: row-major [M][xstride] (8 padding
  // columns stagger the rows over the banks), or (CM) chunk-major
  // [chunk][XROWS][8], where the 16 rows of one MFMA A operand are 256
  // contiguous bytes (no bank conflict without padding)
  auto xs_offset = [&](int m, int c) __attribute__((always_inline)) {
    return CM ? (c * XROWS + m) * 8 : m * p.xstride + 8 * c;
  };
  uint4 xv[4];
  constexpr int SF = 2;  // SiLU chunks per thread fetched ahead
  SiluFetch sf[SF];
  AttnFetch af;  // one attention chunk per thread fetched ahead
  // X_NORM: sums of squares of row tid / 16 (16 threads per row, M <= 16),
  // then h and the norm weight of this thread's first chunks
  constexpr int NSS = NORM_MAX_GROUPS / 16;
  float ssv[NSS];
  uint4 nwv[4];
  if (XSRC == X_NORM) {
    // unconditional loads of clamped indexes (values outside the row's groups
    // are dropped in the sum): predicated loads here made the compiler copy
    // the whole array per load and wait for each in turn
    const float* ssr = p.nss + (int64_t)min(tid >> 4, p.M - 1) * p.nG;
    const int j = tid & 15;
#pragma unroll
    for (int i = 0; i < NSS; ++i) ssv[i] = ssr[min(j + 16 * i, p.nG - 1)];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (u * NT >= total) break;
      const int i = min(u * NT + tid, total - 1);
      int m, c;
      chunk_mc(i, m, c);
      xv[u] = *reinterpret_cast<const uint4*>(p.nh + (int64_t)m * p.ldnh + kbase + 8 * c);
      nwv[u] = *reinterpret_cast<const uint4*>(p.nw + kbase + 8 * c);
    }
  } else if (bf16_source(XSRC)) {
    // bf16 x: whole batch entries past the end are skipped (uniform), a partial
    // one re-reads the last chunk (clamped), so no load is predicated.  (The
    // predicated form makes the compiler wait for every weight after staging.)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (u * NT >= total) break;
      const int i = min(u * NT + tid, total - 1);
      int m, c;
      chunk_mc(i, m, c);
      xv[u] = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + kbase + 8 * c);
    }
  } else if (XSRC == X_SILU) {
#pragma unroll
    for (int u = 0; u < SF; ++u) {
      const int i = u * NT + tid;
      if (i < total) {
        int m, c;
        chunk_mc(i, m, c);
        silu_fetch(p, m, kbase + 8 * c, sf[u]);
      }
    }
  } else if (tid < total) {
    int m, c;
    chunk_mc(tid, m, c);
    attn_fetch(p, m, kbase + 8 * c, af);
  }
  // Keep the scheduler from hoisting the (cheaper to address) weight loads
  // above the x loads.
  __builtin_amdgcn_sched_barrier(0);

  // Weight and absmax loads of every k-step.  LoRA and padding waves read row
  // 0 and the last k-step is re-read past nk; those values are never used.
  uint4 wv[2 * KPW];
  float av[KPW];
  {
    const int wr = wtile ? n_row : 0;
    const uint8_t* wrow = p.w + (int64_t)wr * (p.K / 2);
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kc = kbase + min(i, nk - 1) * KSTEP + 64 * lg;
      const uint4* wp = reinterpret_cast<const uint4*>(wrow + kc / 2);
      wv[2 * i] = load_w<!wide_source(XSRC)>(wp);
      wv[2 * i + 1] = load_w<!wide_source(XSRC)>(wp + 1);
      av[i] = p.absmax[((int64_t)wr * p.K + kc) >> p.bs_shift];
    }
  }
  // FIN: the finish's inputs that no K slice produces, behind the weights (the
  // MFMAs wait only for the loads before them), and the LoRA wave's A rows
  FinPre fpre;
  if (FIN) fin_prefetch<WPG>(p, blockIdx.x, fpre);
  uint4 a8f[FIN ? 8 * KPW : 1];
  if (FIN && lwave && p.r > 0) {
    const uint16_t* arow = p.la[0] + (int64_t)(ln < p.r ? ln : 0) * p.K + kbase + 64 * lg;
#pragma unroll
    for (int i = 0; i < KPW; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        a8f[8 * i + j] = *reinterpret_cast<const uint4*>(arow + min(i, nk - 1) * KSTEP + 8 * j);
  }

  // Stage x[:, kbase : kbase + nk*256] in LDS (decode8 order), four chunks per
  // thread per batch.  A batch entry that starts past the end is skipped by
  // the whole workgroup.  The bf16 source clamps the chunk index (the last
  // chunk is then written twice with the same value); the other sources
  // predicate.  At decode shapes every chunk comes from the loads issued
  // above; larger M stages the rest here, behind the weights.
  constexpr bool CLAMP = bf16_source(XSRC) || XSRC == X_NORM;
  __shared__ float sInv[16];
  if (XSRC == X_NORM) {
    // 1 / rms of each row: the row's group sums in order per thread, then
    // across its 16 threads
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NSS; ++i) ss += (tid & 15) + 16 * i < p.nG ? ssv[i] : 0.f;
    ss = sum16(ss);
    if ((tid & 15) == 0 && (tid >> 4) < p.M)
      sInv[tid >> 4] = 1.f / sqrtf(ss / (float)p.K + p.neps);
    __syncthreads();
  }
  for (int base = 0; base < total; base += 4 * NT) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (base + u * NT >= total) break;
      const int i = CLAMP ? min(base + u * NT + tid, total - 1) : base + u * NT + tid;
      if (CLAMP || i < total) {
        int m, c;
        chunk_mc(i, m, c);
        if (XSRC == X_ATTN)
          v[u] = base == 0 && u == 0 ? attn_finish(p, af) : attn_chunk(p, m, kbase + 8 * c);
        else if (XSRC == X_SILU)
          v[u] = base == 0 && u < SF ? silu_finish(p, sf[u]) : silu_chunk(p, m, kbase + 8 * c);
        else if (XSRC == X_NORM)
          v[u] = base == 0
                     ? norm8(xv[u], nwv[u], sInv[m])
                     : norm8(*reinterpret_cast<const uint4*>(p.nh + (int64_t)m * p.ldnh + kbase +
                                                             8 * c),
                             *reinterpret_cast<const uint4*>(p.nw + kbase + 8 * c), sInv[m]);
        else
          v[u] = base == 0 ? xv[u]
                           : *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + kbase +
                                                             8 * c);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (base + u * NT >= total) break;
      const int i = CLAMP ? min(base + u * NT + tid, total - 1) : base + u * NT + tid;
      if (CLAMP || i < total) {
        int m, c;
        chunk_mc(i, m, c);
        *reinterpret_cast<uint4*>(xs + xs_offset(m, c)) = deinterleave8(v[u]);
      }
    }
  }
  __syncthreads();
  if (!FIN && tile >= p.ntiles) return;

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // lane (ln, lg) multiplies row 16 mt + ln over K values 64 lg + 8 j of each
  // k-step: chunk 8 lg + j, then + 32 per k-step (xstep)
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = xs + xs_offset(min(mt * 16 + ln, p.M - 1), 8 * lg);
  auto xstep = [&](int i, int j) __attribute__((always_inline)) {
    return CM ? (32 * i + j) * XROWS * 8 : i * KSTEP + 8 * j;
  };

  if (wtile) {
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      if (i >= nk) break;
      const Lut t = make_lut(code, av[i]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint4 bw = decode8(word(wv[2 * i + (j >> 2)], j & 3), t);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = mfma16x16x32(
              *reinterpret_cast<const uint4*>(xrow[mt] + xstep(i, j)), bw, acc[mt]);
      }
    }
    // FIN: wave 0's LoRA-A tile before any store (the wait for the A rows
    // would otherwise also wait for the stores to be acknowledged)
    f32x4_t lacc = {0.f, 0.f, 0.f, 0.f};
    if (FIN && lwave && p.r > 0) {
      const bool r_ok = ln < p.r;
#pragma unroll
      for (int i = 0; i < KPW; ++i) {
        if (i >= nk) break;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          lacc = mfma16x16x32(*reinterpret_cast<const uint4*>(xrow[0] + xstep(i, j)),
                              deinterleave8(r_ok ? a8f[8 * i + j] : make_uint4(0, 0, 0, 0)),
                              lacc);
      }
    }
    float* out = p.part + (int64_t)slice * p.Mp * p.N + n_row;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mt * 16 + 4 * lg + q;
        if (m < p.M) out[(int64_t)m * p.N] = acc[mt][q];
      }
    if (FIN && lwave && p.r > 0) {
      float* tout = p.fin_tpart + ((int64_t)blockIdx.x * gridDim.y + slice) * p.M * 16 + ln;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 4 * lg + q;
        if (m < p.M) tout[m * 16] = lacc[q];
      }
    }
  }
  if (!FIN && !wtile) {
    // LoRA-A tile of segment seg: lane n = rank index, A is read as bf16.
    const int seg = tile - p.NT;
    const bool r_ok = ln < p.r;
    const uint16_t* arow = sel_seg(p.la, seg) + (int64_t)(r_ok ? ln : 0) * p.K + kbase + 64 * lg;
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      if (i >= nk) break;
      uint4 a8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        a8[j] = r_ok ? *reinterpret_cast<const uint4*>(arow + i * KSTEP + 8 * j)
                     : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint4 bv = deinterleave8(a8[j]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = mfma16x16x32(
              *reinterpret_cast<const uint4*>(xrow[mt] + xstep(i, j)), bv, acc[mt]);
      }
    }
    float* out = p.tpart + ((int64_t)slice * p.nseg + seg) * p.Mp * 16 + ln;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mt * 16 + 4 * lg + q;
        if (m < p.M) out[m * 16] = acc[mt][q];
      }
  }
  if (FIN) {
    // Arrival: this workgroup's partials are in the XCD's L2 once its stores
    // are acknowledged (the vector L1 writes through); the group's counter is
    // an L2 atomic.  The last of the S slices resets the counter, drops its
    // L1 lines (a CU keeps no line of another workgroup's partials from this
    // kernel, but the invalidate costs nothing) and finishes the group.  Every
    // workgroup of a group has the same linear id modulo 8 (gridDim.x is a
    // multiple of 8), so the group runs on one XCD and shares one L2;
    // xcd_arrive checks that and flags a group that did not (fin_err).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int s_last;
    if (tid == 0)
      s_last = xcd_arrive(p.fin_cnt + (int64_t)blockIdx.x * FIN_CNT_STRIDE, (int)gridDim.y,
                          p.fin_err);
    __syncthreads();
    if (!s_last) return;
    asm volatile("buffer_inv sc0" ::: "memory");
    fin_group<WPG>(p, blockIdx.x, fpre);
  }
}

// y[m, n] from partial sums: a thread finishes four columns of row m.
__global__ void __launch_bounds__(256) nf4_finish(LinParts o, uint16_t* __restrict__ y,
                                                  int64_t ldy) {
  __shared__ float ts[MAXSEG * 16];
  const int m = blockIdx.y;
  const int n = (blockIdx.x * 256 + threadIdx.x) * 4;
  // this thread's partial sums go out before the LoRA t barrier, so the
  // finish is one memory round trip
  Fetch4<> f;
  if (n < o.N) lin_fetch4(o, m, n, f);
  lin_load_t(o, m, ts);
  __syncthreads();
  if (n >= o.N) return;
  float v[4];
  lin_finish4(o, ts, f, v);
  uint16_t* yr = y + (int64_t)m * ldy + n;
#pragma unroll
  for (int c = 0; c < 4; ++c) yr[c] = f2bf(v[c]);
}

struct PartPlan {
  int MT, NT, ntiles, kpw, S, xstride;
  int mchunk;  // rows per launch: M, or a multiple of 16 when x of M rows overflows LDS
  bool ok;     // false: no (k-steps, row chunk) fits both the slice cap and LDS
  size_t lds, part_bytes, tpart_bytes;
};

bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

// Shape-level support of the split-K path (alignment is checked per call).
PartPlan plan_part(int M, int N, int K, int r, int nseg);

bool part_shape_ok(int M, int N, int K, int r, int nseg, int blocksize, const int* seg_end) {
  if (!(M >= 1 && M <= 64 && N > 0 && N % 16 == 0 && K > 0 && K % KSTEP == 0)) return false;
  if (K > MAX_SLICES * KPW_MAX * KSTEP) return false;  // K <= 40960
  if (!(r >= 0 && r <= 16 && nseg >= 1 && nseg <= MAXSEG)) return false;
  if (!pow2(blocksize) || blocksize < 64) return false;
  for (int s = 0; seg_end && s < nseg; ++s)
    if (seg_end[s] % 16 != 0) return false;
  return plan_part(M, N, K, r, nseg).ok;
}

// LDS bytes of an x slice of kpw k-steps for a launch of `rows` rows:
// row-major with 8 padding columns, or chunk-major over the row tile count
// (xs_chunk_major: 5 k-steps of more than 16 rows, which fit 160 KiB only
// without padding; the row-major staging loads are better coalesced).
size_t xs_bytes(int rows, int kpw) {
  int mt = (rows + 15) / 16;
  if (mt == 3) mt = 4;
  return xs_chunk_major(mt, kpw) ? (size_t)mt * 16 * kpw * KSTEP * 2
                                 : (size_t)rows * (kpw * KSTEP + 8) * 2;
}

PartPlan plan_part(int M, int N, int K, int r, int nseg) {
  PartPlan p{};
  p.MT = (M + 15) / 16;
  if (p.MT == 3) p.MT = 4;  // launched as the MT = 4 kernel
  const int KS = K / KSTEP;
  p.NT = N / 16;
  p.ntiles = p.NT + (r > 0 ? nseg : 0);
  // Long K (down_proj, K = 8960) at decode batches: fewer, longer K slices
  // measured faster (fewer partial sums to write and for the consumer to read
  // back).  Wider batches keep the full target: their x slices take 16-wave
  // workgroups, so the halved target left most CUs idle (config 4's down_proj
  // at 32 rows: 9 slices x 8 groups = 72 workgroups; 18 slices of 2 k-steps on
  // 8-wave workgroups give 288: 5861 -> 6517 tok/s).
  const int target = K >= 4096 && M <= 16 ? g_target_waves / 2 : g_target_waves;
  const int s_target = (target + p.ntiles - 1) / p.ntiles;
  int kpw = (KS + s_target - 1) / s_target;
  // More than 16 rows may take 5 k-steps per slice, staged chunk-major
  // (xs_chunk_major), which needs no padding columns, so 64 rows fit LDS
  // exactly (Qwen2-7B's down_proj at 64 rows: 15 K slices x 16 tile groups =
  // 240 workgroups, one per CU, where 4 k-steps gave 19 x 16 = 304 and a
  // second round on 48 CUs).
  static const int choices_n[] = {1, 2, 3, 4, 6, 8};
  static const int choices_w[] = {1, 2, 3, 4, 5, 6, 8};
  const bool wide = p.MT > 1;
  const int* choices = wide ? choices_w : choices_n;
  const int nch = wide ? 7 : 6;
  int pick = KPW_MAX;
  for (int i = 0; i < nch; ++i)
    if (choices[i] >= kpw) {
      pick = choices[i];
      break;
    }
  const size_t lds_cap = M > 16 ? PART_LDS_BIG : PART_LDS_MAX;
  while (pick > 1 && xs_bytes(M, pick) > lds_cap) {
    int lower = 1;
    for (int i = 0; i < nch; ++i)
      if (choices[i] < pick) lower = choices[i];
    pick = lower;
  }
  // consumers read at most MAX_SLICES partial sums per output
  while ((KS + pick - 1) / pick > MAX_SLICES && pick < KPW_MAX) {
    for (int i = 0; i < nch; ++i)
      if (choices[i] > pick) {
        pick = choices[i];
        break;
      }
  }
  p.kpw = pick;
  p.S = (KS + pick - 1) / pick;
  p.xstride = pick * KSTEP + 8;
  // Wide batches of very long K (> 20 slices of 5 k-steps) stage more x than
  // LDS holds: their rows are launched in chunks of 32 or 16 rows, each writing
  // its rows of the same partial-sum layout.
  p.mchunk = M;
  if (xs_bytes(M, pick) > lds_cap) p.mchunk = xs_bytes(32, pick) <= lds_cap ? 32 : 16;
  p.ok = xs_bytes(std::min(M, p.mchunk), pick) <= lds_cap && p.S <= MAX_SLICES;
  if (p.mchunk < M) p.MT = p.mchunk / 16;
  p.lds = xs_bytes(std::min(M, p.mchunk), pick);
  p.part_bytes = (size_t)p.S * M * N * 4;
  p.tpart_bytes = r > 0 ? (size_t)p.S * nseg * M * 16 * 4 : 0;
  return p;
}

// Workgroups are dispatched round-robin over the 8 XCDs by linear id
// x + y * gridDim.x.  With gridDim.x a multiple of 8, every K slice of a tile
// group runs on the same XCD, so the absmax lines that the slices of a row
// share are fetched from HBM into one L2 only.
constexpr int NUM_XCD = 8;


template <int MT, int KPW, int XSRC, bool FIN = false>
int launch_part_k(const PartArgs& a, const PartPlan& pl, const dim3& grid, const dim3& block,
                  hipStream_t st) {
  if (pl.lds > (size_t)PART_LDS_MAX)
    if (int rc = allow_dynamic_lds<nf4_part_mfma<MT, KPW, XSRC, FIN>, PART_LDS_BIG>()) return rc;
  nf4_part_mfma<MT, KPW, XSRC, FIN><<<grid, block, pl.lds, st>>>(a);
  return launch_check("nf4_part_mfma");
}

template <int MT, int XSRC>
int launch_part(const PartArgs& a, const PartPlan& pl, hipStream_t st) {
  constexpr int WPG = waves_per_group(XSRC);
  const int groups = (int)cdiv(pl.ntiles, WPG);
  const dim3 grid((unsigned)(cdiv(groups, NUM_XCD) * NUM_XCD), (unsigned)pl.S), block(64 * WPG);
  switch (pl.kpw) {
    case 1: return launch_part_k<MT, 1, XSRC>(a, pl, grid, block, st);
    case 2: return launch_part_k<MT, 2, XSRC>(a, pl, grid, block, st);
    case 3: return launch_part_k<MT, 3, XSRC>(a, pl, grid, block, st);
    case 4: return launch_part_k<MT, 4, XSRC>(a, pl, grid, block, st);
    case 5:
      if constexpr (MT > 1) return launch_part_k<MT, 5, XSRC>(a, pl, grid, block, st);
      return einval("5 k-steps per K slice take more than 16 rows");
    case 6: return launch_part_k<MT, 6, XSRC>(a, pl, grid, block, st);
    default: return launch_part_k<MT, 8, XSRC>(a, pl, grid, block, st);
  }
}

// FIN launch: one workgroup per (tile group, K slice), the LoRA-A tile of
// every workgroup on its wave 0; a.ntiles = NT (no LoRA tiles).  gridDim.x is a multiple of 8, so
// the K slices of a tile group share an XCD (the finish relies on it).
template <int XSRC>
int launch_part_fin(const PartArgs& a, const PartPlan& pl, hipStream_t st) {
  constexpr int WPG = waves_per_group(XSRC);
  const int groups = pl.NT / WPG;
  const dim3 grid((unsigned)(cdiv(groups, NUM_XCD) * NUM_XCD), (unsigned)pl.S), block(64 * WPG);
  switch (pl.kpw) {
    case 1: return launch_part_k<1, 1, XSRC, true>(a, pl, grid, block, st);
    case 2: return launch_part_k<1, 2, XSRC, true>(a, pl, grid, block, st);
    default: return einval("in-kernel finish: at most 2 k-steps per K slice");
  }
}

// Where a FIN launch writes (the residual add after the linear).
struct FinTarget {
  float* tpart = nullptr;  // [groups][S][M][16]
  int* cnt = nullptr;      // [groups * FIN_CNT_STRIDE]
  int* err = nullptr;      // XCD check flag
  const uint16_t* res = nullptr;
  uint16_t* h = nullptr;
  int64_t ld = 0;
  float* ss = nullptr;     // [M][groups]
};

// Attention-output source of x (o_proj of the decode step), or all-null.
struct AttnSource {
  const float* o = nullptr;
  const float* ml = nullptr;
  const int32_t* len = nullptr;
  int S = 0, bps = 0, Hq = 0, cap = 0;
};

// gate|up partial-sum source of x (down_proj of the decode step), or null.
struct SiluSource {
  const float* part = nullptr;
  int S = 0;
};

// RMSNorm source of x (q|k|v of the decode step after nf4_fold_residual), or null.
struct NormSource {
  const uint16_t* h = nullptr;
  int64_t ldh = 0;
  const float* sumsq = nullptr;
  int groups = 0;
  const uint16_t* weight = nullptr;
  float eps = 0.f;
};

int run_partials(const uint16_t* x, int64_t ldx, const uint8_t* w, const float* absmax,
                 const float* code16, int blocksize, const uint16_t* const* la,
                 const grpo_linear_parts_t& h, hipStream_t st, const AttnSource* att = nullptr,
                 const SiluSource* silu = nullptr, const NormSource* nrm = nullptr,
                 const FinTarget* fin = nullptr) {
  const bool xsrc = att || silu || nrm;
  if (!part_shape_ok(h.M, h.N, h.K, h.r, h.nseg, blocksize, h.seg_end)) {
    set_error("shape not supported by the split-K NF4 linear");
    return GRPO_EUNSUPPORTED;
  }
  const PartPlan pl = plan_part(h.M, h.N, h.K, h.r, h.nseg);
  if (!pl.ok) {
    set_error("shape not supported by the split-K NF4 linear");
    return GRPO_EUNSUPPORTED;
  }
  if (xsrc && pl.mchunk < h.M) {
    set_error("x staged from attention or gate|up partials must fit LDS in one launch");
    return GRPO_EUNSUPPORTED;
  }
  if (h.splits != pl.S) return einval("parts.splits differs from grpo_nf4_linear_plan");
  if ((!x && !xsrc) || !w || !absmax || !code16 || !h.part) return einval("null pointer");
  if (h.r > 0 && !h.tpart) return einval("r > 0 needs tpart");
  if (!xsrc && (ldx < h.K || ldx % 8 != 0)) return einval("ldx must be >= K and a multiple of 8");
  if ((!xsrc && !aligned16(x)) || !aligned16(w)) return einval("x and w must be 16-byte aligned");
  PartArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.w = w;
  a.absmax = absmax;
  a.code16 = code16;
  a.bs_shift = __builtin_ctz((unsigned)blocksize);
  for (int s = 0; s < h.nseg; ++s) {
    a.la[s] = h.r > 0 ? la[s] : nullptr;
    if (h.r > 0 && (!a.la[s] || !aligned16(a.la[s])))
      return einval("lora_a must be non-null and 16-byte aligned");
  }
  a.part = h.part;
  a.tpart = h.tpart;
  a.M = h.M;
  a.Mp = h.M;
  a.N = h.N;
  a.K = h.K;
  a.NT = pl.NT;
  a.ntiles = pl.ntiles;
  a.nseg = h.nseg;
  a.r = h.r;
  a.xstride = pl.xstride;
  if (fin) {
    // in-kernel finish: <= 16 rows, one LoRA segment, whole tile groups
    constexpr int WPG = waves_per_group(X_ATTN);
    if (!att || pl.MT != 1 || h.nseg != 1 || pl.NT % WPG != 0 || pl.S > FIN_MAX_SLICES ||
        pl.kpw > 2) {
      set_error("shape not supported by the in-kernel linear finish");
      return GRPO_EUNSUPPORTED;
    }
    const int groups = pl.NT / WPG;
    if (!fin->cnt || !fin->err || !fin->res || !fin->h || !fin->ss || (h.r > 0 && !fin->tpart))
      return einval("null pointer");
    if (fin->ld < h.N || fin->ld % 4 || !aligned8(fin->res) || !aligned8(fin->h))
      return einval("residual/h: ld must be >= N and a multiple of 4, rows 8-byte aligned");
    if (h.bias[0] && !aligned8(h.bias[0])) return einval("bias must be 8-byte aligned");
    if (h.r > 0 && !h.lora_b[0]) return einval("r > 0 needs lora_b");
    a.ntiles = pl.NT;
    a.fin_tpart = fin->tpart;
    a.fin_cnt = fin->cnt;
    a.fin_err = fin->err;
    a.fin_res = fin->res;
    a.fin_h = fin->h;
    a.fin_ld = fin->ld;
    a.fin_ss = fin->ss;
    a.fin_bias = static_cast<const uint16_t*>(h.bias[0]);
    a.fin_lb = static_cast<const uint16_t*>(h.lora_b[0]);
    a.fin_scaling = h.scaling;
    a.fin_lb_vec = h.r == 16 && aligned16(h.lora_b[0]);
    (void)groups;
  }
  if (att) {
    a.att_o = att->o;
    a.att_ml = att->ml;
    a.att_len = att->len;
    a.att_S = att->S;
    a.att_bps = att->bps;
    a.att_Hq = att->Hq;
    a.att_cap = att->cap;
    if (fin) return launch_part_fin<X_ATTN>(a, pl, st);
    switch (pl.MT) {
      case 1: return launch_part<1, X_ATTN>(a, pl, st);
      case 2: return launch_part<2, X_ATTN>(a, pl, st);
      default: return launch_part<4, X_ATTN>(a, pl, st);
    }
  }
  if (nrm) {
    if (pl.MT != 1) {
      set_error("the RMSNorm x source takes at most 16 rows");
      return GRPO_EUNSUPPORTED;
    }
    a.nh = nrm->h;
    a.ldnh = nrm->ldh;
    a.nss = nrm->sumsq;
    a.nG = nrm->groups;
    a.nw = nrm->weight;
    a.neps = nrm->eps;
    return launch_part<1, X_NORM>(a, pl, st);
  }
  if (silu) {
    a.gu_part = silu->part;
    a.gu_S = silu->S;
    switch (pl.MT) {
      case 1: return launch_part<1, X_SILU>(a, pl, st);
      case 2: return launch_part<2, X_SILU>(a, pl, st);
      default: return launch_part<4, X_SILU>(a, pl, st);
    }
  }
  for (int m0 = 0; m0 < h.M; m0 += pl.mchunk) {
    PartArgs c = a;
    c.M = std::min(pl.mchunk, h.M - m0);
    c.x = x + (int64_t)m0 * ldx;
    c.part = h.part + (int64_t)m0 * h.N;
    c.tpart = h.tpart ? h.tpart + (int64_t)m0 * 16 : nullptr;
    int rc;
    const int64_t wgs16 = cdiv(cdiv(pl.ntiles, 16), NUM_XCD) * NUM_XCD * pl.S;
    if (pl.lds > (size_t)PART_LDS_MAX && wgs16 <= 128 && 2 * pl.lds <= (size_t)PART_LDS_BIG) {
      switch (pl.MT) {
        case 1: rc = launch_part<1, X_WIDE8>(c, pl, st); break;
        case 2: rc = launch_part<2, X_WIDE8>(c, pl, st); break;
        default: rc = launch_part<4, X_WIDE8>(c, pl, st); break;
      }
    } else if (pl.lds > (size_t)PART_LDS_MAX) {
      switch (pl.MT) {
        case 1: rc = launch_part<1, X_WIDE>(c, pl, st); break;
        case 2: rc = launch_part<2, X_WIDE>(c, pl, st); break;
        default: rc = launch_part<4, X_WIDE>(c, pl, st); break;
      }
    } else {
      switch (pl.MT) {
        case 1: rc = launch_part<1, X_BF16>(c, pl, st); break;
        case 2: rc = launch_part<2, X_BF16>(c, pl, st); break;
        default: rc = launch_part<4, X_BF16>(c, pl, st); break;
      }
    }
    if (rc) return rc;
  }
  return GRPO_OK;
}

int run_finish(const grpo_linear_parts_t* h, uint16_t* y, int64_t ldy, hipStream_t st) {
  LinParts o;
  if (int rc = make_parts(h, &o)) return rc;
  if (!y) return einval("null y");
  if (ldy < o.N) return einval("ldy smaller than N");
  nf4_finish<<<dim3((unsigned)cdiv(o.N / 4, 256), (unsigned)o.M), 256, 0, st>>>(o, y, ldy);
  return launch_check("nf4_finish");
}

// ------------------------------------------ gate|up with SiLU * up --
//
// act[m, j] = bf16(bf16(silu(g)) * u) with g = bf16(x . Wg[j, :]) and
// u = bf16(x . Wu[j, :]): the MLP's gate and up projections of the stacked
// [2I, K] NF4 weight (rows 0..I-1 gate, I..2I-1 up; bnb Linear4bit, no LoRA,
// no bias) followed by fused_ops.py:79-112.  One workgroup per 16 columns j
// (gate tile t and up tile t): waves 0..S-1 take K slices 0..S-1 of the gate
// tile, waves S..2S-1 those of the up tile; the slices are summed through LDS
// in slice order (the float32 order of the split-K consumers), so down_proj
// reads a finished bf16 input instead of float32 partial sums.

struct GuArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  const float* absmax;
  const float* code16;
  int bs_shift;
  uint16_t* act;
  int64_t lda;
  int M, I, K;
  int act_tiles;  // write act in the fold tile layout (fold_tile_index; M <= 8)
  int act_vec;    // act 16-byte aligned and lda % 8 == 0: 8 columns per 16-byte store
  // x = RMSNorm(h) from per-group sums of squares, when nh is set (units kernel, M <= 8)
  const uint16_t* nh;
  int64_t ldnh;
  const float* nss;  // [M][nG], nG % 4 == 0, nG <= GU_NORM_MAX_GROUPS, rows 16-byte aligned
  int nG;
  const uint16_t* nw;
  float neps;
};
constexpr int GU_NORM_MAX_GROUPS = 256;  // sums of squares per row (8 lanes x 8 float4)

// Position of element e (0..7) of an 8-element chunk in the decode8 order
// [0, 2, 4, 6, 1, 3, 5, 7].
__host__ __device__ constexpr int il_pos(int e) { return (e >> 1) + 4 * (e & 1); }

// Fold tile layout of an activation [M <= 8][K] read by nf4_fold_residual:
// for item i = k / 512 and MFMA j = (k / 8) % 8, the 64 lanes' 16-byte A
// operands are one contiguous 1 KiB block, lane = m + 8 * ((k / 256) % 2) +
// 16 * ((k / 64) % 4), its 8 elements in the decode8 order.  Rows >= M and
// columns >= K are never written (the buffer starts zero-filled).
__host__ __device__ constexpr int64_t fold_tile_index(int m, int k) {
  return ((int64_t)((k >> 9) * 8 + ((k >> 3) & 7)) * 64 + m + 8 * ((k >> 8) & 1) +
          16 * ((k >> 6) & 3)) * 8 + il_pos(k & 7);
}

__device__ __forceinline__ void store_act(const GuArgs& p, int m, int col, float v) {
  if (p.act_tiles)
    p.act[fold_tile_index(m, col)] = f2bf(v);
  else
    p.act[(int64_t)m * p.lda + col] = f2bf(v);
}

constexpr int GU_XU = 8;  // x chunks per thread loaded ahead of the weights

// S (slices per tile) is a template parameter: with the thread count known at
// compile time the x chunks stay in registers (a runtime count sent them to
// scratch memory).
template <int KPW, int S>
__global__ void __launch_bounds__(128 * S) nf4_gate_up_silu(GuArgs p) {
  constexpr int MT = 1;
  extern __shared__ __align__(16) uint16_t xs[];  // [M][K + 8] (decode8 order), then sums
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  constexpr int NTH = 128 * S;
  const int t = blockIdx.x;
  const bool up = wave >= S;
  const int slice = up ? wave - S : wave;
  const int KS = p.K / KSTEP;
  const int ks0 = slice * KPW;
  const int nk = min(KPW, KS - ks0);  // >= 1: S = ceil(KS / KPW)
  const int n_row = (up ? p.I : 0) + t * 16 + ln;
  const int xstride = p.K + 8;
  float* red = reinterpret_cast<float*>(xs + p.M * xstride);  // [2S][M][16]
  static_assert(MT == 1, "M <= 16");

  // Load order as in nf4_part_mfma: codebook (scalar loads), x (whole K, the
  // first GU_XU chunks per thread; whole entries past the end skipped, a
  // partial one clamped), then this wave's weights, unconditional.
  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];
  const int chunks = p.K / 8, total = p.M * chunks;
  uint4 xv[GU_XU];
#pragma unroll
  for (int u = 0; u < GU_XU; ++u) {
    if (u * NTH >= total) break;
    const int i = min(u * NTH + tid, total - 1);
    const int m = i / chunks, c = i - m * chunks;
    xv[u] = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + 8 * c);
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 wv[2 * KPW];
  float av[KPW];
  {
    const uint8_t* wrow = p.w + (int64_t)n_row * (p.K / 2);
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kc = (ks0 + min(i, nk - 1)) * KSTEP + 64 * lg;
      const uint4* wp = reinterpret_cast<const uint4*>(wrow + kc / 2);
      wv[2 * i] = load_w<true>(wp);
      wv[2 * i + 1] = load_w<true>(wp + 1);
      av[i] = p.absmax[((int64_t)n_row * p.K + kc) >> p.bs_shift];
    }
  }
  for (int base = 0; base < total; base += GU_XU * NTH) {
#pragma unroll
    for (int u = 0; u < GU_XU; ++u) {
      if (base + u * NTH >= total) break;
      const int i = min(base + u * NTH + tid, total - 1);
      const int m = i / chunks, c = i - m * chunks;
      const uint4 v = base == 0 ? xv[u]
                                : *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + 8 * c);
      *reinterpret_cast<uint4*>(xs + m * xstride + 8 * c) = deinterleave8(v);
    }
  }
  __syncthreads();

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xrow[mt] = xs + min(mt * 16 + ln, p.M - 1) * xstride + ks0 * KSTEP + 64 * lg;
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    if (i >= nk) break;
    const Lut lt = make_lut(code, av[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint4 bw = decode8(word(wv[2 * i + (j >> 2)], j & 3), lt);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = mfma16x16x32(*reinterpret_cast<const uint4*>(xrow[mt] + i * KSTEP + 8 * j), bw,
                               acc[mt]);
    }
  }
  // lane (n = ln, group lg) holds D[m = mt*16 + 4*lg + q][n]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = mt * 16 + 4 * lg + q;
      if (m < p.M) red[(wave * p.M + m) * 16 + ln] = acc[mt][q];
    }
  __syncthreads();
  for (int i = tid; i < p.M * 16; i += NTH) {
    const int m = i >> 4, n = i & 15;
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      g += red[(s * p.M + m) * 16 + n];
      u += red[((S + s) * p.M + m) * 16 + n];
    }
    const float gv = round_bf(g);
    const float o = round_bf(gv * (1.f / (1.f + expf(-gv)))) * round_bf(u);
    store_act(p, m, t * 16 + n, o);
  }
}

// gate|up + SiLU in units of 8 output columns (4 for the decode step's folded
// units, FOLD below) over a grid of at most one workgroup per CU.  Unit u
// covers act columns 8u .. 8u+7: the MFMA tile's 16
// B-columns are gate rows 8u .. 8u+7 (lanes n < 8) and up rows I+8u .. I+8u+7
// (lanes n >= 8), so the SiLU pairs a tile's columns n and n + 8.  Workgroup
// g takes units g, g + G, g + 2G, ...; its W waves take the (unit, k-step)
// items of those units round-robin, each item one k-step of 256 on one wave.
// Against one workgroup per 16 columns (nf4_gate_up_silu) this stages x into
// LDS once per CU instead of once per workgroup -- x was half the bytes each
// CU moved -- and balances the decode at the grain of one k-step (a CU's share
// of 8-column units differs by at most one unit, not by one 16-column pair).
// Item partial tiles meet in LDS and are summed in k-step order.
constexpr int GUU_XU = 6;  // x chunks per thread loaded before the weights
// Items whose weights are in flight ahead of the one decoded: one (config 3
// 3670 -> 3686 tok/s and config 4 9214 -> 9284 against two; three gave 3618).
#ifndef GRPO_GUU_LA
#define GRPO_GUU_LA 1
#endif
constexpr int GUU_LA = GRPO_GUU_LA;

// MT row tiles of 16 (MT = 2: 17..32 rows, whose x of K <= 1536 still fits
// LDS whole with the item tiles: config 4's G = 32).  ROWS (M <= 8, the
// decode step's rows): wave w stages columns [w c, w c + c) of every row
// (c = ceil(K / 8 / W) chunks of 8), lane l row l / 8 and chunks l % 8,
// l % 8 + 8, ... of the range -- no row/column division per chunk, and each
// RMSNorm weight chunk is loaded by one wave (8 lanes, one address) instead
// of every wave.  Otherwise chunk i of the M x K/8 chunks goes to thread
// i mod (64 W).
template <int W, int IPW, bool NORM, int MT = 1, bool ROWS = false>
__global__ void __launch_bounds__(64 * W) nf4_gate_up_units(GuArgs p) {
  static_assert(!NORM || MT == 1, "the RMSNorm source takes at most 8 rows");
  static_assert(!ROWS || (MT == 1 && W >= 8), "8 lanes per row, rows <= 8");
  touch_kernargs<sizeof(GuArgs)>();
  constexpr int NTH = 64 * W;
  extern __shared__ __align__(16) uint16_t xs[];  // [M][K + 8] (decode8 order), then tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int G = gridDim.x, g0 = blockIdx.x;
  const int KS = p.K / KSTEP;
  // FOLD (with ROWS; K / 256 even): units of 4 gate + 4 up columns, an item
  // two k-steps of a unit: B columns n < 8 take the first k-step of the pair,
  // columns n >= 8 the same 8 weight rows at the second, and A rows m >= 8
  // hold x row m - 8 at the second (D[m][n] + D[m + 8][n + 8] is the item's
  // product).  Twice the units per workgroup at the same item size: a
  // workgroup's share of the 6720 config-3 items is 24 or 27 (at most 7 per
  // SIMD) instead of 24 or 30 (8 per SIMD).
  constexpr bool FOLD = ROWS;
  constexpr int UC = FOLD ? 4 : 8;     // act columns per unit
  const int KI = FOLD ? KS / 2 : KS;  // items per unit
  constexpr int KI_STEP = FOLD ? 2 * KSTEP : KSTEP;
  const int U = p.I / UC;
  const int nu = (U - g0 + G - 1) / G;  // >= 1: the grid has at most U workgroups
  const int nitems = nu * KI;
  const int xstride = p.K + 8;
  // item tiles [nitems][Mp / 4][16][4] (Mp = M rounded up to 4): lane (n, lg)
  // stores its rows 4 lg .. 4 lg + 3 of column n as one 16-byte write
  // (FOLD: [nitems][2 halves][8 columns][8 rows], 512 bytes)
  const int mq = (p.M + 3) >> 2;
  float* red = reinterpret_cast<float*>(xs + p.M * xstride);
  // row of unit u for this lane's column: UC u + rsel
  const int rsel = FOLD ? ((ln & 7) < 4 ? (ln & 7) : p.I + (ln & 7) - 4)
                        : (ln < 8 ? ln : p.I + ln - 8);
  // Element e = row * K + k of item (unit i, k-step k) splits into a uniform
  // part (UC (g0 + i G) K + KI_STEP k) and this lane's constant part
  // (rsel K + 64 lg, + 256 for FOLD's columns n >= 8): the weight bytes are
  // the uniform base plus a 32-bit lane offset (no per-item vector address
  // arithmetic), and so is the absmax index when the blocksize divides 256
  // (then it divides both parts).
  const uint32_t lane_e = (uint32_t)rsel * (uint32_t)p.K + 64u * lg + (FOLD && ln >= 8 ? KSTEP : 0);
  const bool sep = p.bs_shift <= 8;

  // x first (GUU_XU chunks per thread: clamped, or for ROWS only the lane's
  // own), then the weights of this wave's first item; its next GUU_LA - 1
  // items after the staging (a longer burst at entry delays the x loads the
  // staging waits for); every item then issues the loads of the item GUU_LA
  // ahead before it waits for its own.  The weight loads are unconditional
  // (an item past the workgroup's last reads the codebook), so each wait is
  // exact: staging waits only for x, an item only for its own weights, and
  // the decode of one item overlaps the loads of the next ones.  The codebook (first needed by the first item) is
  // loaded after the first item's weights: a scalar load issued earlier makes
  // the waits for the kernel arguments that address the weights wait for it.
  const int chunks = p.K / 8, total = p.M * chunks;
  // RMSNorm source (NORM): every wave holds the group sums of squares of all
  // rows, lane l those of row l / 8 (four groups per float4 load: float4s
  // l % 8, l % 8 + 8, ...), loaded first
  constexpr int NSS = GU_NORM_MAX_GROUPS / 32;
  float4 ssv[NSS];
  const uint16_t* xsrc = NORM ? p.nh : p.x;
  const int64_t xld = NORM ? p.ldnh : p.ldx;
  const int sub = lane & 7, lrow = min(lane >> 3, p.M - 1);
  if (NORM) {
    const float4* ssr = reinterpret_cast<const float4*>(p.nss + (int64_t)lrow * p.nG);
#pragma unroll
    for (int q = 0; q < NSS; ++q)
      if (ROWS) {
        // conditional: no loads issued before these, so no wait depends on them
        if (sub + 8 * q < (p.nG >> 2)) ssv[q] = ssr[sub + 8 * q];
      } else {
        ssv[q] = ssr[min(sub + 8 * q, (p.nG >> 2) - 1)];
      }
  }
  // ROWS: this wave's chunk range [c_lo, c_hi), lane l chunks c_lo + l % 8 + 8 u
  const int cpw = (chunks + W - 1) / W;
  const int c_lo = min(wave * cpw, chunks), c_hi = min(c_lo + cpw, chunks);
  uint4 xv[GUU_XU], nwv[GUU_XU];
#pragma unroll
  for (int u = 0; u < GUU_XU; ++u) {
    if (ROWS) {
      // conditional: the loads after these (the weights) are not, so the
      // staging's wait for them is exact
      const int c = c_lo + sub + 8 * u;
      if (c < c_hi) {
        xv[u] = *reinterpret_cast<const uint4*>(xsrc + (int64_t)lrow * xld + 8 * c);
        if (NORM) nwv[u] = *reinterpret_cast<const uint4*>(p.nw + 8 * c);
      }
    } else {
      const int i = min(u * NTH + tid, total - 1);
      const int m = i / chunks, c = i - m * chunks;
      xv[u] = *reinterpret_cast<const uint4*>(xsrc + (int64_t)m * xld + 8 * c);
      if (NORM) nwv[u] = *reinterpret_cast<const uint4*>(p.nw + 8 * c);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  uint4 wv[2 * IPW];
  float av[IPW];
  // (unit slot, k-step) of this wave's item t = wave + W t, advanced without
  // divisions (uniform); items past the last re-read the last one
  const int qlast = nitems - 1;
  int ci = wave / KI, ck = wave - ci * KI, cq = wave;  // item of the next load_item
  auto load_item = [&](int t) __attribute__((always_inline)) {
    // An item past the workgroup's last (the look-ahead of a wave's last
    // item) loads the 64-byte codebook instead, an L2 hit: the epilogue
    // reuses those registers, so it waits for these loads.
    const bool past = cq > qlast;
    const uint32_t ue = (uint32_t)(UC * (g0 + ci * G)) * (uint32_t)p.K + (uint32_t)(ck * KI_STEP);
    const uint4* wp = past ? reinterpret_cast<const uint4*>(p.code16)
                           : reinterpret_cast<const uint4*>(p.w + (ue >> 1) + (lane_e >> 1));
    wv[2 * t] = load_w<true>(wp);
    wv[2 * t + 1] = load_w<true>(wp + 1);
    const float* ap = past ? p.code16
                    : sep  ? p.absmax + (ue >> p.bs_shift) + (lane_e >> p.bs_shift)
                           : p.absmax + ((ue + lane_e) >> p.bs_shift);
    av[t] = *ap;
    cq += W;
    ck += W;
    while (ck >= KI) {
      ck -= KI;
      ++ci;
    }
  };
  load_item(0);  // the look-ahead's other items after the staging
  __builtin_amdgcn_sched_barrier(0);
  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];
  // lane l: 1 / rms of row l / 8 (the row's sum over its 8 lanes by DPP)
  float inv_l = 0.f;
  if (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int q = 0; q < NSS; ++q)
      if (sub + 8 * q < (p.nG >> 2)) ss += (ssv[q].x + ssv[q].y) + (ssv[q].z + ssv[q].w);
    ss = sum8(ss);
    inv_l = 1.f / sqrtf(ss / (float)p.K + p.neps);
  }
  if (ROWS) {
    if ((lane >> 3) < p.M) {
      const int m = lane >> 3;
      for (int c0 = c_lo; c0 < c_hi; c0 += 8 * GUU_XU) {
#pragma unroll
        for (int u = 0; u < GUU_XU; ++u) {
          const int c = c0 + sub + 8 * u;
          if (c < c_hi) {
            uint4 v = c0 == c_lo ? xv[u]
                                 : *reinterpret_cast<const uint4*>(xsrc + (int64_t)m * xld + 8 * c);
            if (NORM)
              v = norm8(v, c0 == c_lo ? nwv[u] : *reinterpret_cast<const uint4*>(p.nw + 8 * c),
                        inv_l);
            *reinterpret_cast<uint4*>(xs + m * xstride + 8 * c) = deinterleave8(v);
          }
        }
      }
    }
  }
  for (int base = 0; !ROWS && base < total; base += GUU_XU * NTH) {
#pragma unroll
    for (int u = 0; u < GUU_XU; ++u) {
      if (base + u * NTH >= total) break;
      const int i = min(base + u * NTH + tid, total - 1);
      const int m = i / chunks, c = i - m * chunks;
      uint4 v = base == 0 ? xv[u]
                          : *reinterpret_cast<const uint4*>(xsrc + (int64_t)m * xld + 8 * c);
      if (NORM)
        v = norm8(v, base == 0 ? nwv[u] : *reinterpret_cast<const uint4*>(p.nw + 8 * c),
                  __shfl(inv_l, 8 * m));
      *reinterpret_cast<uint4*>(xs + m * xstride + 8 * c) = deinterleave8(v);
    }
  }
#pragma unroll
  for (int t = 1; t < GUU_LA && t < IPW; ++t) load_item(t);
  __syncthreads();

  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    xrow[mt] = FOLD ? xs + min(ln & 7, p.M - 1) * xstride + 64 * lg + (ln >= 8 ? KSTEP : 0)
                    : xs + min(16 * mt + ln, p.M - 1) * xstride + 64 * lg;
  const int my_items = (nitems - wave + W - 1) / W;  // items of this wave (may be 0)
#pragma unroll
  for (int t = 0; t < IPW; ++t) {
    if (t >= my_items) break;
    if (t + GUU_LA < IPW) load_item(t + GUU_LA);
    const int k = (wave + W * t) % KI;
    const Lut lt = make_lut(code, av[t]);
    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint4 bw = decode8(word(wv[2 * t + (j >> 2)], j & 3), lt);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = mfma16x16x32(*reinterpret_cast<const uint4*>(xrow[mt] + k * KI_STEP + 8 * j),
                               bw, acc[mt]);
    }
    // lane (n = ln, group lg) holds D[m = 16 mt + 4 lg + r][n]
    const int q = wave + W * t;
    if (FOLD) {
      // item tile [2 halves][8 columns][8 rows]: half h = n / 8 from the
      // lanes with rows 8 h .. 8 h + 7 (lg / 2 == h)
      if ((ln >> 3) == (lg >> 1))
        *reinterpret_cast<f32x4_t*>(red + q * 128 + (ln >> 3) * 64 + (ln & 7) * 8 + 4 * (lg & 1)) =
            acc[0];
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        if (4 * mt + lg < mq)
          *reinterpret_cast<f32x4_t*>(red + ((q * mq + 4 * mt + lg) * 16 + ln) * 4) = acc[mt];
    }
  }
  __syncthreads();
  // (unit, row, column) outputs, output i to thread i mod NTH: FOLD, i =
  // 32 un + 4 m + n (column n < 4 of the unit: gate n, up n + 4, each the sum
  // of the two halves of its items); otherwise i = (un M + m) 8 + n (gate n,
  // up n + 8).  The sums run over the unit's k-steps in order.
  const int nout = FOLD ? nu * 32 : nu * p.M * 8;
  for (int i = tid; i < nout; i += NTH) {
    int un, m, n;
    if (FOLD) {
      un = i >> 5;
      m = (i >> 2) & 7;
      n = i & 3;
      if (m >= p.M) continue;
    } else {
      un = i / (p.M * 8);
      const int rem = i - un * p.M * 8;
      m = rem >> 3;
      n = rem & 7;
    }
    float g = 0.f, u = 0.f;
    for (int k = 0; k < KI; ++k) {
      if (FOLD) {
        const float* tile = red + (un * KI + k) * 128 + m;
        g += tile[8 * n];
        g += tile[64 + 8 * n];
        u += tile[8 * (n + 4)];
        u += tile[64 + 8 * (n + 4)];
      } else {
        const float* tile = red + ((un * KI + k) * mq + (m >> 2)) * 64 + (m & 3);
        g += tile[4 * n];
        u += tile[4 * (n + 8)];
      }
    }
    const float gv = round_bf(g);
    const float o = round_bf(gv * (1.f / (1.f + expf(-gv)))) * round_bf(u);
    store_act(p, m, UC * (g0 + un * G) + n, o);
  }
}

// ------------------------------------ gate|up + SiLU for 17..64 rows --
//
// act[m, 8u + n] = bf16(bf16(silu(bf16(g))) * bf16(u)) for wide decode batches,
// g and u the gate and up products of x row m with W rows 8u + n and I + 8u + n
// (the units of nf4_gate_up_units: one 16-column MFMA tile pairs 8 gate and 8
// up rows).  x of 64 rows does not fit LDS whole, and split-K partial sums of
// [2I] columns (64 x 37,888 x 4 B per slice for the 7B MLP) plus a SiLU*mul
// launch cost more than the products, so every unit's accumulators stay in
// registers across K while x passes through LDS in chunks of 512 K values
// (two k-steps), double-buffered: the next chunk is loaded into registers
// while the current one is multiplied, and the next chunk's weights are in
// flight as well.  One workgroup per CU takes units g, g + G, ...; wave w
// takes k-step lane w & 1 (k-steps 2c + (w & 1) of chunk c) and the
// workgroup's units j = (w >> 1) + 4i, so one staged A operand (x rows, 32 K)
// feeds the MFMAs of up to GUW_UPW units.  At the end the two k-step lanes of
// a unit are summed through LDS (even k-steps + odd k-steps), the gate and up
// columns meet by a row rotation of 8 lanes, and lanes n < 8 write act.
constexpr int GUW_W = 8;                   // waves per workgroup
constexpr int GUW_S = 2;                   // k-step lanes
constexpr int GUW_GROUPS = GUW_W / GUW_S;  // unit groups
constexpr int GUW_UPW = 3;                 // most units per wave
constexpr int GUW_KC = GUW_S * KSTEP;      // K values of one staged chunk
constexpr int GUW_XSTRIDE = GUW_KC + 8;    // LDS row stride of a chunk (elements)
constexpr int GUW_EPS = 20;                // LDS row stride of the epilogue's sums (floats)

template <int MT>
__global__ void __launch_bounds__(64 * GUW_W) nf4_gate_up_wide(GuArgs p) {
  constexpr int NTH = 64 * GUW_W;
  constexpr int XU = 2 * MT;  // x chunks (16 B) per thread per staged chunk: 16*MT rows x 64
  extern __shared__ __align__(16) uint16_t xs[];  // 2 x [M][GUW_XSTRIDE], decode8 order
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int ksl = wave & (GUW_S - 1), grp = wave / GUW_S;
  const int G = gridDim.x, g0 = blockIdx.x;
  const int KS = p.K / KSTEP;
  const int NC = (KS + GUW_S - 1) / GUW_S;
  const int U = p.I / 8;
  const int nu = (U - g0 + G - 1) / G;                          // >= 1 (grid <= U)
  const int myu = (nu - grp + GUW_GROUPS - 1) / GUW_GROUPS;     // units of this wave, 0..UPW
  const int rsel = ln < 8 ? ln : p.I + ln - 8;                  // row of unit u: 8u + rsel
  const int bufsz = p.M * GUW_XSTRIDE;
  const int total = p.M * (GUW_KC / 8);                          // 16-byte x chunks per chunk

  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];

  // Loads: all unconditional with clamped indexes, so every wait is exact
  // (a chunk past the end re-reads the last one, a missing unit the wave's
  // last or the workgroup's first).
  uint4 xv[XU];
  auto load_x = [&](int c) __attribute__((always_inline)) {
    c = min(c, NC - 1);
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int i = min(u * NTH + tid, total - 1);
      const int m = i >> 6, cc = i & 63;
      const int col = min(c * GUW_KC + 8 * cc, p.K - 8);
      xv[u] = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + col);
    }
  };
  auto store_x = [&](int c) __attribute__((always_inline)) {
    uint16_t* buf = xs + (c & 1) * bufsz;
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int i = min(u * NTH + tid, total - 1);
      const int m = i >> 6, cc = i & 63;
      *reinterpret_cast<uint4*>(buf + m * GUW_XSTRIDE + 8 * cc) = deinterleave8(xv[u]);
    }
  };
  auto load_w_chunk = [&](int c, uint4 (&wv)[2 * GUW_UPW], float (&av)[GUW_UPW])
      __attribute__((always_inline)) {
    const int ks = min(c * GUW_S + ksl, KS - 1);
    const int kc = ks * KSTEP + 64 * lg;
#pragma unroll
    for (int t = 0; t < GUW_UPW; ++t) {
      const int j = min(grp + GUW_GROUPS * min(t, max(myu - 1, 0)), nu - 1);
      const int64_t row = (int64_t)8 * (g0 + j * G) + rsel;
      const uint4* wp = reinterpret_cast<const uint4*>(p.w + row * (p.K / 2) + kc / 2);
      wv[2 * t] = load_w<false>(wp);
      wv[2 * t + 1] = load_w<false>(wp + 1);
      av[t] = p.absmax[(row * p.K + kc) >> p.bs_shift];
    }
  };

  f32x4_t acc[GUW_UPW][MT];
#pragma unroll
  for (int t = 0; t < GUW_UPW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int c, const uint4 (&wv)[2 * GUW_UPW], const float (&av)[GUW_UPW])
      __attribute__((always_inline)) {
    if (c * GUW_S + ksl >= KS || myu == 0) return;  // wave-uniform
    const uint16_t* buf = xs + (c & 1) * bufsz + ksl * KSTEP + 64 * lg;
    const uint16_t* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xrow[mt] = buf + min(mt * 16 + ln, p.M - 1) * GUW_XSTRIDE;
    Lut lt[GUW_UPW];
#pragma unroll
    for (int t = 0; t < GUW_UPW; ++t) lt[t] = make_lut(code, av[t]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint4 a[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) a[mt] = *reinterpret_cast<const uint4*>(xrow[mt] + 8 * j);
#pragma unroll
      for (int t = 0; t < GUW_UPW; ++t) {
        if (t >= myu) break;
        const uint4 bw = decode8(word(wv[2 * t + (j >> 2)], j & 3), lt[t]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma16x16x32(a[mt], bw, acc[t][mt]);
      }
    }
  };

  uint4 wa[2 * GUW_UPW], wb[2 * GUW_UPW];
  float aa[GUW_UPW], ab[GUW_UPW];
  load_x(0);
  load_w_chunk(0, wa, aa);
  store_x(0);
  load_x(1);
  __syncthreads();
  // chunk c: the next chunk's weights are issued, chunk c is multiplied from
  // LDS buffer c & 1, chunk c + 1 (loaded during chunk c - 1) goes into the
  // other buffer, chunk c + 2 is loaded.
  auto step = [&](int c, const uint4 (&wc)[2 * GUW_UPW], const float (&ac)[GUW_UPW],
                  uint4 (&wn)[2 * GUW_UPW], float (&an)[GUW_UPW]) __attribute__((always_inline)) {
    load_w_chunk(c + 1, wn, an);
    compute(c, wc, ac);
    store_x(c + 1);
    load_x(c + 2);
    __syncthreads();
  };
  for (int c = 0; c < NC; c += 2) {
    step(c, wa, aa, wb, ab);
    if (c + 1 < NC) step(c + 1, wb, ab, wa, aa);
  }

  // Both k-step lanes leave their sums in LDS (the x buffers are free) as
  // [slot][lane][m][GUW_EPS] floats, slot = grp + GROUPS t: columns 0..7 gate,
  // 8..15 up, padded to 20 so that the 64 lanes' stores of one r hit 64
  // distinct banks.  Then every thread finishes (slot, row) pairs: both lanes'
  // gate and up sums, SiLU, 8 bf16 in one 16-byte store.
  float* red = reinterpret_cast<float*>(xs);
#pragma unroll
  for (int t = 0; t < GUW_UPW; ++t) {
    if (t >= myu) break;
    const int slot = grp + GUW_GROUPS * t;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // lane (n = ln, group lg) holds D[m = 16 mt + 4 lg + r][n]
        const int m = mt * 16 + 4 * lg + r;
        if (m < p.M) red[((slot * GUW_S + ksl) * p.M + m) * GUW_EPS + ln] = acc[t][mt][r];
      }
  }
  __syncthreads();
  for (int i = tid; i < nu * p.M; i += NTH) {
    const int slot = i / p.M, m = i - slot * p.M;
    const float* r0 = red + ((slot * GUW_S) * p.M + m) * GUW_EPS;
    const float* r1 = r0 + p.M * GUW_EPS;
    float o[8];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const float4 g0 = *reinterpret_cast<const float4*>(r0 + 4 * q);
      const float4 g1 = *reinterpret_cast<const float4*>(r1 + 4 * q);
      const float4 u0 = *reinterpret_cast<const float4*>(r0 + 8 + 4 * q);
      const float4 u1 = *reinterpret_cast<const float4*>(r1 + 8 + 4 * q);
      const float gs[4] = {g0.x + g1.x, g0.y + g1.y, g0.z + g1.z, g0.w + g1.w};
      const float us[4] = {u0.x + u1.x, u0.y + u1.y, u0.z + u1.z, u0.w + u1.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float gv = round_bf(gs[e]);
        o[4 * q + e] = round_bf(gv * (1.f / (1.f + expf(-gv)))) * round_bf(us[e]);
      }
    }
    uint16_t* dst = p.act + (int64_t)m * p.lda + 8 * (g0 + slot * G);
    if (p.act_vec) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]),
                                                  pack_bf2(o[4], o[5]), pack_bf2(o[6], o[7]));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[e] = f2bf(o[e]);
    }
  }
}

#ifndef GRPO_GU_UNITS_GRID
#define GRPO_GU_UNITS_GRID 256
#endif
#ifndef GRPO_GU_UNITS_W
#define GRPO_GU_UNITS_W 8
#endif
int g_gu_units_grid = GRPO_GU_UNITS_GRID;  // workgroups of nf4_gate_up_units (the CU count)
constexpr int GU_UNITS_W = GRPO_GU_UNITS_W;  // waves per workgroup
constexpr int GU_UNITS_IPW = 8;              // most (unit, k-step) items per wave

#ifndef GRPO_GU_KPW
#define GRPO_GU_KPW 3
#endif
int g_gu_kpw = GRPO_GU_KPW;  // k-steps per wave of the gate|up kernel (S = ceil(K/256 / kpw) <= 8); measured best

struct GuPlan {
  int kpw, S, MT;
  size_t lds;
};

// Work split of nf4_gate_up_units: rows <= its waves with an even number of
// k-steps take the folded units (4 + 4 columns, two k-steps per item, one
// staged x row per wave), other shapes units of 8 + 8 columns, one k-step per
// item.  U units over G <= CU-count workgroups, nu per workgroup, KI items
// per unit, `tile` LDS bytes per item partial.
bool units_fold(int M, int K) { return M <= std::min(GU_UNITS_W, 8) && (K / KSTEP) % 2 == 0; }
struct UnitsShape {
  int U, KI, G, nu;
  size_t tile;
};
UnitsShape units_shape(int M, int I, int K) {
  const bool f = units_fold(M, K);
  UnitsShape u;
  u.U = I / (f ? 4 : 8);
  u.KI = K / KSTEP / (f ? 2 : 1);
  u.G = std::min(u.U, g_gu_units_grid);
  u.nu = (u.U + u.G - 1) / u.G;
  u.tile = f ? 512 : (size_t)((M + 3) / 4 * 4) * 16 * 4;
  return u;
}

// LDS of nf4_gate_up_units (x, then the item tiles) and whether it takes the
// shape (at most one workgroup per CU, every item of a wave in registers, 64
// KiB of LDS up to 16 rows).
size_t units_lds(int M, int I, int K) {
  const UnitsShape u = units_shape(M, I, K);
  return (size_t)M * (K + 8) * 2 + (size_t)u.nu * u.KI * u.tile;
}
bool units_ok(int M, int I, int K) {
  if (M < 1 || M > 32 || I <= 0 || I % 8 || K <= 0 || K % KSTEP) return false;
  if ((int64_t)2 * I * K >= ((int64_t)1 << 32)) return false;  // 32-bit element offsets
  const UnitsShape u = units_shape(M, I, K);
  // up to 16 rows in 64 KiB of LDS; 17..32 rows (two row tiles) in up to 160 KiB
  const size_t cap = M <= 16 ? 65536 : (size_t)PART_LDS_BIG;
  return (u.nu * u.KI + GU_UNITS_W - 1) / GU_UNITS_W <= GU_UNITS_IPW && units_lds(M, I, K) <= cap;
}

// 17..32 rows on the unit kernel with two row tiles (x and the item tiles in LDS).
bool units2_ok(int M, int I, int K, int blocksize) {
  return M > 16 && pow2(blocksize) && blocksize >= 64 && units_ok(M, I, K);
}

// Shape support of nf4_gate_up_silu; returns false for shapes it does not take.
bool plan_gu(int M, int I, int K, int blocksize, GuPlan* pl) {
  if (M < 1 || M > 16 || I <= 0 || I % 16 || K <= 0 || K % KSTEP) return false;
  if (!pow2(blocksize) || blocksize < 64) return false;
  const int KS = K / KSTEP;
  int kpw = std::min(g_gu_kpw, KS);
  while ((KS + kpw - 1) / kpw > 8) ++kpw;
  if (kpw > 3) return false;
  pl->kpw = kpw;
  pl->S = (KS + kpw - 1) / kpw;
  pl->MT = 1;
  pl->lds = (size_t)M * (K + 8) * 2 + (size_t)2 * pl->S * M * 16 * 4;
  return pl->lds <= 65536;
}

// Shape support of nf4_gate_up_wide (17..64 rows) and its LDS bytes.
bool gu_wide_ok(int M, int I, int K, int blocksize, size_t* lds) {
  if (M < 17 || M > 64 || I <= 0 || I % 8 || K < KSTEP || K % KSTEP) return false;
  if (!pow2(blocksize) || blocksize < 64) return false;
  const int U = I / 8;
  const int G = std::min(U, g_gu_units_grid);
  if ((U + G - 1) / G > GUW_GROUPS * GUW_UPW) return false;
  const size_t xbytes = (size_t)2 * M * GUW_XSTRIDE * 2;
  const size_t rbytes = (size_t)GUW_GROUPS * GUW_UPW * GUW_S * M * GUW_EPS * 4;
  *lds = std::max(xbytes, rbytes);
  return *lds <= (size_t)PART_LDS_BIG;
}

// ---------------------------------------------------- generic linear --

struct GenArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  const float* absmax;
  const float* code16;
  int blocksize, nseg, r;
  int seg_end[MAXSEG];
  const uint16_t* bias[MAXSEG];
  const uint16_t* la[MAXSEG];
  const uint16_t* lb[MAXSEG];
  float scaling;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
};

// Any shape: one thread per output; the reference arithmetic spelled out.
__global__ void __launch_bounds__(256) nf4_linear_generic(GenArgs p) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)p.M * p.N) return;
  const int m = (int)(idx / p.N), n = (int)(idx % p.N);
  int seg = 0;
  while (seg + 1 < p.nseg && n >= p.seg_end[seg]) ++seg;
  const int n_loc = n - (seg > 0 ? p.seg_end[seg - 1] : 0);
  const uint16_t* xr = p.x + (int64_t)m * p.ldx;
  float acc = 0.f;
  for (int k = 0; k < p.K; ++k) {
    const int64_t e = (int64_t)n * p.K + k;
    const uint32_t byte = p.w[e >> 1];
    const uint32_t q = (e & 1) ? (byte & 15u) : (byte >> 4);
    const float wv = round_bf(p.code16[q] * p.absmax[e / p.blocksize]);
    acc += bf2f(xr[k]) * wv;
  }
  float v = round_bf(acc);
  if (p.bias[seg]) v = round_bf(v + bf2f(p.bias[seg][n_loc]));
  if (p.r > 0) {
    float u = 0.f;
    for (int rr = 0; rr < p.r; ++rr) {
      const uint16_t* ar = p.la[seg] + (int64_t)rr * p.K;
      float t = 0.f;
      for (int k = 0; k < p.K; ++k) t += bf2f(xr[k]) * bf2f(ar[k]);
      u += round_bf(t) * bf2f(p.lb[seg][(int64_t)n_loc * p.r + rr]);
    }
    u = round_bf(round_bf(u) * round_bf(p.scaling));
    v = round_bf(v + u);
  }
  p.y[(int64_t)m * p.ldy + n] = f2bf(v);
}

// ------------------------------------------------------ linear driver --

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// One NF4 (+ LoRA) linear into y: split-K partials + finish when the shape,
// alignment and workspace allow it (M <= 64), else the NF4 GEMM, else the
// generic kernel.
int run_linear(const GenArgs& g, void* workspace, size_t workspace_bytes, hipStream_t st) {
  bool fast = part_shape_ok(g.M, g.N, g.K, g.r, g.nseg, g.blocksize, g.seg_end) &&
              g.ldx % 8 == 0 && aligned16(g.x) && aligned16(g.w);
  for (int s = 0; fast && s < g.nseg && g.r > 0; ++s) fast = aligned16(g.la[s]);
  if (fast) {
    const PartPlan pl = plan_part(g.M, g.N, g.K, g.r, g.nseg);
    const size_t need = align256(pl.part_bytes) + pl.tpart_bytes;
    if (!workspace || workspace_bytes < need) {
      set_error("workspace of %zu bytes needed, %zu given", need, workspace_bytes);
      return GRPO_EWORKSPACE;
    }
    grpo_linear_parts_t h{};
    h.part = static_cast<float*>(workspace);
    h.tpart = g.r > 0 ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) +
                                                 align256(pl.part_bytes))
                      : nullptr;
    h.splits = pl.S;
    h.M = g.M;
    h.N = g.N;
    h.K = g.K;
    h.nseg = g.nseg;
    h.r = g.r;
    for (int s = 0; s < g.nseg; ++s) {
      h.seg_end[s] = g.seg_end[s];
      h.bias[s] = g.bias[s];
      h.lora_b[s] = g.lb[s];
    }
    h.scaling = g.scaling;
    if (int rc = run_partials(g.x, g.ldx, g.w, g.absmax, g.code16, g.blocksize, g.la, h, st))
      return rc;
    return run_finish(&h, g.y, g.ldy, st);
  }
  // Wider batches: the NF4 GEMM, one launch for all segments of the stacked weight.
  bool gemm = g.ldx % 8 == 0 && aligned16(g.x) && aligned16(g.w);
  for (int s = 0, start = 0; gemm && s < g.nseg; start = g.seg_end[s], ++s)
    gemm = nf4_gemm_ok(g.M, g.seg_end[s] - start, g.K, g.r, g.blocksize) &&
           (g.r == 0 || aligned16(g.la[s]));
  if (gemm) {
    // Few tiles and a long K: the K slices write float32 partial sums (LinParts
    // layout over all segments) and nf4_finish applies the epilogue.
    // A workspace smaller than the plan's partial sums runs the linear unsplit.
    GemmPlan pl = nf4_gemm_plan(g.M, g.K, g.r, g.nseg, g.seg_end);
    if (pl.S > 1 && (!workspace || workspace_bytes < align256(pl.part_bytes) + pl.tpart_bytes))
      pl.S = 1;
    GemmSplit sp{};
    grpo_linear_parts_t h{};
    GemmSegs sg{};
    sg.nseg = g.nseg;
    for (int s = 0; s < g.nseg; ++s) {
      sg.seg_end[s] = g.seg_end[s];
      sg.bias[s] = g.bias[s];
      sg.la[s] = g.la[s];
      sg.lb[s] = g.lb[s];
    }
    if (pl.S > 1) {
      sp.S = pl.S;
      sp.kst = pl.kst;
      sp.ldp = g.N;
      sp.psl = (int64_t)g.M * g.N;
      sp.tsl = (int64_t)g.nseg * g.M * 16;
      sp.tseg = (int64_t)g.M * 16;
      h.part = static_cast<float*>(workspace);
      h.tpart = g.r > 0 ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) +
                                                   align256(pl.part_bytes))
                        : nullptr;
      h.splits = pl.S;
      h.M = g.M;
      h.N = g.N;
      h.K = g.K;
      h.nseg = g.nseg;
      h.r = g.r;
      for (int s = 0; s < g.nseg; ++s) {
        h.seg_end[s] = g.seg_end[s];
        h.bias[s] = g.bias[s];
        h.lora_b[s] = g.lb[s];
      }
      h.scaling = g.scaling;
    }
    sp.part = h.part;
    sp.tpart = h.tpart;
    // one launch for every segment
    if (int rc = nf4_gemm_launch(g.x, g.ldx, g.w, 0, g.absmax, g.code16, g.blocksize, sg, g.r,
                                 g.scaling, g.y, g.ldy, g.M, g.K, st, pl.S > 1 ? &sp : nullptr))
      return rc;
    return pl.S > 1 ? nf4_gemm_finish(&h, g.y, g.ldy, st) : GRPO_OK;
  }
  const int64_t total = (int64_t)g.M * g.N;
  nf4_linear_generic<<<dim3((unsigned)cdiv(total, 256)), 256, 0, st>>>(g);
  return launch_check("nf4_linear_generic");
}

size_t workspace_bytes_for(int M, int N, int K, int r, int nseg, int blocksize,
                           const int* seg_end) {
  if (!part_shape_ok(M, N, K, r, nseg, blocksize, seg_end)) {
    // The NF4 GEMM: partial sums when it splits K.  Without the segment ends
    // (a size query) the plan of one N-column segment bounds every split of N
    // (more segments make at least as many tiles, so no more slices).
    GemmPlan pl;
    if (seg_end) {
      for (int s = 0, start = 0; s < nseg; start = seg_end[s], ++s)
        if (!nf4_gemm_ok(M, seg_end[s] - start, K, r, blocksize)) return 0;
      pl = nf4_gemm_plan(M, K, r, nseg, seg_end);
    } else {
      if (!nf4_gemm_ok(M, N, K, r, blocksize)) return 0;
      pl = nf4_gemm_plan(M, K, r, 1, &N);
      pl.tpart_bytes = r > 0 ? (size_t)pl.S * nseg * M * 16 * 4 : 0;
    }
    return pl.S > 1 ? align256(pl.part_bytes) + pl.tpart_bytes : 0;
  }
  const PartPlan pl = plan_part(M, N, K, r, nseg);
  return align256(pl.part_bytes) + pl.tpart_bytes;
}

int check_common(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                 const float* code16, int blocksize, int r, const void* y, int64_t ldy, int M,
                 int N, int K) {
  if (M < 0 || N < 0 || K < 0) return einval("negative dimension");
  if (r < 0) return einval("r < 0");
  if (blocksize <= 0) return einval("blocksize must be > 0");
  if (M == 0 || N == 0) return GRPO_OK;
  if (!x || !w || !absmax || !code16 || !y) return einval("null pointer");
  if (ldx < K || ldy < N) return einval("row stride smaller than the row");
  return GRPO_OK;
}

}  // namespace

namespace grpo {

int make_parts(const grpo_linear_parts_t* h, LinParts* d) {
  if (!h) return einval("null parts descriptor");
  if (h->splits < 1 || h->M < 1 || h->N < 1 || h->K < 1) return einval("bad parts dimensions");
  if (h->splits > MAX_SLICES) return einval("parts: at most 20 K slices");
  if (h->nseg < 1 || h->nseg > MAXSEG) return einval("nseg must be in [1, 4]");
  if (h->r < 0 || h->r > 16) return einval("parts: r must be in [0, 16]");
  if (!h->part || (h->r > 0 && !h->tpart)) return einval("parts: null partial-sum buffer");
  int prev = 0;
  for (int s = 0; s < h->nseg; ++s) {
    if (h->seg_end[s] <= prev) return einval("parts: segment ends must increase");
    prev = h->seg_end[s];
    if (h->r > 0 && !h->lora_b[s]) return einval("parts: r > 0 needs lora_b per segment");
  }
  if (prev != h->N) return einval("parts: last segment end must equal N");
  d->part = h->part;
  d->tpart = h->tpart;
  d->S = h->splits;
  d->M = h->M;
  d->N = h->N;
  d->K = h->K;
  d->nseg = h->nseg;
  d->r = h->r;
  d->lb_vec = h->r == 16;
  d->bias_vec = true;
  for (int s = 0; s < MAXSEG; ++s) {
    const bool on = s < h->nseg;
    d->seg_end[s] = on ? h->seg_end[s] : h->N;
    d->bias[s] = on ? static_cast<const uint16_t*>(h->bias[s]) : nullptr;
    d->lb[s] = on && h->r > 0 ? static_cast<const uint16_t*>(h->lora_b[s]) : nullptr;
    if (on && h->r > 0) d->lb_vec = d->lb_vec && aligned16(h->lora_b[s]);
    if (d->bias[s]) d->bias_vec = d->bias_vec && (reinterpret_cast<uintptr_t>(d->bias[s]) & 7u) == 0;
  }
  if (h->N % 16 != 0) return einval("parts: N must be a multiple of 16");
  for (int s = 0; s < h->nseg; ++s)
    if (h->seg_end[s] % 16 != 0) return einval("parts: segment ends must be multiples of 16");
  if ((reinterpret_cast<uintptr_t>(h->part) & 15u) != 0 ||
      (h->tpart && (reinterpret_cast<uintptr_t>(h->tpart) & 15u) != 0))
    return einval("parts: partial-sum buffers must be 16-byte aligned");
  d->scaling = h->scaling;
  return GRPO_OK;
}

// Float32 absmax of a double-quantized state: one FMA per block, as the
// reference's kernel computes it (lora_forward.py:187-199: the multiply and
// add of code2[q] * absmax2 + offset contract into one fused multiply-add).
__global__ void __launch_bounds__(256) nf4_absmax_expand_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ code2,
    const float* __restrict__ absmax2, int bs2, float offset, int64_t n, float* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    out[i] = __fmaf_rn(code2[q[i]], absmax2[i / bs2], offset);
}

}  // namespace grpo

extern "C" int grpo_nf4_absmax_expand(const uint8_t* absmax_q, const float* code2,
                                      const float* absmax2, int bs2, float offset,
                                      int64_t n_blocks, float* out, grpo_stream_t stream) {
  if (n_blocks < 0) return einval("n_blocks < 0");
  if (bs2 <= 0) return einval("state2 blocksize must be > 0");
  if (n_blocks == 0) return GRPO_OK;
  if (!absmax_q || !code2 || !absmax2 || !out) return einval("null pointer");
  const int64_t blocks = std::min<int64_t>(cdiv(n_blocks, 256), 8192);
  nf4_absmax_expand_kernel<<<dim3((unsigned)blocks), 256, 0, as_stream(stream)>>>(
      absmax_q, code2, absmax2, bs2, offset, n_blocks, out);
  return launch_check("nf4_absmax_expand");
}

namespace {

template <bool F16>
int run_dequant(const uint8_t* w, const float* absmax, const float* code16, void* out,
                int64_t numel, int blocksize, grpo_stream_t stream) {
  if (numel < 0) return einval("numel < 0");
  if (blocksize <= 0) return einval("blocksize must be > 0");
  if (numel == 0) return GRPO_OK;
  if (!w || !absmax || !code16 || !out) return einval("null pointer");
  hipStream_t st = as_stream(stream);
  if (numel % 16 == 0 && blocksize % 16 == 0 && (reinterpret_cast<uintptr_t>(w) & 7u) == 0 &&
      aligned16(out)) {
    const int64_t nvec = numel / 16;
    const int64_t blocks = std::min<int64_t>(cdiv(nvec, 256), 8192);
    nf4_dequant_vec<F16><<<dim3((unsigned)blocks), 256, 0, st>>>(
        reinterpret_cast<const uint2*>(w), absmax, code16, reinterpret_cast<uint4*>(out), nvec,
        blocksize);
  } else {
    const int64_t blocks = std::min<int64_t>(cdiv(numel, 256), 8192);
    nf4_dequant_scalar<F16><<<dim3((unsigned)blocks), 256, 0, st>>>(
        w, absmax, code16, reinterpret_cast<uint16_t*>(out), numel, blocksize);
  }
  return launch_check("nf4_dequant");
}

}  // namespace

extern "C" int grpo_nf4_dequant(const uint8_t* w, const float* absmax, const float* code16,
                                void* out, int64_t numel, int blocksize, grpo_stream_t stream) {
  return run_dequant<false>(w, absmax, code16, out, numel, blocksize, stream);
}

extern "C" int grpo_nf4_dequant_f16(const uint8_t* w, const float* absmax, const float* code16,
                                    void* out, int64_t numel, int blocksize,
                                    grpo_stream_t stream) {
  return run_dequant<true>(w, absmax, code16, out, numel, blocksize, stream);
}

extern "C" int grpo_nf4_linear_plan(int M, int N, int K, int r, int nseg, int blocksize,
                                    int* splits, size_t* part_bytes, size_t* tpart_bytes) {
  if (!part_shape_ok(M, N, K, r, nseg, blocksize, nullptr)) {
    set_error("shape not supported by the split-K NF4 linear");
    return GRPO_EUNSUPPORTED;
  }
  const PartPlan pl = plan_part(M, N, K, r, nseg);
  if (!pl.ok) {
    set_error("shape not supported by the split-K NF4 linear");
    return GRPO_EUNSUPPORTED;
  }
  if (splits) *splits = pl.S;
  if (part_bytes) *part_bytes = pl.part_bytes;
  if (tpart_bytes) *tpart_bytes = pl.tpart_bytes;
  return GRPO_OK;
}

extern "C" int grpo_nf4_linear_partials(const void* x, int64_t ldx, const uint8_t* w,
                                        const float* absmax, const float* code16, int blocksize,
                                        const void* const* lora_a,
                                        const grpo_linear_parts_t* parts, grpo_stream_t stream) {
  if (!parts) return einval("null parts descriptor");
  if (blocksize <= 0) return einval("blocksize must be > 0");
  LinParts check;
  if (int rc = make_parts(parts, &check)) return rc;
  const uint16_t* la[MAXSEG] = {nullptr, nullptr, nullptr, nullptr};
  if (parts->r > 0) {
    if (!lora_a) return einval("r > 0 needs lora_a");
    for (int s = 0; s < parts->nseg; ++s) la[s] = static_cast<const uint16_t*>(lora_a[s]);
  }
  return run_partials(static_cast<const uint16_t*>(x), ldx, w, absmax, code16, blocksize, la,
                      *parts, as_stream(stream));
}

extern "C" int grpo_nf4_linear_finish(const grpo_linear_parts_t* parts, void* y, int64_t ldy,
                                      grpo_stream_t stream) {
  return run_finish(parts, static_cast<uint16_t*>(y), ldy, as_stream(stream));
}

extern "C" size_t grpo_nf4_lora_linear_workspace_bytes(int M, int N, int K, int r, int nseg,
                                                       int blocksize) {
  return workspace_bytes_for(M, N, K, r, nseg, blocksize, nullptr);
}

extern "C" int grpo_nf4_lora_linear(const void* x, int64_t ldx, const uint8_t* w,
                                    const float* absmax, const float* code16, int blocksize,
                                    const void* bias, const void* lora_a, const void* lora_b, int r,
                                    float scaling, void* y, int64_t ldy, int M, int N, int K,
                                    void* workspace, size_t workspace_bytes,
                                    grpo_stream_t stream) {
  if (int rc = check_common(x, ldx, w, absmax, code16, blocksize, r, y, ldy, M, N, K)) return rc;
  if (M == 0 || N == 0) return GRPO_OK;
  if (r > 0 && (!lora_a || !lora_b)) return einval("r > 0 needs lora_a and lora_b");
  GenArgs g{};
  g.x = static_cast<const uint16_t*>(x);
  g.ldx = ldx;
  g.w = w;
  g.absmax = absmax;
  g.code16 = code16;
  g.blocksize = blocksize;
  g.nseg = 1;
  g.seg_end[0] = N;
  g.bias[0] = static_cast<const uint16_t*>(bias);
  g.la[0] = r > 0 ? static_cast<const uint16_t*>(lora_a) : nullptr;
  g.lb[0] = r > 0 ? static_cast<const uint16_t*>(lora_b) : nullptr;
  g.r = r;
  g.scaling = scaling;
  g.y = static_cast<uint16_t*>(y);
  g.ldy = ldy;
  g.M = M;
  g.N = N;
  g.K = K;
  return run_linear(g, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int grpo_nf4_lora_linear_grouped(const void* x, int64_t ldx, const uint8_t* w,
                                            const float* absmax, const float* code16,
                                            int blocksize, int nseg, const int* seg_rows,
                                            const void* const* bias, const void* const* lora_a,
                                            const void* const* lora_b, int r, float scaling,
                                            void* y, int64_t ldy, int M, int K, void* workspace,
                                            size_t workspace_bytes, grpo_stream_t stream) {
  if (nseg < 1 || nseg > MAXSEG) return einval("nseg must be in [1, 4]");
  if (!seg_rows) return einval("null seg_rows");
  int N = 0;
  for (int s = 0; s < nseg; ++s) {
    if (seg_rows[s] <= 0) return einval("segment with no rows");
    N += seg_rows[s];
  }
  if (int rc = check_common(x, ldx, w, absmax, code16, blocksize, r, y, ldy, M, N, K)) return rc;
  if (M == 0) return GRPO_OK;
  GenArgs g{};
  g.x = static_cast<const uint16_t*>(x);
  g.ldx = ldx;
  g.w = w;
  g.absmax = absmax;
  g.code16 = code16;
  g.blocksize = blocksize;
  g.nseg = nseg;
  int end = 0;
  for (int s = 0; s < nseg; ++s) {
    end += seg_rows[s];
    g.seg_end[s] = end;
    g.bias[s] = bias ? static_cast<const uint16_t*>(bias[s]) : nullptr;
    g.la[s] = r > 0 && lora_a ? static_cast<const uint16_t*>(lora_a[s]) : nullptr;
    g.lb[s] = r > 0 && lora_b ? static_cast<const uint16_t*>(lora_b[s]) : nullptr;
    if (r > 0 && (!g.la[s] || !g.lb[s])) return einval("r > 0 needs lora_a and lora_b per segment");
    if (nseg > 1 && (int64_t)seg_rows[s] * K % blocksize != 0)
      return einval("every segment must hold whole absmax blocks");
  }
  g.r = r;
  g.scaling = scaling;
  g.y = static_cast<uint16_t*>(y);
  g.ldy = ldy;
  g.M = M;
  g.N = N;
  g.K = K;
  return run_linear(g, workspace, workspace_bytes, as_stream(stream));
}

namespace {
int run_partials_attn(const void* attn_workspace, const int32_t* context_lens, int Hq, int Hkv,
                      int D, int block_size, int max_blocks, const uint8_t* w,
                      const float* absmax, const float* code16, int blocksize,
                      const void* const* lora_a, const grpo_linear_parts_t* parts,
                      grpo_stream_t stream, const FinTarget* fin) {
  if (!parts) return einval("null parts descriptor");
  if (blocksize <= 0) return einval("blocksize must be > 0");
  LinParts check;
  if (int rc = make_parts(parts, &check)) return rc;
  if (!attn_workspace || !context_lens) return einval("null pointer");
  if (!aligned16(attn_workspace)) return einval("attention workspace must be 16-byte aligned");
  if (Hkv <= 0 || Hq <= 0 || D != 128 || parts->K != Hq * D)
    return einval("attention input needs head_dim 128 and K == Hq * 128");
  AttnSource att;
  if (attn_plan_geometry(parts->M, Hq, Hkv, D, block_size, max_blocks, &att.bps, &att.S) != 0) {
    set_error("attention geometry not supported by the split attention kernel");
    return GRPO_EUNSUPPORTED;
  }
  if (att.S > ATTN_MAX_SPLITS) return einval("too many attention splits");
  att.o = static_cast<const float*>(attn_workspace);
  att.ml = att.o + (size_t)parts->M * Hq * att.S * D;
  att.len = context_lens;
  att.Hq = Hq;
  att.cap = max_blocks * block_size;
  const uint16_t* la[MAXSEG] = {nullptr, nullptr, nullptr, nullptr};
  if (parts->r > 0) {
    if (!lora_a) return einval("r > 0 needs lora_a");
    for (int s = 0; s < parts->nseg; ++s) la[s] = static_cast<const uint16_t*>(lora_a[s]);
  }
  return run_partials(nullptr, 0, w, absmax, code16, blocksize, la, *parts, as_stream(stream),
                      &att, nullptr, nullptr, fin);
}
}  // namespace

extern "C" int grpo_nf4_linear_partials_attn(const void* attn_workspace,
                                             const int32_t* context_lens, int Hq, int Hkv,
                                             int D, int block_size, int max_blocks,
                                             const uint8_t* w, const float* absmax,
                                             const float* code16, int blocksize,
                                             const void* const* lora_a,
                                             const grpo_linear_parts_t* parts,
                                             grpo_stream_t stream) {
  return run_partials_attn(attn_workspace, context_lens, Hq, Hkv, D, block_size, max_blocks, w,
                           absmax, code16, blocksize, lora_a, parts, stream, nullptr);
}

extern "C" int grpo_nf4_linear_attn_residual_groups(int M, int N, int K, int r, int blocksize,
                                                    size_t* tpart_bytes, size_t* counter_bytes) {
  constexpr int WPG = waves_per_group(X_ATTN);
  if (!part_shape_ok(M, N, K, r, 1, blocksize, nullptr)) return 0;
  const PartPlan pl = plan_part(M, N, K, r, 1);
  if (!pl.ok || pl.MT != 1 || pl.NT % WPG != 0 || pl.S > FIN_MAX_SLICES || pl.kpw > 2) return 0;
  const int groups = pl.NT / WPG;
  if (tpart_bytes) *tpart_bytes = (size_t)groups * pl.S * M * 16 * sizeof(float);
  if (counter_bytes) *counter_bytes = (size_t)groups * FIN_CNT_STRIDE * sizeof(int);
  return groups;
}

extern "C" int grpo_nf4_linear_attn_residual(
    const void* attn_workspace, const int32_t* context_lens, int Hq, int Hkv, int D,
    int block_size, int max_blocks, const uint8_t* w, const float* absmax, const float* code16,
    int blocksize, const void* const* lora_a, const grpo_linear_parts_t* parts,
    float* group_tpart, int* counters, int* xcd_err, const void* residual, void* h_out,
    int64_t ld, float* sumsq, grpo_stream_t stream) {
  FinTarget fin;
  fin.tpart = group_tpart;
  fin.cnt = counters;
  fin.err = xcd_err;
  fin.res = static_cast<const uint16_t*>(residual);
  fin.h = static_cast<uint16_t*>(h_out);
  fin.ld = ld;
  fin.ss = sumsq;
  return run_partials_attn(attn_workspace, context_lens, Hq, Hkv, D, block_size, max_blocks, w,
                           absmax, code16, blocksize, lora_a, parts, stream, &fin);
}

extern "C" int grpo_nf4_linear_partials_silu(const grpo_linear_parts_t* gate_up, const uint8_t* w,
                                             const float* absmax, const float* code16,
                                             int blocksize, const grpo_linear_parts_t* parts,
                                             grpo_stream_t stream) {
  if (!parts || !gate_up) return einval("null parts descriptor");
  if (blocksize <= 0) return einval("blocksize must be > 0");
  LinParts check, gu;
  if (int rc = make_parts(parts, &check)) return rc;
  if (int rc = make_parts(gate_up, &gu)) return rc;
  if (gu.r != 0) return einval("gate|up source must have no LoRA term");
  for (int s = 0; s < gu.nseg; ++s)
    if (gu.bias[s]) return einval("gate|up source must have no bias");
  if (gu.M != parts->M || gu.N != 2 * parts->K)
    return einval("gate|up source must be [M, 2K] for a down projection of input width K");
  if (gu.S > GU_MAX_SLICES) {
    set_error("gate|up source has more than 2 K slices");
    return GRPO_EUNSUPPORTED;
  }
  SiluSource src;
  src.part = gu.part;
  src.S = gu.S;
  const uint16_t* la[MAXSEG] = {nullptr, nullptr, nullptr, nullptr};
  if (parts->r > 0) return einval("down projection with LoRA is not supported here");
  return run_partials(nullptr, 0, w, absmax, code16, blocksize, la, *parts, as_stream(stream),
                      nullptr, &src);
}

extern "C" int grpo_nf4_gate_up_silu_supported(int M, int I, int K, int blocksize) {
  GuPlan pl;
  size_t lds;
  return plan_gu(M, I, K, blocksize, &pl) || units2_ok(M, I, K, blocksize) ||
                 gu_wide_ok(M, I, K, blocksize, &lds) ||
                 (M > 64 && nf4_gemm_silu_ok(M, I, K, blocksize))
             ? 1
             : 0;
}

namespace {
int run_gate_up(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                const float* code16, int blocksize, int I, int K, int M, void* act, int64_t lda,
                int act_tiles, hipStream_t st, const NormSource* nrm = nullptr);
}  // namespace

extern "C" int grpo_nf4_gate_up_silu(const void* x, int64_t ldx, const uint8_t* w,
                                     const float* absmax, const float* code16, int blocksize,
                                     int I, int K, int M, void* act, int64_t lda,
                                     grpo_stream_t stream) {
  return run_gate_up(x, ldx, w, absmax, code16, blocksize, I, K, M, act, lda, 0,
                     as_stream(stream));
}

extern "C" int grpo_nf4_gate_up_silu_tiles(const void* x, int64_t ldx, const uint8_t* w,
                                           const float* absmax, const float* code16,
                                           int blocksize, int I, int K, int M, void* act_tiles,
                                           grpo_stream_t stream) {
  if (M > 8) return einval("the fold tile layout holds at most 8 rows");
  return run_gate_up(x, ldx, w, absmax, code16, blocksize, I, K, M, act_tiles, I, 1,
                     as_stream(stream));
}

extern "C" int grpo_nf4_gate_up_silu_tiles_norm(const void* h, int64_t ldh, const float* sumsq,
                                                int groups, const void* norm_weight, float eps,
                                                const uint8_t* w, const float* absmax,
                                                const float* code16, int blocksize, int I, int K,
                                                int M, void* act_tiles, grpo_stream_t stream) {
  if (M > 8) return einval("the fold tile layout holds at most 8 rows");
  if (!h || !sumsq || !norm_weight) return einval("null pointer");
  if (groups < 4 || groups > GU_NORM_MAX_GROUPS || groups % 4)
    return einval("groups must be a multiple of 4 in [4, 256]");
  if (!aligned16(norm_weight) || !aligned16(sumsq))
    return einval("norm_weight and sumsq must be 16-byte aligned");
  NormSource src;
  src.h = static_cast<const uint16_t*>(h);
  src.ldh = ldh;
  src.sumsq = sumsq;
  src.groups = groups;
  src.weight = static_cast<const uint16_t*>(norm_weight);
  src.eps = eps;
  return run_gate_up(h, ldh, w, absmax, code16, blocksize, I, K, M, act_tiles, I, 1,
                     as_stream(stream), &src);
}

extern "C" int grpo_nf4_gate_up_silu_tiles_norm_supported(int M, int I, int K, int blocksize) {
  GuPlan pl;
  return M <= 8 && plan_gu(M, I, K, blocksize, &pl) && units_ok(M, I, K) ? 1 : 0;
}

extern "C" int grpo_nf4_linear_partials_norm(const void* h, int64_t ldh, const float* sumsq,
                                             int groups, const void* norm_weight, float eps,
                                             const uint8_t* w, const float* absmax,
                                             const float* code16, int blocksize,
                                             const void* const* lora_a,
                                             const grpo_linear_parts_t* parts,
                                             grpo_stream_t stream) {
  if (!parts) return einval("null parts descriptor");
  if (blocksize <= 0) return einval("blocksize must be > 0");
  LinParts check;
  if (int rc = make_parts(parts, &check)) return rc;
  if (!h || !sumsq || !norm_weight) return einval("null pointer");
  if (groups < 1 || groups > NORM_MAX_GROUPS) return einval("groups must be in [1, 256]");
  if (ldh < parts->K || ldh % 8 || !aligned16(h) || !aligned16(norm_weight))
    return einval("h and norm_weight must be 16-byte aligned with ldh >= K, ldh % 8 == 0");
  const uint16_t* la[MAXSEG] = {nullptr, nullptr, nullptr, nullptr};
  if (parts->r > 0) {
    if (!lora_a) return einval("r > 0 needs lora_a");
    for (int s = 0; s < parts->nseg; ++s) la[s] = static_cast<const uint16_t*>(lora_a[s]);
  }
  NormSource src;
  src.h = static_cast<const uint16_t*>(h);
  src.ldh = ldh;
  src.sumsq = sumsq;
  src.groups = groups;
  src.weight = static_cast<const uint16_t*>(norm_weight);
  src.eps = eps;
  return run_partials(nullptr, 0, w, absmax, code16, blocksize, la, *parts, as_stream(stream),
                      nullptr, nullptr, &src);
}

namespace {
int run_gate_up(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                const float* code16, int blocksize, int I, int K, int M, void* act, int64_t lda,
                int act_tiles, hipStream_t st, const NormSource* nrm) {
  GuPlan pl;
  size_t wlds = 0;
  // more than 64 rows (prefill chunks): the NF4 GEMM's gate|up SiLU form
  if (M > 64 && !act_tiles && !nrm && nf4_gemm_silu_ok(M, I, K, blocksize))
    return nf4_gemm_silu_launch(static_cast<const uint16_t*>(x), ldx, w, absmax, code16,
                                blocksize, I, K, M, static_cast<uint16_t*>(act), lda, st);
  // 17..32 rows whose x and item tiles fit LDS run the units kernel on two row
  // tiles (x staged once, no chunk barriers; config 4's 32 x 8960 x 1536: 14.3
  // -> 13.2 us per traced launch, 6522 -> 6842 tok/s), the other wide shapes
  // the chunked wide kernel
  const bool units2 = !nrm && !act_tiles && units2_ok(M, I, K, blocksize);
  const bool wide = !units2 && !nrm && !act_tiles && gu_wide_ok(M, I, K, blocksize, &wlds);
  if (!wide && !units2 && !plan_gu(M, I, K, blocksize, &pl)) {
    set_error("shape not supported by the fused gate|up SiLU kernel");
    return GRPO_EUNSUPPORTED;
  }
  if (!x || !w || !absmax || !code16 || !act) return einval("null pointer");
  if (ldx < K || ldx % 8 || !aligned16(x) || !aligned16(w))
    return einval("x and w must be 16-byte aligned with ldx >= K, ldx % 8 == 0");
  if (lda < I) return einval("lda smaller than I");
  GuArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = w;
  a.absmax = absmax;
  a.code16 = code16;
  a.bs_shift = __builtin_ctz((unsigned)blocksize);
  a.act = static_cast<uint16_t*>(act);
  a.lda = lda;
  a.M = M;
  a.I = I;
  a.K = K;
  a.act_tiles = act_tiles;
  a.act_vec = aligned16(act) && lda % 8 == 0;
  if (nrm) {
    a.nh = nrm->h;
    a.ldnh = nrm->ldh;
    a.nss = nrm->sumsq;
    a.nG = nrm->groups;
    a.nw = nrm->weight;
    a.neps = nrm->eps;
  }
  if (wide) {
    const int G = std::min(I / 8, g_gu_units_grid);
    const dim3 grid((unsigned)G), block(64 * GUW_W);
    switch ((M + 15) / 16) {
#define GUW_CASE(MT)                                                        \
  case MT:                                                                  \
    if (int rc = allow_dynamic_lds<nf4_gate_up_wide<MT>, PART_LDS_BIG>()) return rc; \
    nf4_gate_up_wide<MT><<<grid, block, wlds, st>>>(a);                     \
    break;
      GUW_CASE(2) GUW_CASE(3) GUW_CASE(4)
#undef GUW_CASE
      default: return einval("gate|up wide kernel: 17..64 rows");
    }
    return launch_check("nf4_gate_up_wide");
  }
  {
    // units kernel: at most one workgroup per CU, every item of a wave in registers
    const int G = units_shape(M, I, K).G;
    const size_t lds = units_lds(M, I, K);
    if (units2) {
      constexpr auto kern = nf4_gate_up_units<GU_UNITS_W, GU_UNITS_IPW, false, 2>;
      if (int rc = allow_dynamic_lds<kern, PART_LDS_BIG>()) return rc;
      nf4_gate_up_units<GU_UNITS_W, GU_UNITS_IPW, false, 2>
          <<<dim3((unsigned)G), 64 * GU_UNITS_W, lds, st>>>(a);
      return launch_check("nf4_gate_up_units");
    }
    if (units_ok(M, I, K)) {
      const bool rows = units_fold(M, K);  // folded units, one staged x row per wave
      if (nrm && rows)
        nf4_gate_up_units<GU_UNITS_W, GU_UNITS_IPW, true, 1, true>
            <<<dim3((unsigned)G), 64 * GU_UNITS_W, lds, st>>>(a);
      else if (nrm)
        nf4_gate_up_units<GU_UNITS_W, GU_UNITS_IPW, true>
            <<<dim3((unsigned)G), 64 * GU_UNITS_W, lds, st>>>(a);
      else if (rows)
        nf4_gate_up_units<GU_UNITS_W, GU_UNITS_IPW, false, 1, true>
            <<<dim3((unsigned)G), 64 * GU_UNITS_W, lds, st>>>(a);
      else
        nf4_gate_up_units<GU_UNITS_W, GU_UNITS_IPW, false>
            <<<dim3((unsigned)G), 64 * GU_UNITS_W, lds, st>>>(a);
      return launch_check("nf4_gate_up_units");
    }
  }
  if (nrm) {
    set_error("the RMSNorm x source needs the 8-column-unit gate|up kernel for this shape");
    return GRPO_EUNSUPPORTED;
  }
  const dim3 grid((unsigned)(I / 16)), block(128 * pl.S);
  switch (pl.kpw * 16 + pl.S) {
#define GU_CASE(KPW, S) \
  case KPW * 16 + S: nf4_gate_up_silu<KPW, S><<<grid, block, pl.lds, st>>>(a); break;
    GU_CASE(1, 1) GU_CASE(1, 2) GU_CASE(1, 3) GU_CASE(1, 4)
    GU_CASE(1, 5) GU_CASE(1, 6) GU_CASE(1, 7) GU_CASE(1, 8)
    GU_CASE(2, 5) GU_CASE(2, 6) GU_CASE(2, 7) GU_CASE(2, 8)
    GU_CASE(3, 6) GU_CASE(3, 7) GU_CASE(3, 8)
    GU_CASE(2, 1) GU_CASE(2, 2) GU_CASE(2, 3) GU_CASE(2, 4)
    GU_CASE(3, 1) GU_CASE(3, 2) GU_CASE(3, 3) GU_CASE(3, 4) GU_CASE(3, 5)
#undef GU_CASE
    default:
      set_error("gate|up SiLU kernel: no instantiation for %d k-steps x %d slices", pl.kpw, pl.S);
      return GRPO_EUNSUPPORTED;
  }
  return launch_check("nf4_gate_up_silu");
}
}  // namespace
