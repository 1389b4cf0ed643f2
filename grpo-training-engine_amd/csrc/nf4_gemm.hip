// NF4 (+ bias, + LoRA) linear for batches of more than 64 rows on gfx950: one
// MFMA GEMM launch that decodes the 4-bit weight in registers and applies the
// reference epilogue in the kernel.  Restates _lora_forward_kernel
// (src/triton_kernels/lora_forward.py:107-260) for any M:
//   acc = sum_k x[m,k] * bf16(code[q(n,k)] * absmax)   (float32 accumulation)
//   v = bf16(acc); v = bf16(v + bias[n])                (:243-247)
//   t = bf16(x A^T)  (rank r <= 32)                     (:210-236)
//   u = bf16(bf16(t . B[n, :]) * bf16(scaling)); y = bf16(v + u)   (:249-257)
//
//  * Tile: a workgroup (4 waves) owns 128 rows m x 128 columns n; wave w owns
//    all 128 rows x columns 32 w .. 32 w + 31 as 8 x 2 tiles of
//    v_mfma_f32_16x16x32_bf16 (A = x rows from LDS, B = W rows decoded in the
//    wave's registers).  Two workgroups per CU (80 KiB of LDS each).
//  * Stage = 128 K values.  Lane (n = lane % 16, group g = lane / 16) of a
//    column tile holds the 32 nibbles [32 g, 32 g + 32) of its weight row (one
//    16-byte load) and their absmax (blocksize >= 32); per stage it builds the
//    block's bf16 codebook bf16(code[j] * absmax) in registers and decodes
//    8 K values per MFMA with v_perm byte lookups (nf4_decode.hpp), in the
//    order [0,2,4,6,1,3,5,7]; x is staged in LDS permuted the same way.
//  * x is double-buffered in LDS: stage s + 1's x and weights are loaded while
//    stage s's MFMAs run; one barrier per stage.
//  * LoRA: wave w also multiplies rows 32 w .. 32 w + 31 by A (one or two
//    16-rank column tiles; A is bf16, no decode).  After the K loop t goes to
//    LDS in bf16 and t . B[n, :] is one more MFMA per output tile (K = 32
//    ranks, ranks >= r zero).
//  * Output: the bf16 tile passes through LDS so every thread stores 16-byte
//    row chunks.
//  * Edges: rows >= M read row M - 1 and are not stored; columns >= N read
//    row N - 1 of W and are not stored; a last stage past K (K % 128 != 0)
//    stages zero x (its weight loads are clamped into the row).
//  * Workgroup -> tile: the dispatcher places workgroup i on XCD i mod 8; the
//    tiles, column tile by column tile, are cut into 8 equal runs and run x
//    goes to the ids = x mod 8, so the row tiles of a column tile read its
//    weights through one L2 and every XCD gets the same number of tiles.
#include <algorithm>
#include <type_traits>

#include "linear_parts.hpp"
#include "nf4_decode.hpp"

using namespace grpo;

namespace {

constexpr int GM_BM = 128;            // rows per workgroup
constexpr int GM_BN = 128;            // columns per workgroup
constexpr int GM_KS = 128;            // K values per stage
constexpr int GM_T = 256;             // threads (4 waves)
constexpr int GM_XS = GM_KS + 8;      // LDS row stride of a staged x stage (elements)
constexpr int GM_TS = 32 + 8;         // LDS row stride of t (elements)
constexpr int GM_OS = GM_BN + 8;      // LDS row stride of the output tile (elements)
constexpr int GM_RT = GM_BM / 16;     // row tiles per wave
constexpr int GM_MAX_R = 32;
constexpr size_t GM_LDS =
    (size_t)(2 * GM_BM * GM_XS + GM_BM * GM_TS) * 2;  // 79,872 bytes
static_assert(GM_BM * GM_OS <= 2 * GM_BM * GM_XS, "output tile reuses the x stages");
constexpr int GM_PS = GM_BN + 4;      // LDS row stride of a float32 partial-sum tile
static_assert(GM_BM * GM_PS * 2 <= 2 * GM_BM * GM_XS, "partial-sum tile reuses the x stages");

struct GemmArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  const float* absmax;
  const float* code16;
  int bs_shift;
  int64_t wrow0;         // weight row of output column 0 (of segment 0)
  // Up to 4 segments: consecutive column ranges [seg_end[s-1], seg_end[s]) of
  // one stacked weight and of y, each with its own bias and LoRA pair (the
  // q|k|v projections of one launch); seg_tile[s] = first column tile of
  // segment s (seg_tile[nseg..4] = NT).
  int nseg;
  int seg_end[MAXSEG];
  int seg_tile[MAXSEG + 1];
  const uint16_t* bias[MAXSEG];  // [N_s] or null
  const uint16_t* la[MAXSEG];    // [r][K] (r > 0)
  const uint16_t* lb[MAXSEG];    // [N_s][r] (r > 0)
  int r;
  float scaling;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int MT, NT;  // row and column tiles
  int nst;     // stages
  int kst;     // stages per K slice (gridDim.y slices)
  bool yvec;   // 16-byte stores of y rows (y aligned, ldy and N multiples of 8)
  bool lbvec;  // 16-byte loads of B rows (lb aligned, r % 8 == 0)
  // K split over gridDim.y slices: float32 partial sums part[slice][m][n]
  // (slice stride psl, row stride ldp) and, from column tile 0, the LoRA t
  // partials tpart[slice][m][16] (slice stride tsl); the epilogue then runs in
  // the finish kernel.  part == null: one slice, epilogue in this kernel.
  float* part;
  int64_t ldp, psl;
  float* tpart;  // segment s at tpart + s * tseg
  int64_t tsl, tseg;
  int silu_I;    // SILU kernels: I (y = act [M, I], row stride ldy)
};

// TC: LoRA rank tiles of 16 (0: no LoRA, 1: r <= 16, 2: r <= 32).  F16: x,
// the weight values, LoRA, bias and y in float16 instead of bf16 (the
// reference's float16 X_DTYPE / LORA_DTYPE, lora_forward.py:141-143, 745-749).
// SILU: the MLP's gate|up projection of the stacked [2I, K] weight (no bias,
// no LoRA) with act = bf16(bf16(silu(g)) * u) applied in the epilogue: the
// tile's columns are 64 gate columns j0 .. j0 + 63 (waves 0, 1) and the same
// 64 up columns (waves 2, 3), and y is act [M, I].
template <int TC, bool F16, bool SILU = false>
__global__ void __launch_bounds__(GM_T, 2) nf4_gemm_mfma(GemmArgs p) {
  constexpr bool LORA = TC > 0;
  static_assert(!SILU || (TC == 0 && !F16), "gate|up + SiLU: bf16, no LoRA");
  extern __shared__ __align__(16) uint16_t lds[];
  uint16_t* const ts = lds + 2 * GM_BM * GM_XS;  // t [128][GM_TS] bf16
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  // Tiles t = nt * MT + mt in order, in 8 contiguous runs of equal length
  // (+-1): run x goes to the workgroups with ids = x mod 8, which the
  // dispatcher places on one XCD, so the row tiles of a column tile share
  // that tile's weights through one L2 and every XCD gets the same work.
  const int b = blockIdx.x, run = b & 7, T = p.MT * p.NT;
  const int t = ((run * T) >> 3) + (b >> 3);
  if (t >= (((run + 1) * T) >> 3)) return;  // past the end of this run
  const int nt = t / p.MT, mt = t - nt * p.MT;
  // the segment of column tile nt (uniform per workgroup) and its columns
  const int seg = (nt >= p.seg_tile[1]) + (nt >= p.seg_tile[2]) + (nt >= p.seg_tile[3]);
  const int c0 = seg > 0 ? sel4(p.seg_end[0], p.seg_end[1], p.seg_end[2], p.seg_end[3],
                                seg - 1) : 0;
  const int N = sel4(p.seg_end[0], p.seg_end[1], p.seg_end[2], p.seg_end[3], seg) - c0;
  const uint16_t* const sbias = sel4(p.bias[0], p.bias[1], p.bias[2], p.bias[3], seg);
  const uint16_t* const sla = sel4(p.la[0], p.la[1], p.la[2], p.la[3], seg);
  const uint16_t* const slb = sel4(p.lb[0], p.lb[1], p.lb[2], p.lb[3], seg);
  const int lt = nt - sel4(p.seg_tile[0], p.seg_tile[1], p.seg_tile[2], p.seg_tile[3], seg);
  const int m0 = mt * GM_BM, n0 = lt * GM_BN;  // n0: column within the segment

  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];

  // x staging: thread (row r0 + 16 u, chunk c) for u < 8; 16 threads per row
  const int r0 = tid >> 4, c8 = 8 * (tid & 15);
  const uint16_t* xr[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) xr[u] = p.x + (int64_t)min(m0 + r0 + 16 * u, p.M - 1) * p.ldx;
  // weight rows of this lane's two column tiles
  const uint8_t* wr[2];
  int64_t we[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int n = min(n0 + 32 * wave + 16 * ct + ln, N - 1);
    if (SILU) {  // gate row j (waves 0, 1) or up row I + j (waves 2, 3)
      const int j = min(lt * (GM_BN / 2) + 32 * (wave & 1) + 16 * ct + ln, p.silu_I - 1);
      we[ct] = ((int64_t)(wave >> 1) * p.silu_I + j) * p.K;
    } else {
      we[ct] = (p.wrow0 + c0 + n) * p.K;
    }
    wr[ct] = p.w + we[ct] / 2;
  }
  // LoRA A rows: rank 16 tc + ln of this lane.  Ranks >= r read rank r - 1:
  // their t columns are finite and meet zero B entries, so they add nothing
  // (no select, which the compiler turns into a predicated load).
  const uint16_t* ar[LORA ? TC : 1];
#pragma unroll
  for (int tc = 0; tc < TC; ++tc) ar[tc] = sla + (int64_t)min(16 * tc + ln, p.r - 1) * p.K;

  uint4 xv[8];
  uint4 wv[2];
  float av[2];
  auto load_stage = [&](int st) __attribute__((always_inline)) {
    const int k0 = st * GM_KS;
    const int kx = min(k0 + c8, p.K - 8);
#pragma unroll
    for (int u = 0; u < 8; ++u) xv[u] = *reinterpret_cast<const uint4*>(xr[u] + kx);
    const int kc = min(k0 + 32 * lg, p.K - 32);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      wv[ct] = *reinterpret_cast<const uint4*>(wr[ct] + kc / 2);
      av[ct] = p.absmax[(we[ct] + kc) >> p.bs_shift];
    }
  };
  auto store_x = [&](int st) __attribute__((always_inline)) {
    uint16_t* buf = lds + (st & 1) * GM_BM * GM_XS;
    const bool kin = st * GM_KS + c8 < p.K;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      *reinterpret_cast<uint4*>(buf + (r0 + 16 * u) * GM_XS + c8) =
          kin ? deinterleave8(xv[u]) : make_uint4(0, 0, 0, 0);
  };

  f32x4_t acc[GM_RT][2];
#pragma unroll
  for (int rt = 0; rt < GM_RT; ++rt) acc[rt][0] = acc[rt][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  f32x4_t tacc[2][LORA ? TC : 1];  // [row tile of the wave's 32 rows][rank tile]
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int tc = 0; tc < TC; ++tc) tacc[i][tc] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int st0 = blockIdx.y * p.kst, st1 = min(p.nst, st0 + p.kst);
  load_stage(st0);
  store_x(st0);
  __syncthreads();
  for (int st = st0; st < st1; ++st) {
    // This stage's LoRA A loads go out before the next stage's prefetch (loads
    // retire in order) and are used after the stage's weight MFMAs.
    uint4 la4[LORA ? TC : 1][4];
    if (LORA) {
      const int kc = min(st * GM_KS + 32 * lg, p.K - 32);
#pragma unroll
      for (int tc = 0; tc < TC; ++tc)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          la4[tc][s] = *reinterpret_cast<const uint4*>(ar[tc] + kc + 8 * s);
    }
    const uint4 wc0 = wv[0], wc1 = wv[1];
    const float ac0 = av[0], ac1 = av[1];
    // The prefetch is unconditional (the last stage re-reads itself): after a
    // conditional load the compiler waits for every load with vmcnt(0).
    const bool more = st + 1 < st1;
    load_stage(min(st + 1, st1 - 1));
    // keep the loads here, ahead of this stage's MFMAs
    __builtin_amdgcn_sched_barrier(0);
    const uint16_t* buf = lds + (st & 1) * GM_BM * GM_XS + ln * GM_XS + 32 * lg;
    const Lut t0 = make_lut<F16>(code, ac0), t1 = make_lut<F16>(code, ac1);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      uint4 a[GM_RT];
#pragma unroll
      for (int rt = 0; rt < GM_RT; ++rt)
        a[rt] = *reinterpret_cast<const uint4*>(buf + rt * 16 * GM_XS + 8 * s);
      const uint4 b0 = decode8(word(wc0, s), t0);
      const uint4 b1 = decode8(word(wc1, s), t1);
#pragma unroll
      for (int rt = 0; rt < GM_RT; ++rt) {
        acc[rt][0] = mfma16x16x32_e<F16>(a[rt], b0, acc[rt][0]);
        acc[rt][1] = mfma16x16x32_e<F16>(a[rt], b1, acc[rt][1]);
      }
    }
    if (LORA) {
      // rows 32 w .. 32 w + 31 of this wave times the A ranks (ranks >= r zero)
      const uint16_t* tb = buf + 32 * wave * GM_XS;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint4 a0 = *reinterpret_cast<const uint4*>(tb + 8 * s);
        const uint4 a1 = *reinterpret_cast<const uint4*>(tb + 16 * GM_XS + 8 * s);
#pragma unroll
        for (int tc = 0; tc < TC; ++tc) {
          const uint4 lb = deinterleave8(la4[tc][s]);
          tacc[0][tc] = mfma16x16x32_e<F16>(a0, lb, tacc[0][tc]);
          tacc[1][tc] = mfma16x16x32_e<F16>(a1, lb, tacc[1][tc]);
        }
      }
    }
    if (more) store_x(st + 1);
    __syncthreads();
  }

  if (p.part) {
    // K slice: float32 partial sums (and column tile 0's LoRA t partials).
    // The tile passes through LDS (the x stages are free after the loop's last
    // barrier) so every thread stores 16-byte row chunks (N % 16 == 0 here).
    float* const ps = reinterpret_cast<float*>(lds);  // [128][GM_PS]
#pragma unroll
    for (int rt = 0; rt < GM_RT; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          ps[(rt * 16 + 4 * lg + q) * GM_PS + 32 * wave + 16 * ct + ln] = acc[rt][ct][q];
    __syncthreads();
    float* pp = p.part + blockIdx.y * p.psl + c0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int c = tid + GM_T * i, row = c >> 5, c4 = 4 * (c & 31);
      const int m = m0 + row, n = n0 + c4;
      if (m < p.M && n < N)
        *reinterpret_cast<float4*>(pp + (int64_t)m * p.ldp + n) =
            *reinterpret_cast<const float4*>(ps + row * GM_PS + c4);
    }
    if (LORA && lt == 0) {
      float* tp = p.tpart + blockIdx.y * p.tsl + seg * p.tseg;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int m = m0 + 32 * wave + 16 * i + 4 * lg + q;
          if (m < p.M) tp[(int64_t)m * 16 + ln] = tacc[i][0][q];
        }
    }
    return;
  }

  // ---- epilogue
  f32x4_t u[GM_RT][2];
  if (LORA) {
    // t rows 32 w + 16 i + 4 lg + q, ranks 16 tc + ln, rounded to bf16
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int tc = 0; tc < 2; ++tc)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          ts[(32 * wave + 16 * i + 4 * lg + q) * GM_TS + 16 * tc + ln] =
              tc < TC ? f2e<F16>(tacc[i][tc < TC ? tc : 0][q]) : (uint16_t)0;
    // B rows: ranks 8 lg .. 8 lg + 7 of column n (ranks >= r zero)
    uint4 bv[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      const int n = min(n0 + 32 * wave + 16 * ct + ln, N - 1);
      const uint16_t* br = slb + (int64_t)n * p.r;
      if (p.lbvec) {
        bv[ct] = 8 * lg < p.r ? *reinterpret_cast<const uint4*>(br + 8 * lg)
                              : make_uint4(0, 0, 0, 0);
      } else {
        uint32_t h[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = 8 * lg + j < p.r ? br[8 * lg + j] : 0u;
        bv[ct] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                            h[6] | (h[7] << 16));
      }
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < GM_RT; ++rt) {
      const uint4 tv = *reinterpret_cast<const uint4*>(ts + (rt * 16 + ln) * GM_TS + 8 * lg);
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
        u[rt][ct] = mfma16x16x32_e<F16>(tv, bv[ct], f32x4_t{0.f, 0.f, 0.f, 0.f});
    }
  }
  float bias[2] = {0.f, 0.f};
  if (sbias) {
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
      bias[ct] = e2f<F16>(sbias[min(n0 + 32 * wave + 16 * ct + ln, N - 1)]);
  }
  const float sc = round_e<F16>(p.scaling);
  // bf16 tile [128][GM_OS] in the x stage buffers (free after the loop's last barrier)
  uint16_t* os = lds;
#pragma unroll
  for (int rt = 0; rt < GM_RT; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v = round_e<F16>(acc[rt][ct][q]);
        if (sbias) v = round_e<F16>(v + bias[ct]);
        if (LORA) v = round_e<F16>(v + round_e<F16>(round_e<F16>(u[rt][ct][q]) * sc));
        os[(rt * 16 + 4 * lg + q) * GM_OS + 32 * wave + 16 * ct + ln] = f2e<F16>(v);
      }
  __syncthreads();
  if (SILU) {
    // act columns j0 .. j0 + 63: thread (row r0 + 32 i, 8 columns 8 (tid % 8)),
    // the gate values at tile columns 0..63, the up values at 64..127
    const int j0 = lt * (GM_BN / 2), rs = tid >> 3, cc = 8 * (tid & 7);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = rs + 32 * i, m = m0 + row;
      if (m >= p.M || j0 + cc >= p.silu_I) continue;
      const uint4 gv = *reinterpret_cast<const uint4*>(os + row * GM_OS + cc);
      const uint4 uv = *reinterpret_cast<const uint4*>(os + row * GM_OS + 64 + cc);
      const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float r2[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float g = h ? bf_hi(gw[q]) : bf_lo(gw[q]);
          const float u = h ? bf_hi(uw[q]) : bf_lo(uw[q]);
          r2[h] = round_bf(g * (1.f / (1.f + expf(-g)))) * u;  // as silu_mul_kernel
        }
        o[q] = pack_bf2(r2[0], r2[1]);
      }
      uint16_t* dst = p.y + (int64_t)m * p.ldy + j0 + cc;
      if (p.yvec) {
        *reinterpret_cast<uint4*>(dst) = make_uint4(o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[j] = (uint16_t)(o[j >> 1] >> (16 * (j & 1)));
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = r0 + 16 * i, m = m0 + row, n = n0 + c8;
    if (m >= p.M || n >= N) continue;
    const uint4 v = *reinterpret_cast<const uint4*>(os + row * GM_OS + c8);
    uint16_t* dst = p.y + (int64_t)m * p.ldy + c0 + n;
    if (p.yvec) {
      *reinterpret_cast<uint4*>(dst) = v;
    } else {
      const uint32_t h[4] = {v.x, v.y, v.z, v.w};
      for (int j = 0; j < 8 && n + j < N; ++j)
        dst[j] = (uint16_t)(h[j >> 1] >> (16 * (j & 1)));
    }
  }
}

// Epilogue of a K-split GEMM: y[m, n] from the partial sums, a workgroup per
// 16 rows x 64 columns, a thread per (row, four columns): every thread's
// partial sums go out at once (one memory round trip).  The LoRA t of the 16
// rows is summed once into LDS (slice order, as every consumer sums them) and
// the 64 columns' LoRA B rows are staged in LDS once (the per-row finish of
// the decode batches loads them for every row: 32 bytes of B per output).
constexpr int FR_ROWS = 16, FR_COLS = 64;

__global__ void __launch_bounds__(256) nf4_finish_rows(LinParts o, uint16_t* __restrict__ y,
                                                       int64_t ldy) {
  __shared__ float ts[FR_ROWS][MAXSEG * 16];
  __shared__ uint4 lbs[FR_COLS * 2];  // B rows (r == 16, 16-byte aligned): two halves per column
  const int tid = threadIdx.x;
  const int m0 = blockIdx.y * FR_ROWS, c0 = blockIdx.x * FR_COLS;
  const int rows = min(FR_ROWS, o.M - m0);
  const int row = tid >> 4, n = c0 + 4 * (tid & 15);
  const int m = m0 + row;
  Fetch4<> f;  // lin_fetch4 without the B rows (staged below)
  if (m < o.M && n < o.N) {
    const float4* p = reinterpret_cast<const float4*>(o.part + (int64_t)m * o.N + n);
    const int64_t stride = (int64_t)o.M * o.N / 4;
#pragma unroll
    for (int k = 0; k < MAX_SLICES; ++k)
      if (k < o.S) f.part[k] = p[k * stride];
    f.seg = lin_seg(o, n);
    f.nl = n - (f.seg > 0 ? sel_seg(o.seg_end, f.seg - 1) : 0);
    const uint16_t* bias = sel_seg(o.bias, f.seg);
    if (bias && o.bias_vec) f.bias = *reinterpret_cast<const uint2*>(bias + f.nl);
  }
  if (o.r > 0) {
    const int per_row = o.nseg * 4;
    const int64_t stride = (int64_t)o.nseg * o.M * 4;  // float4s per slice
    for (int i = tid; i < rows * per_row; i += 256) {
      const int rr = i / per_row, it = i - rr * per_row;
      const int seg = it >> 2, q = it & 3;
      const float4* p =
          reinterpret_cast<const float4*>(o.tpart + ((int64_t)seg * o.M + m0 + rr) * 16) + q;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int k = 0; k < o.S; ++k) {
        const float4 v = p[k * stride];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
      float* t = &ts[rr][seg * 16 + 4 * q];
      t[0] = round_bf(acc.x);
      t[1] = round_bf(acc.y);
      t[2] = round_bf(acc.z);
      t[3] = round_bf(acc.w);
    }
    if (o.lb_vec && tid < FR_COLS * 2) {
      const int col = min(c0 + (tid >> 1), o.N - 1);
      const int seg = lin_seg(o, col);
      const int nl = col - (seg > 0 ? sel_seg(o.seg_end, seg - 1) : 0);
      lbs[tid] = reinterpret_cast<const uint4*>(sel_seg(o.lb, seg) + (int64_t)nl * 16)[tid & 1];
    }
  }
  __syncthreads();
  if (m >= o.M || n >= o.N) return;
  if (o.r > 0 && o.lb_vec) {
#pragma unroll
    for (int j = 0; j < 8; ++j) f.lb[j] = lbs[8 * (tid & 15) + j];
  }
  float v[4];
  lin_finish4(o, ts[row], f, v);
  uint16_t* yr = y + (int64_t)m * ldy + n;
  if (aligned8(yr)) {
    *reinterpret_cast<uint2*>(yr) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) yr[c] = f2bf(v[c]);
  }
}

bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }


bool gemm_ok(int M, int N, int K, int r, int blocksize) {
  return M >= 1 && N >= 1 && K >= 32 && K % 32 == 0 && r >= 0 && r <= GM_MAX_R &&
         pow2(blocksize) && blocksize >= 32;
}

}  // namespace

namespace grpo {

bool nf4_gemm_ok(int M, int N, int K, int r, int blocksize) {
  return gemm_ok(M, N, K, r, blocksize);
}

GemmPlan nf4_gemm_plan(int M, int K, int r, int nseg, const int* seg_end) {
  const int nst = (int)cdiv(K, GM_KS);
  GemmPlan pl{1, nst, 0, 0};
  const int64_t mt = cdiv(M, GM_BM);
  int64_t tiles = 0;
  bool split_ok = r <= 16 && nseg >= 1 && nseg <= MAXSEG;
  for (int s = 0, start = 0; s < nseg; start = seg_end[s], ++s) {
    tiles += mt * cdiv(seg_end[s] - start, GM_BN);
    split_ok = split_ok && seg_end[s] % 16 == 0;
  }
  if (!split_ok || nst < 6) return pl;
  // Time model (us) of S K slices, from measurements on MI355X: a workgroup
  // stage (128 K values) takes about 2.2 us whatever the tile count (its loads'
  // latency), 512 workgroups run at once; a split adds the float32 partial
  // sums (written and read back, ~4 TB/s), the finish launch and, with LoRA,
  // the finish's per-output rank sums (~2 ns per 1000 outputs).
  const int N = seg_end[nseg - 1];
  const double outs = (double)M * N;
  auto est = [&](int S, int* kst, int* slices) {
    *kst = (int)cdiv(nst, S);
    *slices = (int)cdiv(nst, *kst);
    double t = (double)cdiv(tiles * *slices, 512) * *kst * 2.2;
    if (*slices > 1) t += *slices * outs * 8.0 / 4e6 + 4.0 + (r > 0 ? outs * 2e-6 : 0.0);
    return t;
  };
  double best = 0.0;
  for (int S = 1; S <= std::min(MAX_SLICES, nst / 3); ++S) {
    int kst, slices;
    const double t = est(S, &kst, &slices);
    if (S == 1 || t < best) {
      best = t;
      pl.S = slices;
      pl.kst = kst;
    }
  }
  if (pl.S > 1) {
    pl.part_bytes = (size_t)pl.S * M * N * 4;
    pl.tpart_bytes = r > 0 ? (size_t)pl.S * nseg * M * 16 * 4 : 0;
  }
  return pl;
}

int nf4_gemm_launch(const uint16_t* x, int64_t ldx, const uint8_t* w, int64_t wrow0,
                    const float* absmax, const float* code16, int blocksize,
                    const GemmSegs& sg, int r, float scaling, uint16_t* y, int64_t ldy, int M,
                    int K, hipStream_t st, const GemmSplit* split, bool f16) {
  if (M < 0 || K < 0 || r < 0 || wrow0 < 0) return einval("negative dimension");
  if (sg.nseg < 1 || sg.nseg > MAXSEG) return einval("nseg must be in [1, 4]");
  int NT = 0, prev = 0;
  for (int s = 0; s < sg.nseg; ++s) {
    if (sg.seg_end[s] <= prev) return einval("segment ends must increase");
    if (!gemm_ok(M, sg.seg_end[s] - prev, K, r, blocksize)) {
      set_error("shape not supported by the NF4 GEMM (K %% 32 == 0, r <= 32, power-of-two "
                "blocksize >= 32)");
      return GRPO_EUNSUPPORTED;
    }
    NT += (int)cdiv(sg.seg_end[s] - prev, GM_BN);
    prev = sg.seg_end[s];
  }
  const int N = prev;
  if (M == 0) return GRPO_OK;
  if (!x || !w || !absmax || !code16 || !y) return einval("null pointer");
  if (ldx < K || ldx % 8 != 0 || !aligned16(x)) return einval("x rows must be 16-byte aligned");
  if (!aligned16(w)) return einval("w must be 16-byte aligned");
  if (ldy < N) return einval("ldy smaller than N");
  GemmArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.w = w;
  a.absmax = absmax;
  a.code16 = code16;
  a.bs_shift = __builtin_ctz((unsigned)blocksize);
  a.wrow0 = wrow0;
  a.nseg = sg.nseg;
  a.yvec = aligned16(y) && ldy % 8 == 0;
  a.lbvec = r > 0 && r % 8 == 0;
  for (int s = 0, tile = 0; s < MAXSEG; ++s) {
    const bool on = s < sg.nseg;
    a.seg_end[s] = on ? sg.seg_end[s] : N;
    a.seg_tile[s] = on ? tile : NT;
    if (on) {
      const int ns = sg.seg_end[s] - (s > 0 ? sg.seg_end[s - 1] : 0);
      tile += (int)cdiv(ns, GM_BN);
      a.bias[s] = sg.bias[s];
      a.la[s] = r > 0 ? sg.la[s] : nullptr;
      a.lb[s] = r > 0 ? sg.lb[s] : nullptr;
      if (r > 0 && (!sg.la[s] || !sg.lb[s])) return einval("r > 0 needs lora_a and lora_b");
      if (r > 0 && !aligned16(sg.la[s])) return einval("lora_a must be 16-byte aligned");
      a.yvec = a.yvec && sg.seg_end[s] % 8 == 0;
      a.lbvec = a.lbvec && aligned16(sg.lb[s]);
    }
  }
  a.seg_tile[MAXSEG] = NT;
  a.r = r;
  a.scaling = scaling;
  a.y = y;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.MT = (int)cdiv(M, GM_BM);
  a.NT = NT;
  a.nst = (int)cdiv(K, GM_KS);
  a.kst = a.nst;
  unsigned slices = 1;
  if (split && split->S > 1) {
    if (r > 16) return einval("a K-split NF4 GEMM takes r <= 16");
    if (f16) return einval("a K-split NF4 GEMM is bf16 only");
    if (!split->part || (r > 0 && !split->tpart)) return einval("null partial-sum buffer");
    a.kst = split->kst;
    slices = (unsigned)split->S;
    if ((int64_t)(slices - 1) * a.kst >= a.nst) return einval("empty K slice");
    a.part = split->part;
    a.ldp = split->ldp;
    a.psl = split->psl;
    a.tpart = split->tpart;
    a.tsl = split->tsl;
    a.tseg = split->tseg;
  }
  const dim3 grid(8u * (unsigned)cdiv((int64_t)a.MT * a.NT, 8), slices);
  const int tc = r > 16 ? 2 : (r > 0 ? 1 : 0);
  int rc = GRPO_OK;
  auto go = [&](auto tag) {
    constexpr auto kern = decltype(tag)::value;
    if (!(rc = allow_dynamic_lds<kern, (int)GM_LDS>())) kern<<<grid, GM_T, GM_LDS, st>>>(a);
  };
  using KernT = void (*)(GemmArgs);
  if (f16) {
    if (tc == 2) go(std::integral_constant<KernT, nf4_gemm_mfma<2, true>>{});
    else if (tc == 1) go(std::integral_constant<KernT, nf4_gemm_mfma<1, true>>{});
    else go(std::integral_constant<KernT, nf4_gemm_mfma<0, true>>{});
  } else {
    if (tc == 2) go(std::integral_constant<KernT, nf4_gemm_mfma<2, false>>{});
    else if (tc == 1) go(std::integral_constant<KernT, nf4_gemm_mfma<1, false>>{});
    else go(std::integral_constant<KernT, nf4_gemm_mfma<0, false>>{});
  }
  return rc ? rc : launch_check("nf4_gemm_mfma");
}

int nf4_gemm_finish(const grpo_linear_parts_t* h, uint16_t* y, int64_t ldy, hipStream_t st) {
  LinParts o;
  if (int rc = make_parts(h, &o)) return rc;
  if (!y) return einval("null y");
  if (ldy < o.N) return einval("ldy smaller than N");
  nf4_finish_rows<<<dim3((unsigned)cdiv(o.N, FR_COLS), (unsigned)cdiv(o.M, FR_ROWS)), 256, 0,
                    st>>>(o, y, ldy);
  return launch_check("nf4_finish_rows");
}

bool nf4_gemm_silu_ok(int M, int I, int K, int blocksize) {
  return I >= 8 && I % 8 == 0 && gemm_ok(M, 2 * I, K, 0, blocksize);
}

int nf4_gemm_silu_launch(const uint16_t* x, int64_t ldx, const uint8_t* w, const float* absmax,
                         const float* code16, int blocksize, int I, int K, int M, uint16_t* act,
                         int64_t lda, hipStream_t st) {
  if (M < 0 || I < 0 || K < 0) return einval("negative dimension");
  if (M == 0 || I == 0) return GRPO_OK;
  if (!nf4_gemm_silu_ok(M, I, K, blocksize)) {
    set_error("shape not supported by the NF4 GEMM's gate|up SiLU form (I %% 8 == 0, K %% 32 "
              "== 0, power-of-two blocksize >= 32)");
    return GRPO_EUNSUPPORTED;
  }
  if (!x || !w || !absmax || !code16 || !act) return einval("null pointer");
  if (ldx < K || ldx % 8 != 0 || !aligned16(x)) return einval("x rows must be 16-byte aligned");
  if (!aligned16(w)) return einval("w must be 16-byte aligned");
  if (lda < I) return einval("lda smaller than I");
  GemmArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.w = w;
  a.absmax = absmax;
  a.code16 = code16;
  a.bs_shift = __builtin_ctz((unsigned)blocksize);
  a.nseg = 1;
  a.M = M;
  a.K = K;
  a.MT = (int)cdiv(M, GM_BM);
  a.NT = (int)cdiv(I, GM_BN / 2);
  for (int s = 0; s < MAXSEG; ++s) {
    a.seg_end[s] = 2 * I;
    a.seg_tile[s] = s == 0 ? 0 : a.NT;
  }
  a.seg_tile[MAXSEG] = a.NT;
  a.y = act;
  a.ldy = lda;
  a.yvec = aligned16(act) && lda % 8 == 0;
  a.nst = a.kst = (int)cdiv(K, GM_KS);
  a.silu_I = I;
  const dim3 grid(8u * (unsigned)cdiv((int64_t)a.MT * a.NT, 8));
  constexpr auto kern = nf4_gemm_mfma<0, false, true>;
  if (int rc = allow_dynamic_lds<kern, (int)GM_LDS>()) return rc;
  kern<<<grid, GM_T, GM_LDS, st>>>(a);
  return launch_check("nf4_gemm_mfma (gate|up SiLU)");
}

}  // namespace grpo

extern "C" int grpo_nf4_gemm_supported(int M, int N, int K, int r, int blocksize) {
  return gemm_ok(M, N, K, r, blocksize) ? 1 : 0;
}

namespace {

int gemm_one(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
             const float* code16, int blocksize, const void* bias, const void* lora_a,
             const void* lora_b, int r, float scaling, void* y, int64_t ldy, int M, int N, int K,
             grpo_stream_t stream, bool f16) {
  if (N < 0) return einval("negative dimension");
  if (N == 0) return GRPO_OK;
  GemmSegs sg{};
  sg.nseg = 1;
  sg.seg_end[0] = N;
  sg.bias[0] = static_cast<const uint16_t*>(bias);
  sg.la[0] = static_cast<const uint16_t*>(lora_a);
  sg.lb[0] = static_cast<const uint16_t*>(lora_b);
  return nf4_gemm_launch(static_cast<const uint16_t*>(x), ldx, w, 0, absmax, code16, blocksize,
                         sg, r, scaling, static_cast<uint16_t*>(y), ldy, M, K,
                         as_stream(stream), nullptr, f16);
}

}  // namespace

extern "C" int grpo_nf4_gemm(const void* x, int64_t ldx, const uint8_t* w, const float* absmax,
                             const float* code16, int blocksize, const void* bias,
                             const void* lora_a, const void* lora_b, int r, float scaling,
                             void* y, int64_t ldy, int M, int N, int K, grpo_stream_t stream) {
  return gemm_one(x, ldx, w, absmax, code16, blocksize, bias, lora_a, lora_b, r, scaling, y, ldy,
                  M, N, K, stream, false);
}

extern "C" int grpo_nf4_gemm_f16(const void* x, int64_t ldx, const uint8_t* w,
                                 const float* absmax, const float* code16, int blocksize,
                                 const void* bias, const void* lora_a, const void* lora_b, int r,
                                 float scaling, void* y, int64_t ldy, int M, int N, int K,
                                 grpo_stream_t stream) {
  return gemm_one(x, ldx, w, absmax, code16, blocksize, bias, lora_a, lora_b, r, scaling, y, ldy,
                  M, N, K, stream, true);
}
