// down_proj + residual add of the decode step (M <= 8 rows) for gfx950: the
// folded NF4 linear (nf4_fold_residual) and its C entry points.
//
// This file is compiled with the max-ILP machine scheduler
// (-amdgpu-sched-strategy=max-ilp, set by the build): the kernel runs one
// workgroup of 8 waves per CU (two waves per SIMD), so the default scheduler's
// register savings for occupancy buy nothing, while the ILP schedule overlaps
// more of each item's decode with its MFMAs (config 3 down_proj 7.65 -> 7.30
// us per launch).  The weight format and the decode are those of nf4_linear.hip
// (nf4_decode.hpp); x arrives in the fold tile layout its gate|up kernel
// writes (fold_tile_index there).
#include "linear_parts.hpp"
#include "nf4_decode.hpp"

using namespace grpo;

namespace {

// ------------------------------ down_proj + residual add for M <= 8 rows --
//
// h_out[m, n] = bf16(residual[m, n] + bf16(x[m, :] . W[n, :])) (NF4 W, no LoRA,
// no bias: the MLP's down_proj and the decoder layer's residual add,
// modeling_qwen2 Qwen2DecoderLayer.forward), and for the next layer's input
// RMSNorm sumsq[m, g] = sum of h_out[m, n]^2 over the 8 columns n of group g
// (float32).  The whole K of a column group runs in one workgroup, so the
// finished rows leave this kernel and the norm needs no launch of its own: the
// next q|k|v kernel stages RMSNorm(h) from h and these sums (X_NORM).
//
// K is folded into the MFMA's rows.  With M <= 8, rows 8..15 of the A operand
// carry the same x rows over a second K range and B columns 8..15 the same 8
// weight columns over that range, so one v_mfma_f32_16x16x32_bf16 covers 8
// columns x 64 K values (the cross quadrants D[0..7][8..15] and D[8..15][0..7]
// are discarded): every lane decodes weights that are used, and a workgroup
// needs 8 columns, not 16, which doubles the workgroups that share the decode.
// Lane (ln, lg) holds column 8t + (ln & 7), x row (ln & 7) and K half
// ln >> 3: in item i (512 K values) its A and B both cover the 64-value block
// i*512 + 256*(ln >> 3) + 64*lg over 8 MFMAs (one LUT per item).  x arrives in
// the fold tile layout (fold_tile_index, written so by the gate|up kernel),
// where the 64 lanes' A operands of one MFMA are one contiguous 1 KiB block,
// or natural [M][ldx] (16 bytes per lane from 64 different lines, permuted
// here: the slow form, for callers without the tile layout).  Waves take
// items w, w + W, ...; the D quadrants of all waves are summed through LDS in
// a fixed order.
struct FoldArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  const float* absmax;
  const float* code16;
  int bs_shift;
  const uint16_t* residual;  // may be null (h_out = y)
  int64_t ldr;
  uint16_t* h_out;
  int64_t ldh;
  float* sumsq;  // [M][G], G = N / 8
  int M, N, K, G;
};

constexpr int FOLD_W = 8;          // waves per workgroup
constexpr int FOLD_ITEM = 512;     // K values of one item (two 256-value halves)
constexpr int FOLD_IPW_MAX = 4;    // items per wave (all loads in flight at once): K <= 16384

template <int IPW, bool TILES>
__global__ void __launch_bounds__(64 * FOLD_W) nf4_fold_residual(FoldArgs p) {
  __shared__ float red[FOLD_W][2][8][8];  // [wave][K half][row][column]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int c = ln & 7, half = ln >> 3;
  const int t = blockIdx.x;
  const int n = 8 * t + c;
  const int items = (p.K + FOLD_ITEM - 1) / FOLD_ITEM;
  const bool tail = p.K % FOLD_ITEM != 0;  // the last item has its first half only

  // Loads: the epilogue's residual value (wave 0, predicated: issued first,
  // so it makes no later wait conservative), the codebook (scalar), then per
  // item the weights, the absmax and x, unconditional (items past the wave's
  // last re-read the last one; the tail item's missing half re-reads its
  // first half, and its x is zeroed before use).
  const int em = tid >> 3, ec = tid & 7;  // epilogue output (row, column) of threads < 64
  uint16_t rres = 0;
  if (tid < 64 && p.residual && em < p.M) rres = p.residual[(int64_t)em * p.ldr + 8 * t + ec];
  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];
  const uint8_t* wrow = p.w + (int64_t)n * (p.K / 2);
  const uint16_t* xrow = p.x + (int64_t)min(c, p.M - 1) * p.ldx;
  uint4 wv[2 * IPW], xv[8 * IPW];
  float av[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int it = min(wave + FOLD_W * i, items - 1);
    int kb = it * FOLD_ITEM + 256 * half + 64 * lg;
    if (kb >= p.K) kb -= 256;
    const uint4* wp = reinterpret_cast<const uint4*>(wrow + kb / 2);
    wv[2 * i] = load_w<true>(wp);
    wv[2 * i + 1] = load_w<true>(wp + 1);
    av[i] = p.absmax[((int64_t)n * p.K + kb) >> p.bs_shift];
    if (TILES) {
      const uint4* xp = reinterpret_cast<const uint4*>(p.x) + (int64_t)it * 8 * 64 + lane;
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[8 * i + j] = xp[j * 64];
    } else {
      const uint4* xp = reinterpret_cast<const uint4*>(xrow + kb);
#pragma unroll
      for (int j = 0; j < 8; ++j) xv[8 * i + j] = xp[j];
    }
    // item i's loads stay ahead of item i + 1's, so its decode waits for them only
    __builtin_amdgcn_sched_barrier(0);
  }

  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const int my_items = (items - wave + FOLD_W - 1) / FOLD_W;  // may be 0
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    if (i >= my_items) break;
    // The tail item's missing half: in the tile layout its x slots (columns
    // >= K) are zero, in the natural layout it re-read the first half, whose
    // x is dropped here by a select (overwriting the loaded registers would
    // make the compiler wait for every load in flight).
    const bool drop = !TILES && tail && wave + FOLD_W * i == items - 1 && half;
    const Lut lt = make_lut(code, av[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      uint4 a = TILES ? xv[8 * i + j] : deinterleave8(xv[8 * i + j]);
      if (!TILES) a = drop ? make_uint4(0, 0, 0, 0) : a;
      acc = mfma16x16x32(a, decode8(word(wv[2 * i + (j >> 2)], j & 3), lt), acc);
    }
  }
  // lane (ln, lg) holds D[4*lg + q][ln]: rows 0..7 of columns 0..7 (lg < 2,
  // ln < 8) are the first K half, rows 8..15 of columns 8..15 (lg >= 2,
  // ln >= 8) the second
  if ((lg >> 1) == half) {
#pragma unroll
    for (int q = 0; q < 4; ++q) red[wave][half][4 * (lg & 1) + q][c] = acc[q];
  }
  __syncthreads();
  if (tid < 64) {
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < FOLD_W; ++w) sum += red[w][0][em][ec] + red[w][1][em][ec];
    const float y = round_bf(sum);
    float hv = 0.f;
    if (em < p.M) {
      hv = p.residual ? round_bf(y + bf2f(rres)) : y;
      p.h_out[(int64_t)em * p.ldh + 8 * t + ec] = f2bf(hv);
    }
    float sq = hv * hv;
    sq += __shfl_xor(sq, 1);
    sq += __shfl_xor(sq, 2);
    sq += __shfl_xor(sq, 4);
    if (ec == 0 && em < p.M) p.sumsq[(int64_t)em * p.G + t] = sq;
  }
}

// Shape support of nf4_fold_residual.
bool fold_ok(int M, int N, int K, int blocksize) {
  if (M < 1 || M > 8 || N <= 0 || N % 8 || K < KSTEP || K % KSTEP) return false;
  if (blocksize < 64 || (blocksize & (blocksize - 1))) return false;
  const int items = (K + FOLD_ITEM - 1) / FOLD_ITEM;
  return (items + FOLD_W - 1) / FOLD_W <= FOLD_IPW_MAX;
}

}  // namespace

extern "C" size_t grpo_fold_tiles_elements(int K) {
  return K > 0 ? (size_t)((K + FOLD_ITEM - 1) / FOLD_ITEM) * FOLD_ITEM * 8 : 0;
}

extern "C" int grpo_nf4_linear_residual_supported(int M, int N, int K, int blocksize) {
  return fold_ok(M, N, K, blocksize) ? 1 : 0;
}

extern "C" int grpo_nf4_linear_residual(const void* x, int64_t ldx, int x_tiles,
                                        const uint8_t* w, const float* absmax,
                                        const float* code16, int blocksize, int N, int K, int M,
                                        const void* residual, int64_t ldr, void* h_out,
                                        int64_t ldh, float* sumsq, grpo_stream_t stream) {
  if (!fold_ok(M, N, K, blocksize)) {
    set_error("shape not supported by the folded NF4 linear (M <= 8, N %% 8 == 0, "
              "K %% 256 == 0, K <= 16384)");
    return GRPO_EUNSUPPORTED;
  }
  if (!x || !w || !absmax || !code16 || !h_out || !sumsq) return einval("null pointer");
  if ((!x_tiles && (ldx < K || ldx % 8)) || !aligned16(x) || !aligned16(w))
    return einval("x and w must be 16-byte aligned with ldx >= K, ldx % 8 == 0");
  if (ldh < N || (residual && ldr < N)) return einval("ldh / ldr smaller than N");
  FoldArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = w;
  a.absmax = absmax;
  a.code16 = code16;
  a.bs_shift = __builtin_ctz((unsigned)blocksize);
  a.residual = static_cast<const uint16_t*>(residual);
  a.ldr = ldr;
  a.h_out = static_cast<uint16_t*>(h_out);
  a.ldh = ldh;
  a.sumsq = sumsq;
  a.M = M;
  a.N = N;
  a.K = K;
  a.G = N / 8;
  const int ipw = ((K + FOLD_ITEM - 1) / FOLD_ITEM + FOLD_W - 1) / FOLD_W;
  const dim3 grid((unsigned)(N / 8)), block(64 * FOLD_W);
  hipStream_t st = as_stream(stream);
  switch (ipw * 2 + (x_tiles ? 1 : 0)) {
#define FOLD_CASE(IPW)                                                          \
  case IPW * 2: nf4_fold_residual<IPW, false><<<grid, block, 0, st>>>(a); break; \
  case IPW * 2 + 1: nf4_fold_residual<IPW, true><<<grid, block, 0, st>>>(a); break;
    FOLD_CASE(1) FOLD_CASE(2) FOLD_CASE(3) FOLD_CASE(4)
#undef FOLD_CASE
    default:
      return einval("folded NF4 linear: no instantiation");
  }
  return launch_check("nf4_fold_residual");
}
