// bf16 lm_head GEMV with fused per-tile argmax, and the device-side greedy
// advance of the decode step (src/triton_kernels/paged_kv.py:800-820 and
// :418-450 greedy branch; the row bookkeeping of :938, :978).
//
// lm_head: logits[m, v] = bf16(x[m, :] . W[v, :]) for the M rows of a decode
// step, W bf16 [V, K] (467 MB for Qwen2-1.5B: the largest single read of the
// step).  One wave = 16 vocabulary rows over all of K on
// v_mfma_f32_16x16x32_bf16 (A = x staged in LDS, B = W^T); W is streamed with
// 16-byte loads laid out so each load instruction covers 64 contiguous bytes
// of every row of the tile.  Each wave also reduces its 16 logits per row to (max, first
// index) and writes that pair, so the argmax over V needs only a small second
// pass instead of re-reading the logits.
#include <math.h>

#include <algorithm>

#include "common.hpp"
#include "decode_state.hpp"

using namespace grpo;

namespace {

constexpr int LM_KSTEP = 256;
// lm_head weights are read once per step: loaded with the non-temporal hint
// (see load_w in nf4_linear.hip).
#ifndef GRPO_LM_WAVES
#define GRPO_LM_WAVES 8
#endif
constexpr int LM_WAVES = GRPO_LM_WAVES;  // vocabulary tiles per workgroup (x staged once per workgroup)
constexpr int ADV_T = 1024;
constexpr size_t LM_LDS_MAX = 163840;  // gfx950: 160 KiB of LDS per workgroup


struct LmArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint16_t* w;
  int V, K, M, NT;
  uint16_t* logits;  // [M][ldl] or null
  int64_t ldl;
  float* pval;       // [M][NT]
  int* pidx;         // [M][NT]
  // x = RMSNorm(h) staged from h (x above) and per-group sums of squares
  // (NORM instantiation, M <= LM_WAVES rows, nG <= 256 groups per row)
  const float* nss;
  int nG;
  const uint16_t* nw;
  float neps;
  int tiled;  // W in the tile layout of lm_weight_tiles_kernel
};
constexpr int LM_NORM_MAX_GROUPS = 256;

// lm_head weight in tile order: the 16-byte operand of lane l for MFMA j of
// k-step ks of vocabulary tile t, W[16 t + (l % 16)][256 ks + 32 j + 8 (l / 16) ..
// + 7], sits at chunk ((t * K / 256 + ks) * 8 + j) * 64 + l, so each load
// instruction of a wave reads 1 KiB of contiguous memory (the row-major layout
// gives 16 separate 64-byte pieces per instruction: 89 against 73 us for a
// plain read of the 467 MB weight at the Qwen2-1.5B shape).
__global__ void __launch_bounds__(256) lm_weight_tiles_kernel(const uint16_t* __restrict__ w,
                                                              uint16_t* __restrict__ wt, int V,
                                                              int K) {
  const int64_t n = (int64_t)V * K / 8;
  const int KS = K / LM_KSTEP;
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < n;
       q += (int64_t)gridDim.x * 256) {
    const int l = (int)(q & 63), j = (int)((q >> 6) & 7);
    const int64_t tk = q >> 9;  // tile * KS + ks
    const int64_t t = tk / KS, ks = tk - t * KS;
    const int64_t row = 16 * t + (l & 15);
    const int64_t k = ks * LM_KSTEP + 32 * j + 8 * (l >> 4);
    reinterpret_cast<uint4*>(wt)[q] = *reinterpret_cast<const uint4*>(w + row * K + k);
  }
}

// Strictly better in the argmax order: larger value, or equal value at a
// smaller index (the first maximum).  NaN never wins.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// The tile's logits (bf16) and, per row, its (max, first index) pair: lane
// (n = ln, group lg) holds logits[m = mt*16 + 4*lg + q][tile*16 + ln].
template <int MT>
__device__ __forceinline__ void lm_epilogue(const LmArgs& p, int tile, int ln, int lg,
                                            const f32x4_t (&acc)[MT]) {
  const int v = tile * 16 + ln;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = mt * 16 + 4 * lg + q;
      const uint16_t b = f2bf(acc[mt][q]);
      float bv = bf2f(b);
      int bi = v;
      if (bv != bv) {  // NaN never wins
        bv = -INFINITY;
        bi = 0x7fffffff;
      }
      // (max, first index) over the 16 lanes of this lane group
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (better(ov, oi, bv, bi)) {
          bv = ov;
          bi = oi;
        }
      }
      if (m < p.M) {
        if (p.logits) p.logits[(int64_t)m * p.ldl + v] = b;
        if (ln == 0) {
          p.pval[(int64_t)m * p.NT + tile] = bv;
          p.pidx[(int64_t)m * p.NT + tile] = bi;
        }
      }
    }
}

template <int MT, bool NORM>
__global__ void __launch_bounds__(64 * LM_WAVES) lm_head_argmax_kernel(LmArgs p) {
  touch_kernargs<sizeof(LmArgs)>();
  extern __shared__ __align__(16) uint16_t xs[];  // [M][K + 8]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int tile = blockIdx.x * LM_WAVES + wave;
  const int xstride = p.K + 8;
  const int KS = p.K / LM_KSTEP;
  const bool live = tile < p.NT;

  // Lane (row ln, group lg) supplies k-slots 8*lg..8*lg+7 of each MFMA j as
  // elements 32*j + 8*lg + 0..7 of the k-step: one 16-byte load per MFMA, and
  // each load instruction reads 64 contiguous bytes of each of the wave's 16
  // rows (16 half-lines; the layout 64*lg + 8*j touched 64 lines, 16 bytes
  // each, and streamed W ~20 % slower).  x is read from LDS in the same order.
  const uint16_t* wrow = p.w + (int64_t)(live ? tile * 16 + ln : 0) * p.K + 8 * lg;
  const uint16_t* wtile = p.w + ((int64_t)(live ? tile : 0) * KS * 8 * 64 + lane) * 8;
  auto wsrc = [&](int ks, int j) __attribute__((always_inline)) {
    return p.tiled ? wtile + ((int64_t)ks * 8 + j) * 512 : wrow + ks * LM_KSTEP + 32 * j;
  };
  // The first k-step's W goes out before x is staged (W does not depend on x).
  uint4 w0[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) w0[j] = load_stream(wsrc(0, j));
  {
    const int chunks = p.K / 8, total = p.M * chunks;
    // after x in the dynamic LDS (a static array would lower the dynamic limit
    // that allow_dynamic_lds sets for every instantiation)
    float* sInv = reinterpret_cast<float*>(xs + p.M * xstride);
    if (NORM) {
      // wave w: 1 / rms of row w from its group sums (4 per lane, clamped
      // indexes, dropped in the sum)
      const float* ssr = p.nss + (int64_t)min(wave, p.M - 1) * p.nG;
      float v[LM_NORM_MAX_GROUPS / 64];
#pragma unroll
      for (int q = 0; q < LM_NORM_MAX_GROUPS / 64; ++q) v[q] = ssr[min(lane + 64 * q, p.nG - 1)];
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < LM_NORM_MAX_GROUPS / 64; ++q) ss += lane + 64 * q < p.nG ? v[q] : 0.f;
      ss = wave_sum_dpp(ss);
      if (lane == 0) sInv[wave] = 1.f / sqrtf(ss / (float)p.K + p.neps);
      __syncthreads();
    }
    for (int i = tid; i < total; i += 64 * LM_WAVES) {
      const int m = i / chunks, c = i - m * chunks;
      uint4 v = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + 8 * c);
      if (NORM) v = norm8(v, *reinterpret_cast<const uint4*>(p.nw + 8 * c), sInv[m]);
      *reinterpret_cast<uint4*>(xs + m * xstride + 8 * c) = v;
    }
  }
  __syncthreads();
  if (!live) return;

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = xs + min(mt * 16 + ln, p.M - 1) * xstride + 8 * lg;

  // One k-step at a time: more loads in flight per wave (double buffering)
  // measured slower here, the HBM stream already being saturated by the
  // number of resident waves.
  for (int ks = 0; ks < KS; ++ks) {
    uint4 w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      w[j] = ks == 0 ? w0[j] : load_stream(wsrc(ks, j));
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = mfma16x16x32(
            *reinterpret_cast<const uint4*>(xrow[mt] + ks * LM_KSTEP + 32 * j), w[j], acc[mt]);
  }

  lm_epilogue<MT>(p, tile, ln, lg, acc);
}

// Wide batches (x [M, K] beyond 160 KiB of LDS, e.g. Qwen2-7B at G = 64): one
// workgroup per CU, each wave owning up to TPW vocabulary tiles (wave w of the
// grid takes tiles w, w + waves, ...), their accumulators in registers.  x is
// staged in K chunks of KC columns, once per chunk per workgroup, and every
// wave streams the W rows of all its tiles over the chunk, the next 256-column
// step's W loads issued before the current step's MFMAs.  (Staging x once per
// tile instead -- one workgroup per 8 tiles, 1 per CU for LDS -- read x from
// L2 ~40 times per CU and left 8 waves per CU without loads in flight during
// each staging: 320 us at M = 64.)  At M = 64, V = 152064, K = 3584 it streams
// W at 5.5 TB/s from the tile order (198 us, the argmax included; 257 us from
// the row-major layout); hipBLASLt's GEMM alone takes 202 us, its logits then
// need an argmax launch (9.6 us).
constexpr int LM_WIDE_WAVES = 8;
constexpr int LM_WIDE_TPW = 5;     // tiles per wave: V <= 5 * 2048 * 16 = 163840

template <int MT>
__global__ void __launch_bounds__(64 * LM_WIDE_WAVES) lm_head_argmax_wide(LmArgs p, int KC) {
  touch_kernargs<sizeof(LmArgs)>();
  extern __shared__ __align__(16) uint16_t xs[];  // [M][KC + 8]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int gw = blockIdx.x * LM_WIDE_WAVES + wave, nw = gridDim.x * LM_WIDE_WAVES;
  const int ntiles = gw < p.NT ? (p.NT - gw + nw - 1) / nw : 0;  // this wave's tiles (<= TPW)
  const int xstride = KC + 8;
  const int KS = p.K / LM_KSTEP, kpc = KC / LM_KSTEP;
  f32x4_t acc[LM_WIDE_TPW][MT];
#pragma unroll
  for (int t = 0; t < LM_WIDE_TPW; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = xs + min(mt * 16 + ln, p.M - 1) * xstride + 8 * lg;
  // W of (tile slot t, k-step ks): rows of tile gw + t*nw, clamped into range
  // for a wave without that tile (its loads are then re-reads, never used);
  // MFMA j's operands are 32 j further (row-major) or 512 j (tile order:
  // lm_weight_tiles_kernel, 1 KiB of contiguous memory per load instruction)
  const int64_t wj = p.tiled ? 512 : 32;
  auto wptr = [&](int t, int ks) __attribute__((always_inline)) {
    const int tile = min(gw + min(t, max(ntiles - 1, 0)) * nw, p.NT - 1);
    return p.tiled ? p.w + (((int64_t)tile * KS + ks) * 512 + lane) * 8
                   : p.w + (int64_t)(tile * 16 + ln) * p.K + 8 * lg + ks * LM_KSTEP;
  };
  for (int c0 = 0; c0 < KS; c0 += kpc) {
    const int nks = min(kpc, KS - c0);
    const int chunks = nks * LM_KSTEP / 8, total = p.M * chunks;
    __syncthreads();  // every wave is done with the previous chunk
    for (int i = tid; i < total; i += 64 * LM_WIDE_WAVES) {
      const int m = i / chunks, c = i - m * chunks;
      *reinterpret_cast<uint4*>(xs + m * xstride + 8 * c) =
          *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + c0 * LM_KSTEP + 8 * c);
    }
    __syncthreads();
    if (ntiles == 0) continue;
    // (tile slot, k-step) items of this chunk in order, the next step's W in
    // flight while one is multiplied; the loads are unconditional (the item
    // past the last re-reads it), so every wait is exact.  (Two steps ahead,
    // with three register sets, measured slower: 268 against 257 us.)
    const int nitems = ntiles * nks;
    uint4 wr[2][8];
    auto load_item = [&](uint4 (&w)[8], int item) __attribute__((always_inline)) {
      const int q = min(item, nitems - 1);
      const uint16_t* wp = wptr(q / nks, c0 + q % nks);
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = load_stream(wp + wj * j);
    };
    load_item(wr[0], 0);
    for (int it = 0; it < nitems; it += 2) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int cur = it + h;
        if (cur >= nitems) break;
        load_item(wr[h ^ 1], cur + 1);
        const int t = cur / nks, ks = cur - t * nks;
#pragma unroll
        for (int ts = 0; ts < LM_WIDE_TPW; ++ts)
          if (ts == t)
#pragma unroll
            for (int j = 0; j < 8; ++j)
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                acc[ts][mt] = mfma16x16x32(
                    *reinterpret_cast<const uint4*>(xrow[mt] + ks * LM_KSTEP + 32 * j),
                    wr[h][j], acc[ts][mt]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < LM_WIDE_TPW; ++t)
    if (t < ntiles) lm_epilogue<MT>(p, gw + t * nw, ln, lg, acc[t]);
}

// Greedy token of row m from the per-tile (max, index) pairs, then the row's
// decode bookkeeping: record the token, advance the lengths, stop at EOS or the
// row's limit, and set the next step's append slot / attention length.
__global__ void __launch_bounds__(ADV_T) decode_advance_kernel(
    const float* __restrict__ pval, const int* __restrict__ pidx, int NT, int64_t* next_out,
    int64_t* tokens, int32_t* pos, int32_t* count, const int32_t* limit, uint8_t* active,
    const int64_t* eos, int64_t* generated, int64_t gen_ld, int32_t* append_pos,
    int32_t* attn_len) {
  touch_kernargs<14 * 8>();
  __shared__ float sv[ADV_T / 64];
  __shared__ int si[ADV_T / 64];
  const int m = blockIdx.x, tid = threadIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int t = tid; t < NT; t += ADV_T) {
    const float v = pval[(int64_t)m * NT + t];
    const int i = pidx[(int64_t)m * NT + t];
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid != 0) return;
  for (int w = 1; w < ADV_T / 64; ++w)
    if (better(sv[w], si[w], bv, bi)) {
      bv = sv[w];
      bi = si[w];
    }
  const int64_t g = bi == 0x7fffffff ? 0 : bi;
  if (next_out) next_out[m] = g;
  if (!tokens) return;
  advance_row(m, g, tokens, pos, count, limit, active, eos, generated, gen_ld, append_pos,
              attn_len);
}

}  // namespace

extern "C" size_t grpo_lm_head_workspace_bytes(int M, int V) {
  if (M <= 0 || V <= 0) return 0;
  return (size_t)M * cdiv(V, 16) * 8;
}

namespace {

struct LmNorm {
  const float* sumsq;
  int groups;
  const uint16_t* weight;
  float eps;
};

int run_lm_head(const void* x, int64_t ldx, const void* w, int V, int K, int M, void* logits,
                int64_t ld_logits, void* workspace, size_t workspace_bytes, hipStream_t st,
                const LmNorm* nrm, bool tiled = false);

}  // namespace

extern "C" int grpo_lm_head_weight_tiles(const void* w, int V, int K, void* w_tiles,
                                         grpo_stream_t stream) {
  if (V <= 0 || K <= 0 || V % 16 || K % LM_KSTEP)
    return einval("needs V % 16 == 0 and K % 256 == 0");
  if (!w || !w_tiles || !aligned16(w) || !aligned16(w_tiles))
    return einval("w and w_tiles must be non-null and 16-byte aligned");
  const int64_t n = (int64_t)V * K / 8;
  lm_weight_tiles_kernel<<<(unsigned)std::min<int64_t>(cdiv(n, 256), 8192), 256, 0,
                           as_stream(stream)>>>(static_cast<const uint16_t*>(w),
                                                static_cast<uint16_t*>(w_tiles), V, K);
  return launch_check("lm_weight_tiles");
}

extern "C" int grpo_lm_head_argmax_tiles(const void* x, int64_t ldx, const void* w_tiles, int V,
                                         int K, int M, void* logits, int64_t ld_logits,
                                         void* workspace, size_t workspace_bytes,
                                         grpo_stream_t stream) {
  return run_lm_head(x, ldx, w_tiles, V, K, M, logits, ld_logits, workspace, workspace_bytes,
                     as_stream(stream), nullptr, true);
}

extern "C" int grpo_lm_head_argmax_norm_tiles(const void* h, int64_t ldh, const float* sumsq,
                                              int groups, const void* norm_weight, float eps,
                                              const void* w_tiles, int V, int K, int M,
                                              void* logits, int64_t ld_logits, void* workspace,
                                              size_t workspace_bytes, grpo_stream_t stream) {
  if (M > LM_WAVES) return einval("the RMSNorm x source takes at most 8 rows");
  if (!sumsq || !norm_weight) return einval("null pointer");
  if (groups < 1 || groups > LM_NORM_MAX_GROUPS) return einval("groups must be in [1, 256]");
  if (!aligned16(norm_weight)) return einval("norm_weight must be 16-byte aligned");
  const LmNorm n{sumsq, groups, static_cast<const uint16_t*>(norm_weight), eps};
  return run_lm_head(h, ldh, w_tiles, V, K, M, logits, ld_logits, workspace, workspace_bytes,
                     as_stream(stream), &n, true);
}

extern "C" int grpo_lm_head_argmax(const void* x, int64_t ldx, const void* w, int V, int K, int M,
                                   void* logits, int64_t ld_logits, void* workspace,
                                   size_t workspace_bytes, grpo_stream_t stream) {
  return run_lm_head(x, ldx, w, V, K, M, logits, ld_logits, workspace, workspace_bytes,
                     as_stream(stream), nullptr);
}

extern "C" int grpo_lm_head_argmax_norm(const void* h, int64_t ldh, const float* sumsq,
                                        int groups, const void* norm_weight, float eps,
                                        const void* w, int V, int K, int M, void* logits,
                                        int64_t ld_logits, void* workspace,
                                        size_t workspace_bytes, grpo_stream_t stream) {
  if (M > LM_WAVES) return einval("the RMSNorm x source takes at most 8 rows");
  if (!sumsq || !norm_weight) return einval("null pointer");
  if (groups < 1 || groups > LM_NORM_MAX_GROUPS) return einval("groups must be in [1, 256]");
  if (!aligned16(norm_weight)) return einval("norm_weight must be 16-byte aligned");
  const LmNorm n{sumsq, groups, static_cast<const uint16_t*>(norm_weight), eps};
  return run_lm_head(h, ldh, w, V, K, M, logits, ld_logits, workspace, workspace_bytes,
                     as_stream(stream), &n);
}

namespace {

int run_lm_head(const void* x, int64_t ldx, const void* w, int V, int K, int M, void* logits,
                int64_t ld_logits, void* workspace, size_t workspace_bytes, hipStream_t st,
                const LmNorm* nrm, bool tiled) {
  if (M <= 0 || V <= 0 || K <= 0) return einval("bad lm_head dimensions");
  if (M > 64) return einval("lm_head argmax supports M <= 64 rows");
  if (V % 16 || K % LM_KSTEP) return einval("lm_head needs V % 16 == 0 and K % 256 == 0");
  if (!x || !w || !workspace) return einval("null pointer");
  if (ldx < K || ldx % 8 || !aligned16(x) || !aligned16(w))
    return einval("x and W must be 16-byte aligned with ldx >= K, ldx % 8 == 0");
  if (logits && ld_logits < V) return einval("ld_logits smaller than V");
  const size_t need = grpo_lm_head_workspace_bytes(M, V);
  if (workspace_bytes < need) {
    set_error("invalid argument: workspace of %zu bytes needed, %zu given", need,
              workspace_bytes);
    return GRPO_EWORKSPACE;
  }
  const size_t lds = (size_t)M * (K + 8) * 2 + (nrm ? LM_WAVES * sizeof(float) : 0);
  if (lds > LM_LDS_MAX && nrm) {
    set_error("lm_head: x [M, K] of the RMSNorm source does not fit in LDS");
    return GRPO_EUNSUPPORTED;
  }
  LmArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = static_cast<const uint16_t*>(w);
  a.V = V;
  a.K = K;
  a.M = M;
  a.NT = V / 16;
  a.logits = static_cast<uint16_t*>(logits);
  a.ldl = ld_logits;
  a.pval = static_cast<float*>(workspace);
  a.pidx = reinterpret_cast<int*>(a.pval + (size_t)M * a.NT);
  a.tiled = tiled ? 1 : 0;
  const dim3 grid((unsigned)cdiv(a.NT, LM_WAVES)), block(64 * LM_WAVES);
  if (lds > LM_LDS_MAX) {
    // x staged in K chunks (the widest multiple of 256 columns that fits), one
    // workgroup per CU, every tile of a wave accumulated in registers
    const int KC = (int)(((LM_LDS_MAX / (2 * (size_t)M)) - 8) / LM_KSTEP) * LM_KSTEP;
    if (KC < LM_KSTEP) return einval("lm_head: too many rows for one x chunk in LDS");
    const size_t clds = (size_t)M * (KC + 8) * 2;
    const int G = std::min((int)cdiv(a.NT, LM_WIDE_WAVES), 256);
    if (cdiv(a.NT, (int64_t)G * LM_WIDE_WAVES) > LM_WIDE_TPW)
      return einval("lm_head: vocabulary too large for the wide kernel");
    const dim3 wgrid((unsigned)G), wblock(64 * LM_WIDE_WAVES);
    if (M <= 16) {
      if (int rc = allow_dynamic_lds<lm_head_argmax_wide<1>, (int)LM_LDS_MAX>()) return rc;
      lm_head_argmax_wide<1><<<wgrid, wblock, clds, st>>>(a, KC);
    } else if (M <= 32) {
      if (int rc = allow_dynamic_lds<lm_head_argmax_wide<2>, (int)LM_LDS_MAX>()) return rc;
      lm_head_argmax_wide<2><<<wgrid, wblock, clds, st>>>(a, KC);
    } else {
      if (int rc = allow_dynamic_lds<lm_head_argmax_wide<4>, (int)LM_LDS_MAX>()) return rc;
      lm_head_argmax_wide<4><<<wgrid, wblock, clds, st>>>(a, KC);
    }
    return launch_check("lm_head_argmax_wide");
  }
  if (nrm) {
    a.nss = nrm->sumsq;
    a.nG = nrm->groups;
    a.nw = nrm->weight;
    a.neps = nrm->eps;
    if (int rc = allow_dynamic_lds<lm_head_argmax_kernel<1, true>, (int)LM_LDS_MAX>()) return rc;
    lm_head_argmax_kernel<1, true><<<grid, block, lds, st>>>(a);
  } else if (M <= 16) {
    if (int rc = allow_dynamic_lds<lm_head_argmax_kernel<1, false>, (int)LM_LDS_MAX>()) return rc;
    lm_head_argmax_kernel<1, false><<<grid, block, lds, st>>>(a);
  } else if (M <= 32) {
    if (int rc = allow_dynamic_lds<lm_head_argmax_kernel<2, false>, (int)LM_LDS_MAX>()) return rc;
    lm_head_argmax_kernel<2, false><<<grid, block, lds, st>>>(a);
  } else {
    if (int rc = allow_dynamic_lds<lm_head_argmax_kernel<4, false>, (int)LM_LDS_MAX>()) return rc;
    lm_head_argmax_kernel<4, false><<<grid, block, lds, st>>>(a);
  }
  return launch_check("lm_head_argmax");
}

}  // namespace

extern "C" int grpo_decode_advance(const void* lm_workspace, int M, int V, int64_t* next_tokens,
                                   int64_t* tokens, int32_t* pos, int32_t* count,
                                   const int32_t* limit, uint8_t* active, const int64_t* eos,
                                   int64_t* generated, int64_t gen_ld, int32_t* append_pos,
                                   int32_t* attn_len, grpo_stream_t stream) {
  if (M <= 0 || V <= 0 || V % 16) return einval("bad advance dimensions");
  if (!lm_workspace) return einval("null workspace");
  if (tokens && (!pos || !count || !limit || !active || !eos || !append_pos || !attn_len))
    return einval("null row state");
  if (generated && gen_ld <= 0) return einval("gen_ld must be > 0");
  const int NT = V / 16;
  const float* pval = static_cast<const float*>(lm_workspace);
  const int* pidx = reinterpret_cast<const int*>(pval + (size_t)M * NT);
  decode_advance_kernel<<<dim3(M), ADV_T, 0, as_stream(stream)>>>(
      pval, pidx, NT, next_tokens, tokens, pos, count, limit, active, eos, generated, gen_ld,
      append_pos, attn_len);
  return launch_check("decode_advance");
}
