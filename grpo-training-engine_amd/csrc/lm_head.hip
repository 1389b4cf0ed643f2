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

namespace {

// ------------------------------------------------ screened greedy argmax --
//
// The greedy token of a decode row needs only the first index of the largest
// bf16 logit, not every logit.  The screened form reads an int8 copy of W (half
// the bytes of the bf16 weight) to bound every logit, then recomputes exactly,
// with the arithmetic of lm_head_argmax_kernel, only the 16-row vocabulary
// tiles that can hold the maximum; the token is the one the full bf16 pass
// gives, bit for bit.
//
// Setup (lm_q8_kernel, once per weight): per vocabulary row v,
// scale_v = fl(max_k |W[v, k]| / 127), q[v, k] = rint(W[v, k] / scale_v) in
// [-127, 127] (stored as q + 128), R_v = ||W[v, :] - scale_v q[v, :]||_2
// (float64, rounded up to float32).
//
// Screen (lm_screen_kernel): with x the bf16 row of the exact pass and x16 its
// float16 rounding, zhat = fl(scale_v * sum_k x16[k] q[v, k]) (float16 MFMA,
// exact products, float32 sums).  The exact pass's float32 logit z~ then
// satisfies |z~ - zhat| <= e with
//   e = ||x||_2 R_v                                  (weight rounding, Cauchy-Schwarz)
//     + scale_v * 127 * ||x - x16||_1                (x16 rounding, |q| <= 127)
//     + scale_v * 127 * g * (||x||_1 + ||x16||_1)    (float32 sums of both passes)
//     + relative slack for the products and sums that form zhat and e,
// g = K * 2^-24 * 1.01 (the worst-case error factor of a float32 sum of K
// terms in any order).  Per tile and row the kernel writes the largest
// zhat + e, and per workgroup and row the largest zhat - e.
//
// Exact pass (lm_exact_advance_kernel): LB = the largest zhat - e of the row is
// at most its largest logit, so the winning bf16 value is at least bf16(LB),
// whose rounding interval starts above LB - |LB| 2^-6.  A tile whose largest
// zhat + e is below that threshold cannot hold a logit that rounds to the
// winning value; every other tile is recomputed exactly and the row's token is
// the first index of the maximum over them.  Non-finite bounds (NaN or
// infinite x or W, x beyond the float16 range) make every tile a candidate;
// an all-zero x does too (every bound is 0).

constexpr int SC_W = 16;         // waves per workgroup of the screen (one workgroup per CU)
constexpr int SC_GRID = 256;     // workgroups of the screen (at most one per tile)
constexpr int EX_WAVES = 8;      // waves per workgroup of the exact pass
constexpr int EX_C = 15;         // workgroups per row of the exact pass (xcd_arrive: <= 15)
constexpr int EX_CNT_STRIDE = 32; // ints between two rows' arrival counters
constexpr int EX_PASSES = 32;    // candidate-scan passes of 64 EX_WAVES tiles: NT <= 16384

__device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : fmaxf(a, b);
}

// bf16 bits of the smallest bf16 value >= f (an upper bound kept in 16 bits;
// NaN stays NaN, +-inf stay): a positive value with dropped bits rounds its
// magnitude up, a negative one truncates toward zero.
__device__ __forceinline__ uint32_t bf16_up(float f) {
  const uint32_t u = __float_as_uint(f);
  if (f != f) return 0x7FC0u;
  return (u >> 16) + ((u & 0xFFFFu) != 0u && f > 0.f ? 1u : 0u);
}

// One wave per vocabulary row; each lane handles 8 consecutive k per step
// (one 8-byte piece of the screening tile order).
__global__ void __launch_bounds__(256) lm_q8_kernel(const uint16_t* __restrict__ w,
                                                    uint8_t* __restrict__ wq,
                                                    float* __restrict__ scale,
                                                    float* __restrict__ rnorm, int V, int K) {
  const int lane = threadIdx.x & 63;
  const int64_t v = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (v >= V) return;
  const uint16_t* wr = w + v * K;
  const int KS = K / LM_KSTEP, pieces = K / 8;
  float amax = 0.f;
  bool bad = false;
  for (int c = lane; c < pieces; c += 64) {
    const uint4 u = *reinterpret_cast<const uint4*>(wr + 8 * c);
    const uint32_t d[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = fabsf(bf_lo(d[i])), b = fabsf(bf_hi(d[i]));
      bad |= !(a <= 3.4e38f) || !(b <= 3.4e38f);
      amax = fmaxf(amax, fmaxf(a, b));
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, o));
    bad = bad || __shfl_xor((int)bad, o);
  }
  const float sc = bad ? __builtin_nanf("") : amax / 127.f;
  const int64_t t = v >> 4, ln = v & 15;
  double rr = 0.0;
  for (int c = lane; c < pieces; c += 64) {
    const uint4 u = *reinterpret_cast<const uint4*>(wr + 8 * c);
    const uint32_t d[4] = {u.x, u.y, u.z, u.w};
    uint32_t b[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = (i & 1) ? bf_hi(d[i >> 1]) : bf_lo(d[i >> 1]);
      float q = sc > 0.f ? rintf(x / sc) : 0.f;
      q = fminf(fmaxf(q, -127.f), 127.f);
      if (bad) q = 0.f;
      const double r = (double)x - (double)sc * (double)q;
      rr += bad ? 0.0 : r * r;
      b[i >> 2] |= (uint32_t)((int)q + 128) << (8 * (i & 3));
    }
    const int k0 = 8 * c, ks = k0 / LM_KSTEP, r0 = k0 % LM_KSTEP;
    const int jj = r0 / 64, h = (r0 % 64) / 32, lg = (r0 % 32) / 8;
    const int64_t off = ((((t * KS + ks) * 4 + jj) * 64 + lg * 16 + ln) * 16) + 8 * h;
    *reinterpret_cast<uint2*>(wq + off) = make_uint2(b[0], b[1]);
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) rr += __shfl_xor(rr, o);
  if (lane == 0) {
    const double R = sqrt(rr);
    float rf = (float)R;
    if ((double)rf < R) rf = nextafterf(rf, INFINITY);
    scale[v] = sc;
    rnorm[v] = bad ? __builtin_nanf("") : rf;
  }
}

// Eight stored bytes q + 128 -> eight float16 q: the bytes become the low
// mantissa bytes of float16 0x6400 (1024 + u, exact), then 1152 is subtracted
// (packed float16, exact).
__device__ __forceinline__ uint4 q8_to_f16(uint32_t lo, uint32_t hi) {
  typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
  const h2_t off = {(_Float16)-1152.f, (_Float16)-1152.f};
  auto cv = [&](uint32_t d, uint32_t sel) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, perm(0x64646464u, d, sel)) + off);
  };
  return make_uint4(cv(lo, 0x04010400u), cv(lo, 0x04030402u), cv(hi, 0x04010400u),
                    cv(hi, 0x04030402u));
}

struct ScreenArgs {
  LmArgs lm;         // x source (NORM: h, sums of squares, norm weight), V, K, M, NT
  const uint4* wq;   // q + 128, chunk ((t * K / 256 + s) * 4 + jj) * 64 + l (16 bytes:
                     // W[16 t + l % 16][256 s + 64 jj + 8 (l / 16) + 0..7] and + 32)
  const float* scale;
  const float* rnorm;
  float* ub;         // [M][NT]: largest zhat + e of the tile
  float* lbw;        // [M][nwg]: largest zhat - e of the workgroup
  uint16_t* uv;      // [V][8]: zhat + e of every vocabulary row, rows m < M, bf16 rounded up
  int nwg;
};

// x of the exact pass staged into xs [M][K + 8] (bf16) exactly as
// lm_head_argmax_kernel stages it (the same values, element for element):
// with NORM, x[m, k] = bf16(bf16(h[m, k] inv[m]) w[k]), inv[m] =
// 1 / sqrt(sum of the row's group sums / K + eps), computed by wave m.  Also
// writes the float16 rounding into x16 when it is non-null.
template <bool NORM>
__device__ __forceinline__ void lm_stage(const LmArgs& p, uint16_t* xs, uint16_t* x16, float* sInv,
                                         int nth) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int xstride = p.K + 8;
  const int chunks = p.K / 8, total = p.M * chunks;
  if (NORM) {
    if (wave < p.M) {
      const float* ssr = p.nss + (int64_t)wave * p.nG;
      float v[LM_NORM_MAX_GROUPS / 64];
#pragma unroll
      for (int q = 0; q < LM_NORM_MAX_GROUPS / 64; ++q) v[q] = ssr[min(lane + 64 * q, p.nG - 1)];
      float ss = 0.f;
#pragma unroll
      for (int q = 0; q < LM_NORM_MAX_GROUPS / 64; ++q) ss += lane + 64 * q < p.nG ? v[q] : 0.f;
      ss = wave_sum_dpp(ss);
      if (lane == 0) sInv[wave] = 1.f / sqrtf(ss / (float)p.K + p.neps);
    }
    __syncthreads();
  }
  for (int i = tid; i < total; i += nth) {
    const int m = i / chunks, c = i - m * chunks;
    uint4 v = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + 8 * c);
    if (NORM) v = norm8(v, *reinterpret_cast<const uint4*>(p.nw + 8 * c), sInv[m]);
    *reinterpret_cast<uint4*>(xs + m * xstride + 8 * c) = v;
    if (x16) {
      const uint32_t d[4] = {v.x, v.y, v.z, v.w};
      uint32_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) o[q] = pack_h2(bf_lo(d[q]), bf_hi(d[q]));
      *reinterpret_cast<uint4*>(x16 + m * xstride + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

template <bool NORM>
__global__ void __launch_bounds__(64 * SC_W) lm_screen_kernel(ScreenArgs s) {
  touch_kernargs<sizeof(ScreenArgs)>();
  const LmArgs& p = s.lm;
  extern __shared__ __align__(16) uint16_t xs[];  // x [M][K + 8], x16 [M][K + 8], floats
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int xstride = p.K + 8;
  const int KS = p.K / LM_KSTEP;
  uint16_t* x16 = xs + p.M * xstride;
  float* fl = reinterpret_cast<float*>(x16 + p.M * xstride);
  float* sInv = fl;           // [8]
  float* sA = fl + 8;         // [8] ||x||_2, rounded up
  float* sB = fl + 16;        // [8] the scale_v coefficient of e
  float* sL = fl + 24;        // [SC_W][8]
  // workgroup b takes tiles [b NT / G, (b + 1) NT / G) (one workgroup per CU,
  // equal shares within one tile); wave w takes tiles tb + w, tb + w + SC_W, ...
  const int G = gridDim.x;
  const int tb = (int)((int64_t)blockIdx.x * p.NT / G);
  const int te = (int)((int64_t)(blockIdx.x + 1) * p.NT / G);
  const int ntw = te - tb > wave ? (te - tb - wave + SC_W - 1) / SC_W : 0;  // tiles of this wave
  // item i = (tile tb + wave + SC_W (i / KS), k-step i % KS); items past the
  // wave's last re-read its first (unconditional loads: exact waits)
  const int nitems = ntw * KS;
  auto wptr = [&](int i) __attribute__((always_inline)) {
    const int it = nitems > 0 ? min(i, nitems - 1) : 0;
    const int t = min(tb + wave + SC_W * (it / KS), p.NT - 1), ks = it % KS;
    return s.wq + ((int64_t)(t * KS + ks) * 4) * 64 + lane;
  };
  uint4 wc[4];
  {
    const uint4* q = wptr(0);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) wc[jj] = load_stream(q + 64 * jj);
  }
  lm_stage<NORM>(p, xs, x16, sInv, 64 * SC_W);
  __syncthreads();
  if (wave < p.M) {
    // row `wave`: ||x||_2, ||x||_1, ||x16||_1, ||x - x16||_1 (float32 sums; the
    // margins below cover their rounding)
    float ss = 0.f, l1 = 0.f, l1h = 0.f, d = 0.f;
    for (int k = lane; k < p.K; k += 64) {
      const float a = bf2f(xs[wave * xstride + k]), b = h2f(x16[wave * xstride + k]);
      ss += a * a;
      l1 += fabsf(a);
      l1h += fabsf(b);
      d += fabsf(a - b);
    }
    ss = wave_sum_dpp(ss);
    l1 = wave_sum_dpp(l1);
    l1h = wave_sum_dpp(l1h);
    d = wave_sum_dpp(d);
    if (lane == 0) {
      const float g = (float)p.K * 0x1p-24f * 1.01f;
      sA[wave] = sqrtf(ss * (1.f + 0x1p-10f)) * (1.f + 0x1p-10f);
      sB[wave] = (127.f * d + 127.f * g * (l1 + l1h)) * (1.f + 0x1p-10f);
    }
  }
  __syncthreads();
  const uint16_t* xrow = x16 + min(ln, p.M - 1) * xstride + 8 * lg;
  float Lw[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  float sc = 0.f, rn = 0.f;
  // item i multiplies buffer (i & 1) while item i + 1's loads fill the other
  // (two named buffers: a register copy between them would wait for the loads)
  auto item = [&](int i, const uint4 (&w)[4]) __attribute__((always_inline)) {
    const int ti = i / KS, ks = i - ti * KS, tile = tb + wave + SC_W * ti;
    if (ks == 0) {
      const int v = min(tile, p.NT - 1) * 16 + ln;
      sc = s.scale[v];
      rn = s.rnorm[v];
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const uint16_t* xa = xrow + ks * LM_KSTEP + 64 * jj;
      acc = mfma16x16x32_e<true>(*reinterpret_cast<const uint4*>(xa), q8_to_f16(w[jj].x, w[jj].y),
                                 acc);
      acc = mfma16x16x32_e<true>(*reinterpret_cast<const uint4*>(xa + 32),
                                 q8_to_f16(w[jj].z, w[jj].w), acc);
    }
    if (ks == KS - 1) {
      // lane (n = ln, group lg) holds sum_k x16[m][k] q[v][k] for m = 4 lg + r;
      // its four rows' bounds of vocabulary row v go out rounded up to bf16 in
      // one 8-byte store (uv [v][8]: the tile's 256 bytes in one instruction)
      float Ur[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * lg + r;
        float U = -INFINITY, L = -INFINITY;
        if (m < p.M) {
          const float zh = sc * acc[r];
          const float e = (sA[m] * rn + sB[m] * sc) * (1.f + 0x1p-16f) + fabsf(zh) * 0x1p-20f;
          U = zh + e;
          L = zh - e;
        }
        Ur[r] = U;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          U = nan_max(U, __shfl_xor(U, o));
          L = nan_max(L, __shfl_xor(L, o));
        }
        if (ln == 0 && m < p.M) s.ub[(int64_t)m * p.NT + tile] = U;
        Lw[r] = nan_max(Lw[r], L);
      }
      if (lg < 2)
        *reinterpret_cast<uint2*>(s.uv + ((int64_t)tile * 16 + ln) * 8 + 4 * lg) =
            make_uint2(bf16_up(Ur[0]) | (bf16_up(Ur[1]) << 16),
                       bf16_up(Ur[2]) | (bf16_up(Ur[3]) << 16));
      acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto load = [&](uint4 (&w)[4], int i) __attribute__((always_inline)) {
    const uint4* q = wptr(i);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) w[jj] = load_stream(q + 64 * jj);
  };
  uint4 wb[4];
  for (int i = 0; i < nitems; i += 2) {
    load(wb, i + 1);
    item(i, wc);
    load(wc, i + 2);
    if (i + 1 < nitems) item(i + 1, wb);  // wave-uniform
  }
  if (ln == 0)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (4 * lg + r < 8) sL[wave * 8 + 4 * lg + r] = Lw[r];
  __syncthreads();
  if (tid < p.M) {
    float L = -INFINITY;
#pragma unroll
    for (int w = 0; w < SC_W; ++w) L = nan_max(L, sL[w * 8 + tid]);
    s.lbw[(int64_t)tid * s.nwg + blockIdx.x] = L;
  }
}

struct ExactArgs {
  LmArgs lm;  // x source (NORM: h, sums of squares, norm weight), W in tile order, V, K, M, NT
  const float* ub;
  const float* lbw;
  const uint16_t* uv;
  int nwg;
  float* bestv;  // [8][EX_C]
  int* besti;    // [8][EX_C]
  int* cnt;      // [8][EX_CNT_STRIDE]: arrival counters (zero, left zero)
  int* xcd_err;  // may be null
  int64_t* next_out;
  int64_t* tokens;
  int32_t* pos;
  int32_t* count;
  const int32_t* limit;
  uint8_t* active;
  const int64_t* eos;
  int64_t* generated;
  int64_t gen_ld;
  int32_t* append_pos;
  int32_t* attn_len;
};

// Workgroup b handles row m = b % 8 and candidates c, c + EX_C, ... (c = b /
// 8): the threshold from the screen's lower bounds, the row's candidate tiles,
// x staged as the full pass stages it, each of its candidate tiles' logits
// with the full pass's arithmetic (the same MFMA sequence on the same operands
// in the same lanes: bit-identical float32 sums), its best (bf16 value, first
// index).  The EX_C workgroups of a row have ids equal modulo 8 (one XCD); the
// last to arrive (xcd_arrive) takes the row's best and does the decode
// bookkeeping of decode_advance_kernel.  A row that is not active keeps its
// token and computes nothing.
template <bool NORM>
__global__ void __launch_bounds__(64 * EX_WAVES) lm_exact_advance_kernel(ExactArgs e) {
  touch_kernargs<sizeof(ExactArgs)>();
  constexpr int NTH = 64 * EX_WAVES;
  constexpr int XU = 4;  // x chunks per thread loaded in the prologue (the rest when staging)
  const LmArgs& p = e.lm;
  extern __shared__ __align__(16) uint16_t xs[];  // x [M][K + 8], floats, candidate list
  const int m = blockIdx.x & 7, c0 = blockIdx.x >> 3;
  if (m >= p.M) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int xstride = p.K + 8;
  const int KS = p.K / LM_KSTEP;
  float* fl = reinterpret_cast<float*>(xs + p.M * xstride);
  float* sInv = fl;                                      // [8]
  float* sRed = fl + 8;                                  // [EX_WAVES]
  int* sBi = reinterpret_cast<int*>(fl + 8 + EX_WAVES);  // [EX_WAVES]
  int* sN = sBi + EX_WAVES;                              // candidate count, last-arrival flag
  int* sPass = sN + 2;                                   // [EX_WAVES][EX_PASSES]
  int* list = sPass + EX_WAVES * EX_PASSES;              // [NT]
  // active[m], read at entry and first used after the threshold (no early wait)
  const int act_m = e.tokens ? (int)e.active[m] : 1;
  // Every load the row needs before its first tile goes out at once: the
  // screen's lower bounds (nwg <= NTH), its upper bounds (tiles [tid per,
  // (tid + 1) per), clamped), and the inputs of the x staging.
  const float* ur = e.ub + (int64_t)m * p.NT;
  const int per = (p.NT + NTH - 1) / NTH;  // passes of NTH tiles, <= EX_PASSES
  const float lbv = e.lbw[(int64_t)m * e.nwg + min(tid, e.nwg - 1)];
  float u[EX_PASSES];  // pass j: tile tid + NTH j (coalesced)
#pragma unroll
  for (int j = 0; j < EX_PASSES; ++j)
    if (j < 20 || j < per) u[j] = ur[min(tid + NTH * j, p.NT - 1)];
  const int chunks = p.K / 8, total = p.M * chunks;
  uint4 hv[XU], wv[XU];
#pragma unroll
  for (int q = 0; q < XU; ++q) {
    const int i = min(tid + q * NTH, total - 1);
    const int mm = i / chunks, cc = i - mm * chunks;
    hv[q] = *reinterpret_cast<const uint4*>(p.x + (int64_t)mm * p.ldx + 8 * cc);
    if (NORM) wv[q] = *reinterpret_cast<const uint4*>(p.nw + 8 * cc);
  }
  float ssv[LM_NORM_MAX_GROUPS / 64];
  if (NORM && wave < p.M) {
    const float* ssr = p.nss + (int64_t)wave * p.nG;
#pragma unroll
    for (int q = 0; q < LM_NORM_MAX_GROUPS / 64; ++q) ssv[q] = ssr[min(lane + 64 * q, p.nG - 1)];
  }
  // threshold: the largest lower bound, less a bf16 rounding interval
  float lb = tid < e.nwg ? lbv : -INFINITY;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) lb = nan_max(lb, __shfl_xor(lb, o));
  if (lane == 0) sRed[wave] = lb;
  if (tid == 0) *sN = 0;
  __syncthreads();
  lb = -INFINITY;
#pragma unroll
  for (int w = 0; w < EX_WAVES; ++w) lb = nan_max(lb, sRed[w]);
  const float thr = (lb == lb && fabsf(lb) <= 3.4e38f)
                        ? lb - fabsf(lb) * 0x1p-6f - 1e-30f : -INFINITY;
  const bool run = __builtin_amdgcn_readfirstlane(act_m) != 0;
  // the row's candidate tiles, !(ub < thr) (a NaN bound is a candidate), in
  // tile order, so that every workgroup of the row builds the same list and
  // takes its share by position: an exclusive scan of the threads' counts
  // places each thread's candidates
  if (run) {
    // pass j covers tiles [NTH j, NTH (j + 1)); a candidate's place is the
    // count of the earlier passes, plus that of the earlier waves of its pass,
    // plus its rank in its wave's ballot
#pragma unroll
    for (int j = 0; j < EX_PASSES; ++j) {
      if (j < per) {  // wave-uniform
        const uint64_t b = __ballot(tid + NTH * j < p.NT && !(u[j] < thr));
        if (lane == 0) sPass[wave * EX_PASSES + j] = __popcll(b);
      }
    }
    __syncthreads();
    // wave 0, lane j: pass j's total over the waves, the exclusive prefix of
    // the totals, then each wave's start in pass j (sPass rewritten in place)
    if (wave == 0) {
      int n[EX_WAVES], tj = 0;
#pragma unroll
      for (int w = 0; w < EX_WAVES; ++w) {
        n[w] = lane < per ? sPass[w * EX_PASSES + lane] : 0;
        tj += n[w];
      }
      int inc = tj;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(inc, o);
        if (lane >= o) inc += v;
      }
      int start = inc - tj;
#pragma unroll
      for (int w = 0; w < EX_WAVES; ++w) {
        if (lane < per) sPass[w * EX_PASSES + lane] = start;
        start += n[w];
      }
      if (lane == 63) sN[0] = inc;  // all candidates (lanes >= per add nothing)
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < EX_PASSES; ++j) {
      if (j < per) {  // wave-uniform
        const int t = tid + NTH * j;
        const bool c = t < p.NT && !(u[j] < thr);
        const uint64_t b = __ballot(c);
        if (c) list[sPass[wave * EX_PASSES + j] + __popcll(b & ((1ull << lane) - 1ull))] = t;
      }
    }
  }
  __syncthreads();
  const int ncand = *sN;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  if (c0 < ncand) {
    // this workgroup's first tile: its loads go out before the x staging
    // Only the candidate rows of a candidate tile are read: lane (n, g) of a
    // row whose bound is below the threshold reads the tile's first chunk
    // instead (one shared line), and its logit is not compared.
    constexpr int KB = 6;  // k-steps whose loads are in flight together
    uint4 w[KB][8];
    auto slot = [&](int tile) __attribute__((always_inline)) {
      return !(bf2f(e.uv[((int64_t)tile * 16 + ln) * 8 + m]) < thr);
    };
    auto load_ks = [&](int tile, int ks0, bool cs) __attribute__((always_inline)) {
      const uint16_t* wtile = p.w + (int64_t)tile * KS * 8 * 64 * 8;
#pragma unroll
      for (int k = 0; k < KB; ++k)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          w[k][j] = load_stream(cs ? wtile + (((int64_t)min(ks0 + k, KS - 1) * 8 + j) * 64 + lane) * 8
                                   : wtile);
    };
    int c = c0 + EX_C * wave;
    bool cs = false;
    if (c < ncand) {
      cs = slot(list[c]);
      load_ks(list[c], 0, cs);
    }
    // x staged as lm_head_argmax_kernel stages it (same values, element for element)
    if (NORM) {
      if (wave < p.M) {
        float ss = 0.f;
#pragma unroll
        for (int q = 0; q < LM_NORM_MAX_GROUPS / 64; ++q)
          ss += lane + 64 * q < p.nG ? ssv[q] : 0.f;
        ss = wave_sum_dpp(ss);
        if (lane == 0) sInv[wave] = 1.f / sqrtf(ss / (float)p.K + p.neps);
      }
      __syncthreads();
    }
#pragma unroll
    for (int q = 0; q < XU; ++q) {
      const int i = tid + q * NTH;
      if (i < total) {
        const int mm = i / chunks, cc = i - mm * chunks;
        const uint4 v = NORM ? norm8(hv[q], wv[q], sInv[mm]) : hv[q];
        *reinterpret_cast<uint4*>(xs + mm * xstride + 8 * cc) = v;
      }
    }
    for (int i = tid + XU * NTH; i < total; i += NTH) {  // x beyond the prefetched chunks
      const int mm = i / chunks, cc = i - mm * chunks;
      uint4 v = *reinterpret_cast<const uint4*>(p.x + (int64_t)mm * p.ldx + 8 * cc);
      if (NORM) v = norm8(v, *reinterpret_cast<const uint4*>(p.nw + 8 * cc), sInv[mm]);
      *reinterpret_cast<uint4*>(xs + mm * xstride + 8 * cc) = v;
    }
    __syncthreads();
    const uint16_t* xrow = xs + min(ln, p.M - 1) * xstride + 8 * lg;
    for (; c < ncand; c += EX_C * EX_WAVES) {
      const int tile = list[c];
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      for (int ks0 = 0; ks0 < KS; ks0 += KB) {
        if (ks0 > 0) load_ks(tile, ks0, cs);
#pragma unroll
        for (int k = 0; k < KB; ++k) {
          if (ks0 + k < KS) {  // wave-uniform
#pragma unroll
            for (int j = 0; j < 8; ++j)
              acc = mfma16x16x32(
                  *reinterpret_cast<const uint4*>(xrow + (ks0 + k) * LM_KSTEP + 32 * j), w[k][j],
                  acc);
          }
        }
      }
      const bool cs_this = cs;
      if (c + EX_C * EX_WAVES < ncand) {
        cs = slot(list[c + EX_C * EX_WAVES]);
        load_ks(list[c + EX_C * EX_WAVES], 0, cs);
      }
      // row m's logits are in lane group m / 4, element m % 4
      const float a = (m & 3) == 0 ? acc[0] : (m & 3) == 1 ? acc[1] : (m & 3) == 2 ? acc[2] : acc[3];
      float v = bf2f(f2bf(a));
      int i = tile * 16 + ln;
      if (v != v || !cs_this) {
        v = -INFINITY;
        i = 0x7fffffff;
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const float ov = __shfl_xor(v, o);
        const int oi = __shfl_xor(i, o);
        if (better(ov, oi, v, i)) {
          v = ov;
          i = oi;
        }
      }
      if (better(v, i, bv, bi)) {
        bv = v;
        bi = i;
      }
    }
  }
  // lane 16 (m / 4) of every wave holds the wave's best for row m
  const int src = 16 * (m >> 2);
  bv = __shfl(bv, src);
  bi = __shfl(bi, src);
  if (lane == 0) {
    sRed[wave] = bv;
    sBi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 0; w < EX_WAVES; ++w)
      if (better(sRed[w], sBi[w], bv, bi)) {
        bv = sRed[w];
        bi = sBi[w];
      }
    e.bestv[m * EX_C + c0] = bv;
    e.besti[m * EX_C + c0] = bi;
    // arrival once the best is in the XCD's L2 (the vector L1 writes through)
    __builtin_amdgcn_s_waitcnt(0);
    sN[1] = xcd_arrive(e.cnt + m * EX_CNT_STRIDE, EX_C, e.xcd_err);
  }
  __syncthreads();
  if (wave != 0 || !sN[1]) return;
  // the last arrival: wave 0 reduces the row's EX_C bests (one per lane) and
  // lane 0 does decode_advance_kernel's bookkeeping (advance_row's rule); the
  // bests and the row state are loaded together
  asm volatile("buffer_inv sc0" ::: "memory");
  bv = -INFINITY;
  bi = 0x7fffffff;
  if (lane < EX_C) {
    bv = e.bestv[m * EX_C + lane];
    bi = e.besti[m * EX_C + lane];
  }
  int32_t rs_count = 0, rs_limit = 0, rs_pos = 0;
  int64_t rs_tok = 0, rs_eos = 0;
  if (e.tokens) {
    rs_count = e.count[m];
    rs_limit = e.limit[m];
    rs_pos = e.pos[m];
    rs_tok = e.tokens[m];
    rs_eos = e.eos[0];
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    const float ov = __shfl_xor(bv, o);
    const int oi = __shfl_xor(bi, o);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane != 0) return;
  const int64_t g = run ? (bi == 0x7fffffff ? 0 : bi) : rs_tok;
  if (e.next_out) e.next_out[m] = g;
  if (!e.tokens) return;
  const bool a = act_m != 0;
  const int32_t cnt = a ? rs_count + 1 : rs_count, ps = a ? rs_pos + 1 : rs_pos;
  if (a) {
    if (e.generated && rs_count >= 0 && rs_count < e.gen_ld)
      e.generated[(int64_t)m * e.gen_ld + rs_count] = g;
    e.pos[m] = ps;
    e.count[m] = cnt;
  }
  const bool still = a && cnt < rs_limit && g != rs_eos;
  e.active[m] = still ? 1 : 0;
  e.tokens[m] = g;
  e.append_pos[m] = still ? ps : -1;
  e.attn_len[m] = still ? ps + 1 : 0;
}

int screen_nwg(int NT) { return std::min(NT, SC_GRID); }

// Screen workspace: int32 counters [8][EX_CNT_STRIDE] (zero before the first
// exact pass, left zero by each), bestv float [8][EX_C], besti int32 [8][EX_C],
// then ub float [M][NT] and lbw float [M][nwg].
constexpr size_t WS_CNT = 0;
constexpr size_t WS_BESTV = WS_CNT + 8 * EX_CNT_STRIDE * 4;
constexpr size_t WS_BESTI = WS_BESTV + 8 * EX_C * 4;
constexpr size_t WS_UB = (WS_BESTI + 8 * EX_C * 4 + 255) / 256 * 256;

size_t screen_ws_bytes(int M, int V) {
  const int NT = V / 16;
  return WS_UB + ((size_t)M * NT + (size_t)M * screen_nwg(NT) + 3 + (size_t)4 * V) * sizeof(float);
}

int check_screen(const void* x, int64_t ldx, int V, int K, int M) {
  if (M <= 0 || M > LM_WAVES) return einval("the screened lm_head takes 1..8 rows");
  if (V <= 0 || K <= 0 || V % 16 || K % LM_KSTEP)
    return einval("the screened lm_head needs V % 16 == 0 and K % 256 == 0");
  if (V / 16 > EX_PASSES * 64 * EX_WAVES) return einval("the screened lm_head takes V <= 262144");
  if (!x || ldx < K || ldx % 8 || !aligned16(x))
    return einval("x must be 16-byte aligned with ldx >= K, ldx % 8 == 0");
  if ((size_t)M * (K + 8) * 4 + 256 + (size_t)SC_W * 8 * 4 > LM_LDS_MAX)
    return einval("x [M, K] of the screened lm_head does not fit in LDS");
  return GRPO_OK;
}

int run_screen(const void* x, int64_t ldx, const LmNorm* nrm, const void* wq, const float* scale,
               const float* rnorm, int V, int K, int M, void* ws, size_t ws_bytes,
               hipStream_t st) {
  if (int rc = check_screen(x, ldx, V, K, M)) return rc;
  if (!wq || !scale || !rnorm || !ws || !aligned16(wq)) return einval("null or misaligned pointer");
  if (ws_bytes < screen_ws_bytes(M, V)) {
    set_error("invalid argument: workspace of %zu bytes needed, %zu given",
              screen_ws_bytes(M, V), ws_bytes);
    return GRPO_EWORKSPACE;
  }
  ScreenArgs s{};
  LmArgs& a = s.lm;
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.V = V;
  a.K = K;
  a.M = M;
  a.NT = V / 16;
  if (nrm) {
    a.nss = nrm->sumsq;
    a.nG = nrm->groups;
    a.nw = nrm->weight;
    a.neps = nrm->eps;
  }
  s.wq = static_cast<const uint4*>(wq);
  s.scale = scale;
  s.rnorm = rnorm;
  s.ub = reinterpret_cast<float*>(static_cast<char*>(ws) + WS_UB);
  s.nwg = screen_nwg(a.NT);
  s.lbw = s.ub + (size_t)M * a.NT;
  s.uv = reinterpret_cast<uint16_t*>(s.lbw + (size_t)M * s.nwg +
                                     ((4 - ((size_t)M * (a.NT + s.nwg)) % 4) % 4));
  const size_t lds = (size_t)M * (K + 8) * 4 + (8 + 8 + 8 + SC_W * 8) * sizeof(float);
  if (nrm) {
    if (int rc = allow_dynamic_lds<lm_screen_kernel<true>, (int)LM_LDS_MAX>()) return rc;
    lm_screen_kernel<true><<<s.nwg, 64 * SC_W, lds, st>>>(s);
  } else {
    if (int rc = allow_dynamic_lds<lm_screen_kernel<false>, (int)LM_LDS_MAX>()) return rc;
    lm_screen_kernel<false><<<s.nwg, 64 * SC_W, lds, st>>>(s);
  }
  return launch_check("lm_screen");
}

int run_exact(const void* x, int64_t ldx, const LmNorm* nrm, const void* w_tiles, int V, int K,
              int M, void* ws, size_t ws_bytes, int* xcd_err, int64_t* next_out, int64_t* tokens, int32_t* pos,
              int32_t* count, const int32_t* limit, uint8_t* active, const int64_t* eos,
              int64_t* generated, int64_t gen_ld, int32_t* append_pos, int32_t* attn_len,
              hipStream_t st) {
  if (int rc = check_screen(x, ldx, V, K, M)) return rc;
  if (!w_tiles || !ws || !aligned16(w_tiles)) return einval("null or misaligned pointer");
  if (ws_bytes < screen_ws_bytes(M, V)) {
    set_error("invalid argument: workspace of %zu bytes needed, %zu given",
              screen_ws_bytes(M, V), ws_bytes);
    return GRPO_EWORKSPACE;
  }
  if (tokens && (!pos || !count || !limit || !active || !eos || !append_pos || !attn_len))
    return einval("null row state");
  if (generated && gen_ld <= 0) return einval("gen_ld must be > 0");
  ExactArgs e{};
  LmArgs& a = e.lm;
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = static_cast<const uint16_t*>(w_tiles);
  a.V = V;
  a.K = K;
  a.M = M;
  a.NT = V / 16;
  a.tiled = 1;
  if (nrm) {
    a.nss = nrm->sumsq;
    a.nG = nrm->groups;
    a.nw = nrm->weight;
    a.neps = nrm->eps;
  }
  char* wb = static_cast<char*>(ws);
  e.ub = reinterpret_cast<const float*>(wb + WS_UB);
  e.nwg = screen_nwg(a.NT);
  e.lbw = e.ub + (size_t)M * a.NT;
  e.uv = reinterpret_cast<const uint16_t*>(e.lbw + (size_t)M * e.nwg +
                                           ((4 - ((size_t)M * (a.NT + e.nwg)) % 4) % 4));
  e.bestv = reinterpret_cast<float*>(wb + WS_BESTV);
  e.besti = reinterpret_cast<int*>(wb + WS_BESTI);
  e.cnt = reinterpret_cast<int*>(wb + WS_CNT);
  e.xcd_err = xcd_err;
  e.next_out = next_out;
  e.tokens = tokens;
  e.pos = pos;
  e.count = count;
  e.limit = limit;
  e.active = active;
  e.eos = eos;
  e.generated = generated;
  e.gen_ld = gen_ld;
  e.append_pos = append_pos;
  e.attn_len = attn_len;
  const size_t lds = (size_t)M * (K + 8) * 2 +
                     (8 + 2 * EX_WAVES + 2 + EX_WAVES * EX_PASSES + (size_t)a.NT) * 4;
  if (lds > LM_LDS_MAX) return einval("the screened lm_head's candidate list does not fit in LDS");
  if (nrm) {
    if (int rc = allow_dynamic_lds<lm_exact_advance_kernel<true>, (int)LM_LDS_MAX>()) return rc;
    lm_exact_advance_kernel<true><<<8 * EX_C, 64 * EX_WAVES, lds, st>>>(e);
  } else {
    if (int rc = allow_dynamic_lds<lm_exact_advance_kernel<false>, (int)LM_LDS_MAX>()) return rc;
    lm_exact_advance_kernel<false><<<8 * EX_C, 64 * EX_WAVES, lds, st>>>(e);
  }
  return launch_check("lm_exact_advance");
}

}  // namespace

extern "C" int grpo_lm_head_q8_tiles(const void* w, int V, int K, void* wq_tiles, float* scale,
                                     float* rnorm, grpo_stream_t stream) {
  if (V <= 0 || K <= 0 || V % 16 || K % LM_KSTEP)
    return einval("needs V % 16 == 0 and K % 256 == 0");
  if (!w || !wq_tiles || !scale || !rnorm || !aligned16(w) || !aligned16(wq_tiles))
    return einval("w and wq_tiles must be non-null and 16-byte aligned");
  lm_q8_kernel<<<(unsigned)cdiv(V, 4), 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(w), static_cast<uint8_t*>(wq_tiles), scale, rnorm, V, K);
  return launch_check("lm_q8");
}

extern "C" size_t grpo_lm_head_screen_workspace_bytes(int M, int V) {
  if (M <= 0 || V <= 0 || V % 16) return 0;
  return screen_ws_bytes(M, V);
}

extern "C" int grpo_lm_head_screen(const void* x, int64_t ldx, const void* wq_tiles,
                                   const float* scale, const float* rnorm, int V, int K, int M,
                                   void* workspace, size_t workspace_bytes, grpo_stream_t stream) {
  return run_screen(x, ldx, nullptr, wq_tiles, scale, rnorm, V, K, M, workspace, workspace_bytes,
                    as_stream(stream));
}

extern "C" int grpo_lm_head_screen_norm(const void* h, int64_t ldh, const float* sumsq, int groups,
                                        const void* norm_weight, float eps, const void* wq_tiles,
                                        const float* scale, const float* rnorm, int V, int K,
                                        int M, void* workspace, size_t workspace_bytes,
                                        grpo_stream_t stream) {
  if (!sumsq || !norm_weight) return einval("null pointer");
  if (groups < 1 || groups > LM_NORM_MAX_GROUPS) return einval("groups must be in [1, 256]");
  if (!aligned16(norm_weight)) return einval("norm_weight must be 16-byte aligned");
  const LmNorm n{sumsq, groups, static_cast<const uint16_t*>(norm_weight), eps};
  return run_screen(h, ldh, &n, wq_tiles, scale, rnorm, V, K, M, workspace, workspace_bytes,
                    as_stream(stream));
}

extern "C" int grpo_lm_head_exact_argmax(const void* x, int64_t ldx, const void* w_tiles, int V,
                                         int K, int M, void* screen_workspace,
                                         size_t workspace_bytes, int* xcd_err,
                                         int64_t* next_tokens, grpo_stream_t stream) {
  if (!next_tokens) return einval("null next_tokens");
  return run_exact(x, ldx, nullptr, w_tiles, V, K, M, screen_workspace, workspace_bytes, xcd_err,
                   next_tokens,
                   nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, nullptr,
                   nullptr, as_stream(stream));
}

extern "C" int grpo_lm_head_exact_advance_norm(
    const void* h, int64_t ldh, const float* sumsq, int groups, const void* norm_weight, float eps,
    const void* w_tiles, int V, int K, int M, void* screen_workspace, size_t workspace_bytes,
    int* xcd_err, int64_t* next_tokens, int64_t* tokens, int32_t* pos, int32_t* count, const int32_t* limit, uint8_t* active,
    const int64_t* eos, int64_t* generated, int64_t gen_ld, int32_t* append_pos,
    int32_t* attn_len, grpo_stream_t stream) {
  if (!sumsq || !norm_weight) return einval("null pointer");
  if (groups < 1 || groups > LM_NORM_MAX_GROUPS) return einval("groups must be in [1, 256]");
  if (!aligned16(norm_weight)) return einval("norm_weight must be 16-byte aligned");
  const LmNorm n{sumsq, groups, static_cast<const uint16_t*>(norm_weight), eps};
  return run_exact(h, ldh, &n, w_tiles, V, K, M, screen_workspace, workspace_bytes, xcd_err,
                   next_tokens, tokens,
                   pos, count, limit, active, eos, generated, gen_ld, append_pos, attn_len,
                   as_stream(stream));
}
