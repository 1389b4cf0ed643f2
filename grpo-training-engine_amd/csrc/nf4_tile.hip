// NF4 (+ LoRA, + bias) linear finished in one launch, for decode batches
// (M <= 32 rows): one workgroup per tile of output columns over the whole K.
//
// y = x W^T with the reference epilogue (src/triton_kernels/lora_forward.py:
// 208-257): v = bf16(acc); v = bf16(v + bias); t = bf16(x A^T);
// u = bf16(bf16(t B^T) * bf16(scaling)); y = bf16(v + u).  The NF4 weight
// format and the decode are those of nf4_decode.hpp.
//
// Why a tile per workgroup.  The split-K path (nf4_linear.hip) cuts K into
// slices over many workgroups and leaves float32 partial sums for the
// consumer to add, or hands them to the last-arriving slice through an L2
// counter.  Either costs a round trip through memory after the MFMAs.  Here
// the waves of ONE workgroup take all of K for the workgroup's columns; their
// accumulator tiles meet in LDS, are summed in a fixed order, and the
// epilogue runs in the same workgroup:
//  * TE_OUT: y stored as bf16 rows (the q|k|v projection of the decode step,
//    read by the attention);
//  * TE_RES: h = bf16(residual + y) and, per row, the sum of h^2 over the
//    workgroup's columns (o_proj of the decode step: the next RMSNorm is
//    staged from h and those sums by its consumer).
//
// Two tilings of v_mfma_f32_16x16x32_bf16 (A = x rows, B = decoded W^T):
//  * plain (9..32 rows): 16 columns per workgroup; k-unit = one k-step of 256
//    K values, lane (n = lane % 16, lg = lane / 16) decoding K values
//    256 u + 64 lg .. + 63 of column n (one absmax block);
//  * FOLD (<= 8 rows, half of the MFMA's 16 rows idle otherwise): 8 columns
//    per workgroup and K folded into the MFMA's rows and columns: for k-unit
//    u (512 K values) rows 0..7 of A carry x over K values 512 u .. 512 u +
//    255 and rows 8..15 the same x rows over the next 256; B columns 0..7 and
//    8..15 the same 8 weight columns over the same two ranges, so D[m][n] +
//    D[m + 8][n + 8] is the product over all 512 (the cross quadrants are
//    discarded).  Twice the workgroups of the plain tiling for the same
//    decode work per wave: at Qwen2-1.5B's q|k|v and o_proj every CU of the
//    device gets one.
// Decode waves take the k-units (wave w: units w, w + WD, ...).  The LoRA
// product x A_s^T (the tile's segment s, over all of K) runs on LoRA waves of
// their own when the workgroup has room (WD + WL <= 8), else on the decode
// waves after their units: its B operand is LoRA A in the packed MFMA order
// of grpo_nf4_tile_pack_lora_a (one contiguous KiB per load instruction;
// row-major A would touch 64 cache lines per instruction).
//
// x sources: TX_BF16 (bf16 rows), or TX_NORM: RMSNorm(h) = bf16(bf16(h * inv)
// * w) with inv = 1 / sqrt(sum(h^2) / K + eps) from per-group sums of squares
// that the producer of h wrote (the input norm of a decode layer).  Every
// workgroup stages all of x (M x K bf16) in LDS, row-major in decode8 order.
#include "linear_parts.hpp"
#include "nf4_decode.hpp"

using namespace grpo;

namespace {

// At most 8 waves (two per SIMD, up to 256 VGPRs each): the VALU time per
// SIMD is set by the k-units it decodes, and every decode wave issues all of
// its weight loads up front.
constexpr int TILE_MAX_WAVES = 8;
constexpr int TILE_KPW_MAX = 4;            // k-units per decode wave
constexpr int TILE_LDS_MAX = 163840;       // x rows + reduction tiles
constexpr int TILE_MAX_ROWS = 32;
constexpr int TILE_NORM_MAX_GROUPS = 256;  // sums of squares per row (TX_NORM)
constexpr int TILE_XU = 8;                 // x chunks per thread loaded before the weights
constexpr int TILE_LPF = 2;                // LoRA k-steps per wave whose A is loaded up front

enum TileX { TX_BF16 = 0, TX_NORM = 1 };
enum TileEpi { TE_OUT = 0, TE_RES = 1 };

struct TileArgs {
  const uint16_t* x;  // TX_BF16: [M][ldx]; TX_NORM: h [M][ldx]
  int64_t ldx;
  const float* nss;   // TX_NORM: [M][nG] sums of squares of h
  int nG;
  const uint16_t* nw; // TX_NORM: RMSNorm weight [K]
  float neps;
  const uint8_t* w;
  const float* absmax;
  const float* code16;
  int bs_shift;
  int M, N, K, KU, WD, WL, nseg, r;
  int seg_end[MAXSEG];
  const uint4* la[MAXSEG];  // packed LoRA A (grpo_nf4_tile_pack_lora_a)
  const uint16_t* lb[MAXSEG];
  const uint16_t* bias[MAXSEG];
  float scaling;
  uint16_t* y;        // TE_OUT: [M][ldy]; TE_RES: h [M][ldy] (may alias res)
  int64_t ldy;
  const uint16_t* res;  // TE_RES: residual [M][ldy]
  float* ss;          // TE_RES: [M][N / columns per workgroup]
  const float* tsrc;  // x A^T as float32 partials [M][tparts][16], or null
  int tparts;
};
constexpr int TILE_TPARTS_MAX = 4;

__device__ __forceinline__ int tile_seg(const TileArgs& p, int n) {
  return (p.nseg > 1 && n >= p.seg_end[0] ? 1 : 0) + (p.nseg > 2 && n >= p.seg_end[1] ? 1 : 0) +
         (p.nseg > 3 && n >= p.seg_end[2] ? 1 : 0);
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));

template <int MT, int KPW, int XS, int EPI, bool FOLD>
__global__ void __launch_bounds__(64 * TILE_MAX_WAVES) nf4_tile_mfma(TileArgs p) {
  static_assert(!FOLD || MT == 1, "the folded tiling takes at most 8 rows");
  touch_kernargs<sizeof(TileArgs)>();
  constexpr int TC = FOLD ? 8 : 16;        // output columns per workgroup
  constexpr int KUL = FOLD ? 512 : KSTEP;  // K values per k-unit
  extern __shared__ __align__(16) uint16_t xs[];  // [M][K + 8] (decode8 order), then tiles
  const int W = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);
  const int NTH = 64 * W;
  const int WD = p.WD, WL = p.WL;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * TC;
  const int seg = tile_seg(p, n0);  // uniform: segment ends are multiples of 16
  const int seg0 = seg > 0 ? sel_seg(p.seg_end, seg - 1) : 0;
  const int xstride = p.K + 8;
  const int chunks = p.K / 8, total = p.M * chunks;
  const bool dwave = wave < WD;             // decode wave (else LoRA wave)
  const int lw = dwave ? wave : wave - WD;  // index among the waves doing LoRA
  const bool lora_here = p.r > 0 && !p.tsrc && (WL > 0 ? !dwave : true);
  const int nlw = WL > 0 ? WL : WD;         // waves sharing the LoRA k-steps
  const int KS = p.K / KSTEP;
  float* red = reinterpret_cast<float*>(xs + p.M * xstride);  // [WD][MT][64][4]
  float* lred = red + WD * MT * 256;                         // [nlw][MT][16 m][16 r]

  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];
  // Load order (see nf4_part_mfma): vector loads retire in order and a wait
  // after a conditional load can only assume the fewest loads in flight, so
  // the conditional loads go first: the epilogue's inputs (only its waves),
  // the row statistics, LoRA A (only LoRA waves); then x and the weights,
  // unconditional (indexes clamped), so the x staging waits for x alone.
  //
  // Epilogue inputs: bias, LoRA B row of this lane's column (ranks 4 lg ..
  // 4 lg + 3) and the residual, loaded by every wave (the epilogue's waves
  // use them: wave mt < MT takes row tile mt) as raw 16-bit values with
  // clamped indexes and stand-in addresses, no arithmetic on them before
  // the epilogue (an operation on a loaded value makes the wave wait for it
  // here).  Folded: lanes n < 8 of lane groups 0, 1 own the outputs (column
  // n0 + n, rows 4 lg + q); the others load in range and idle.
  const bool epi_wave = wave < MT;
  const int ecol = n0 + (ln & (TC - 1));
  const int nl = ecol - seg0;
  const uint16_t* bp = sel_seg(p.bias, seg);
  const uint16_t* lbp = p.r > 0 ? sel_seg(p.lb, seg) + (int64_t)nl * p.r
                                : reinterpret_cast<const uint16_t*>(p.code16);
  const uint32_t bias_raw =
      (bp ? bp : reinterpret_cast<const uint16_t*>(p.code16))[bp ? nl : 0];
  uint32_t lb_raw[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) lb_raw[j] = lbp[p.r > 0 ? min(4 * lg + j, p.r - 1) : 0];
  // x A^T partials given by the producer of x (tsrc): rows m = ln (clamped),
  // ranks 4 lg .. 4 lg + 3, every part (clamped; extra parts dropped)
  // (unconditional: the codebook stands in when there is none, values unused)
  float4 tg[MT][TILE_TPARTS_MAX];
  {
    const float* tb = p.tsrc ? p.tsrc : p.code16;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < TILE_TPARTS_MAX; ++q) {
        const int64_t ti = p.tsrc ? ((int64_t)min(16 * mt + ln, p.M - 1) * p.tparts +
                                     min(q, p.tparts - 1)) * 16 + 4 * lg
                                  : 0;
        tg[mt][q] = *reinterpret_cast<const float4*>(tb + ti);
      }
  }
  uint32_t res_raw[MT][4];
  if (EPI == TE_RES) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        res_raw[mt][q] =
            p.res[(int64_t)min(16 * mt + 4 * (FOLD ? (lg & 1) : lg) + q, p.M - 1) * p.ldy + ecol];
  }
  __builtin_amdgcn_sched_barrier(0);

  // TX_NORM: 16 threads per row sum the row's group sums, four groups per
  // float4 load (rows tid / 16, and tid / 16 + NTH / 16 for two row tiles);
  // the norm weight goes to LDS once (all rows share it)
  constexpr int NSS4 = TILE_NORM_MAX_GROUPS / 64;
  float4 ssv[MT][NSS4];
  uint4* snw = reinterpret_cast<uint4*>(lred + (p.r > 0 ? nlw * MT * 256 : 0));  // [K / 8]
  uint4 nwv = make_uint4(0, 0, 0, 0);
  if (XS == TX_NORM) {
#pragma unroll
    for (int h = 0; h < MT; ++h) {
      const int m = min((tid >> 4) + h * (NTH >> 4), p.M - 1);
      const float4* ssr = reinterpret_cast<const float4*>(p.nss + (int64_t)m * p.nG);
      const int j = tid & 15;
#pragma unroll
      for (int i = 0; i < NSS4; ++i) ssv[h][i] = ssr[min(j + 16 * i, (p.nG >> 2) - 1)];
    }
    nwv = *reinterpret_cast<const uint4*>(p.nw + 8 * min(tid, chunks - 1));
  }
  __builtin_amdgcn_sched_barrier(0);
  // LoRA: this wave's k-steps lw, lw + nlw, ...; the packed A of the first
  // TILE_LPF of them (8 x 16 bytes per lane each) loaded here, unconditional
  // (clamped to the wave's last k-step), the others where they are used
  // (one k-step up front when the wave also holds 3 or 4 k-units of weights)
  constexpr int LPF = KPW <= 2 ? TILE_LPF : 1;
  const uint4* ap = lora_here ? sel_seg(p.la, seg) + lane : nullptr;
  const int nls = lora_here ? (KS - lw + nlw - 1) / nlw : 0;
  uint4 a8[LPF][8];
  if (lora_here) {
#pragma unroll
    for (int i = 0; i < LPF; ++i) {
      const int ks = lw + nlw * max(0, min(i, nls - 1));
#pragma unroll
      for (int j = 0; j < 8; ++j) a8[i][j] = ap[(ks * 8 + j) * 64];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // x chunks of the first batch: TILE_XU per thread, unconditional (indexes
  // clamped; a clamped chunk is staged twice with the same value)
  uint4 xv[TILE_XU];
#pragma unroll
  for (int u = 0; u < TILE_XU; ++u) {
    const int i = min(u * NTH + tid, total - 1);
    const int m = i / chunks, c = i - m * chunks;
    xv[u] = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + 8 * c);
  }
  __builtin_amdgcn_sched_barrier(0);

  // decode wave: its k-units wave, wave + WD, ... (nk of them).  Every wave
  // issues these loads (a LoRA wave those of decode wave wave % WD, values
  // unused), so no wait of the loads before them is conservative.
  const int dw = dwave ? wave : wave % WD;
  const int nk = min(KPW, (p.KU - dw + WD - 1) / WD);
  const int wcol = n0 + (FOLD ? (ln & 7) : ln);          // weight row of this lane
  const int wk = (FOLD ? 256 * (ln >> 3) : 0) + 64 * lg;  // its K offset within a unit
  uint4 wv[2 * KPW];
  float av[KPW];
  {
    const uint8_t* wrow = p.w + (int64_t)wcol * (p.K / 2);
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int ku = dw + WD * min(i, nk - 1);
      const int kc = ku * KUL + wk;
      const uint4* wp = reinterpret_cast<const uint4*>(wrow + kc / 2);
      wv[2 * i] = load_w<true>(wp);
      wv[2 * i + 1] = load_w<true>(wp + 1);
      av[i] = p.absmax[((int64_t)wcol * p.K + kc) >> p.bs_shift];
    }
  }
  // Stage x in LDS (decode8 order).  TX_NORM: 1 / rms per row and the norm
  // weight into LDS first.
  __shared__ float sInv[TILE_MAX_ROWS];
  if (XS == TX_NORM) {
    if (tid < chunks) snw[tid] = nwv;
    for (int c = tid + NTH; c < chunks; c += NTH) snw[c] = *reinterpret_cast<const uint4*>(p.nw + 8 * c);
#pragma unroll
    for (int h = 0; h < MT; ++h) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < NSS4; ++i)
        if ((tid & 15) + 16 * i < (p.nG >> 2)) s += (ssv[h][i].x + ssv[h][i].y) + (ssv[h][i].z + ssv[h][i].w);
      s = sum16(s);
      const int m = (tid >> 4) + h * (NTH >> 4);
      if ((tid & 15) == 0 && m < p.M) sInv[m] = 1.f / sqrtf(s / (float)p.K + p.neps);
    }
    __syncthreads();
  }
  // the first batch from the registers loaded above, the rest (more than
  // TILE_XU chunks per thread) loaded here
#pragma unroll
  for (int u = 0; u < TILE_XU; ++u) {
    const int i = min(u * NTH + tid, total - 1);
    const int m = i / chunks, c = i - m * chunks;
    const uint4 xr = XS == TX_NORM ? norm8(xv[u], snw[c], sInv[m]) : xv[u];
    *reinterpret_cast<uint4*>(xs + m * xstride + 8 * c) = deinterleave8(xr);
  }
  for (int base = TILE_XU * NTH; base < total; base += 4 * NTH) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(base + u * NTH + tid, total - 1);
      const int m = i / chunks, c = i - m * chunks;
      v[u] = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + 8 * c);
      if (XS == TX_NORM) v[u] = norm8(v[u], snw[c], sInv[m]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = min(base + u * NTH + tid, total - 1);
      const int m = i / chunks, c = i - m * chunks;
      *reinterpret_cast<uint4*>(xs + m * xstride + 8 * c) = deinterleave8(v[u]);
    }
  }
  __syncthreads();

  // A operand rows: plain, lane (ln, lg) multiplies row 16 mt + ln over K
  // values 256 u + 64 lg + 8 j; folded, row ln % 8 over 512 u + 256 (ln / 8)
  // + 64 lg + 8 j.  The LoRA product always takes the plain form.
  const uint16_t* xrow[MT];
  const uint16_t* xrowp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    xrowp[mt] = xs + min(16 * mt + ln, p.M - 1) * xstride + 64 * lg;
    xrow[mt] = FOLD ? xs + min(ln & 7, p.M - 1) * xstride + 256 * (ln >> 3) + 64 * lg : xrowp[mt];
  }
  if (dwave) {
    f32x4_t acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      if (i >= nk) break;
      const int ku = wave + WD * i;
      const Lut t = make_lut(code, av[i]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint4 bw = decode8(word(wv[2 * i + (j >> 2)], j & 3), t);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = mfma16x16x32(*reinterpret_cast<const uint4*>(xrow[mt] + ku * KUL + 8 * j),
                                 bw, acc[mt]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      *reinterpret_cast<f32x4_t*>(red + ((wave * MT + mt) * 64 + lane) * 4) = acc[mt];
  }
  if (lora_here) {
    // t partial over this wave's k-steps: B = packed A (lane (rank ln, lg)
    // holds A[ln][256 ks + 64 lg + 8 j ..], decode8 order, zero past r)
    f32x4_t lacc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) lacc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < LPF; ++i) {
      if (i >= nls) break;
      const int ks = lw + nlw * i;
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          lacc[mt] = mfma16x16x32(*reinterpret_cast<const uint4*>(xrowp[mt] + ks * KSTEP + 8 * j),
                                  a8[i][j], lacc[mt]);
    }
    for (int i = LPF; i < nls; ++i) {
      const int ks = lw + nlw * i;
      uint4 b8[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) b8[j] = ap[(ks * 8 + j) * 64];
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          lacc[mt] = mfma16x16x32(*reinterpret_cast<const uint4*>(xrowp[mt] + ks * KSTEP + 8 * j),
                                  b8[j], lacc[mt]);
    }
    // LoRA t transposed to [m][rank] (lane (rank ln, lg) holds rows 4 lg + q)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) lred[(lw * MT + mt) * 256 + (4 * lg + q) * 16 + ln] = lacc[mt][q];
  }
  __syncthreads();
  if (!epi_wave) return;

  const float sc = round_bf(p.scaling);
  const int mt = wave;
  // sum over the decode waves in order (wave w holds k-units w, w + WD, ...);
  // folded: D[m][n] (lane n, lg) + D[m + 8][n + 8] (lane n + 8, lg + 2)
  f32x4_t s = {0.f, 0.f, 0.f, 0.f};
  for (int w = 0; w < WD; ++w) {
    const float* rw = red + (w * MT + mt) * 256;
    s += *reinterpret_cast<const f32x4_t*>(rw + lane * 4);
    if (FOLD) s += *reinterpret_cast<const f32x4_t*>(rw + ((lane + 40) & 63) * 4);
  }
  f32x4_t u = {0.f, 0.f, 0.f, 0.f};
  if (p.r > 0) {
    // t[m = ln][ranks 4 lg .. 4 lg + 3] = bf16(sum over the LoRA waves), then
    // u[m][n] = t[m, :] . B[n, :] on one 16x16x16 bf16 MFMA (B zero past r)
    f32x4_t t = {0.f, 0.f, 0.f, 0.f};
    if (p.tsrc) {
#pragma unroll
      for (int q = 0; q < TILE_TPARTS_MAX; ++q)
        if (q < p.tparts) t += f32x4_t{tg[mt][q].x, tg[mt][q].y, tg[mt][q].z, tg[mt][q].w};
    } else {
      for (int w = 0; w < nlw; ++w)
        t += *reinterpret_cast<const f32x4_t*>(lred + (w * MT + mt) * 256 + ln * 16 + 4 * lg);
    }
    uint32_t lb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) lb[j] = 4 * lg + j < p.r ? lb_raw[j] : 0u;
    const i16x4_t av4 = __builtin_bit_cast(i16x4_t, make_uint2(pack_bf2(t[0], t[1]),
                                                               pack_bf2(t[2], t[3])));
    const i16x4_t bv4 =
        __builtin_bit_cast(i16x4_t, make_uint2(lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16)));
    u = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av4, bv4, u, 0, 0, 0);
  }
  const float bias_v = bf2f((uint16_t)bias_raw);
  const bool owner = FOLD ? (ln < 8 && lg < 2) : true;
  const bool has_bias = sel_seg(p.bias, seg) != nullptr;
  float sq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int m = 16 * mt + 4 * lg + q;
    float v = round_bf(s[q]);
    if (has_bias) v = round_bf(v + bias_v);
    if (p.r > 0) v = round_bf(v + round_bf(round_bf(u[q]) * sc));
    if (EPI == TE_RES) v = round_bf(v + bf2f((uint16_t)res_raw[mt][q]));
    const bool ok = owner && m < p.M;
    if (ok) p.y[(int64_t)m * p.ldy + ecol] = f2bf(v);
    sq[q] = ok ? v * v : 0.f;
  }
  if (EPI == TE_RES) {
    // per row: sum of h^2 over the workgroup's columns (lanes 0..TC-1 of a
    // DPP row)
#pragma unroll
    for (int q = 0; q < 4; ++q) sq[q] = FOLD ? sum8(sq[q]) : sum16(sq[q]);
    if (ln == 0 && owner) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 16 * mt + 4 * lg + q;
        if (m < p.M) p.ss[(int64_t)m * (p.N / TC) + blockIdx.x] = sq[q];
      }
    }
  }
}

// Packed LoRA A: for k-step ks and MFMA j, the 64 lanes' 16-byte B operands
// (lane (rank ln = lane % 16, lg = lane / 16): A[ln][256 ks + 64 lg + 8 j ..
// + 7] in decode8 order, zero for ln >= r) are one contiguous KiB.
__global__ void __launch_bounds__(256) tile_pack_lora_a_kernel(const uint16_t* __restrict__ a,
                                                               int r, int K, int64_t lda,
                                                               uint4* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (ks * 8 + j) * 64 + lane
  if (i >= (int64_t)(K / KSTEP) * 8 * 64) return;
  const int lane = (int)(i & 63), kj = (int)(i >> 6);
  const int ks = kj >> 3, j = kj & 7;
  const int rk = lane & 15, lg = lane >> 4;
  uint4 v = make_uint4(0, 0, 0, 0);
  if (rk < r)
    v = deinterleave8(*reinterpret_cast<const uint4*>(a + (int64_t)rk * lda + ks * KSTEP +
                                                       64 * lg + 8 * j));
  out[i] = v;
}

struct TilePlan {
  int WD, WL, KPW, MT;
  bool fold;
  size_t lds;
  bool ok;
};

TilePlan plan_tile(int M, int N, int K, int r, int nseg, int blocksize, bool norm = false,
                   bool tgiven = false) {
  TilePlan t{};
  if (M < 1 || M > TILE_MAX_ROWS || N < 16 || N % 16 || K < KSTEP || K % KSTEP) return t;
  if (r < 0 || r > 16 || nseg < 1 || nseg > MAXSEG) return t;
  if (blocksize < 64 || (blocksize & (blocksize - 1))) return t;
  t.fold = M <= 8 && K % 512 == 0;
  t.MT = M > 16 ? 2 : 1;
  const int KU = K / (t.fold ? 512 : KSTEP);
  t.KPW = (KU + TILE_MAX_WAVES - 1) / TILE_MAX_WAVES;
  if (t.KPW > TILE_KPW_MAX) return t;
  t.WD = (KU + t.KPW - 1) / t.KPW;
  // LoRA waves of their own when the workgroup has room for as many
  t.WL = r > 0 && !tgiven && 2 * t.WD <= TILE_MAX_WAVES ? t.WD : 0;
  const int nlw = t.WL > 0 ? t.WL : t.WD;
  // x rows, the decode and LoRA tiles, the norm weight (RMSNorm source)
  t.lds = (size_t)M * (K + 8) * 2 +
          (size_t)(t.WD + (r > 0 && !tgiven ? nlw : 0)) * t.MT * 256 * 4 +
          (norm ? (size_t)K * 2 : 0);
  t.ok = t.lds <= TILE_LDS_MAX;
  return t;
}


template <int MT, int KPW, int XS, int EPI, bool FOLD>
int launch_tile_k(const TileArgs& a, const TilePlan& pl, hipStream_t st) {
  constexpr auto kern = nf4_tile_mfma<MT, KPW, XS, EPI, FOLD>;
  if (pl.lds > 65536)
    if (int rc = allow_dynamic_lds<kern, TILE_LDS_MAX>()) return rc;
  const int tc = FOLD ? 8 : 16;
  nf4_tile_mfma<MT, KPW, XS, EPI, FOLD>
      <<<dim3(a.N / tc), dim3(64 * (pl.WD + pl.WL)), pl.lds, st>>>(a);
  return launch_check("nf4_tile_mfma");
}

template <int MT, int XS, int EPI, bool FOLD>
int launch_tile_kpw(const TileArgs& a, const TilePlan& pl, hipStream_t st) {
  switch (pl.KPW) {
    case 1: return launch_tile_k<MT, 1, XS, EPI, FOLD>(a, pl, st);
    case 2: return launch_tile_k<MT, 2, XS, EPI, FOLD>(a, pl, st);
    case 3: return launch_tile_k<MT, 3, XS, EPI, FOLD>(a, pl, st);
    default: return launch_tile_k<MT, 4, XS, EPI, FOLD>(a, pl, st);
  }
}

template <int XS, int EPI>
int launch_tile(const TileArgs& a, const TilePlan& pl, hipStream_t st) {
  if (pl.fold) return launch_tile_kpw<1, XS, EPI, true>(a, pl, st);
  if (pl.MT == 1) return launch_tile_kpw<1, XS, EPI, false>(a, pl, st);
  return launch_tile_kpw<2, XS, EPI, false>(a, pl, st);
}

// Common checks and argument set-up of the three entry points.
int tile_args(const grpo_tile_linear_t* lin, const void* x, int64_t ldx, const uint8_t* w,
              const float* absmax, const float* code16, int blocksize, void* y, int64_t ldy,
              TileArgs* a, TilePlan* pl, bool norm = false) {
  if (!lin) return einval("null linear descriptor");
  const int M = lin->M, N = lin->N, K = lin->K;
  const bool tgiven = lin->r > 0 && lin->lora_t;
  *pl = plan_tile(M, N, K, lin->r, lin->nseg, blocksize, norm, tgiven);
  if (!pl->ok) {
    set_error("shape not supported by the one-launch NF4 linear (M <= 32, N %% 16 == 0, "
              "K %% 256 == 0, x within LDS)");
    return GRPO_EUNSUPPORTED;
  }
  if (!x || !w || !absmax || !code16 || !y) return einval("null pointer");
  if (ldx < K || ldx % 8 || !aligned16(x) || !aligned16(w))
    return einval("x rows must be 16-byte aligned with ldx >= K, ldx % 8 == 0; w 16-byte aligned");
  if (ldy < N) return einval("ldy must be >= N");
  int prev = 0;
  for (int s = 0; s < lin->nseg; ++s) {
    if (lin->seg_end[s] <= prev || lin->seg_end[s] % 16)
      return einval("segment ends must increase and be multiples of 16");
    prev = lin->seg_end[s];
    if (lin->r > 0 && !lin->lora_b[s]) return einval("r > 0 needs lora_b per segment");
    if (lin->r > 0 && !tgiven && (!lin->lora_a[s] || !aligned16(lin->lora_a[s])))
      return einval("r > 0 needs packed lora_a (16-byte aligned) per segment");
  }
  if (tgiven && (lin->nseg != 1 || lin->lora_t_parts < 1 ||
                 lin->lora_t_parts > TILE_TPARTS_MAX || !aligned16(lin->lora_t)))
    return einval("lora_t needs one segment, 1..4 parts and 16-byte alignment");
  if (prev != N) return einval("the last segment end must equal N");
  TileArgs& t = *a;
  t = TileArgs{};
  t.x = static_cast<const uint16_t*>(x);
  t.ldx = ldx;
  t.w = w;
  t.absmax = absmax;
  t.code16 = code16;
  t.bs_shift = __builtin_ctz((unsigned)blocksize);
  t.M = M;
  t.N = N;
  t.K = K;
  t.KU = K / (pl->fold ? 512 : KSTEP);
  t.WD = pl->WD;
  t.WL = pl->WL;
  t.nseg = lin->nseg;
  t.r = lin->r;
  for (int s = 0; s < MAXSEG; ++s) {
    const bool on = s < lin->nseg;
    t.seg_end[s] = on ? lin->seg_end[s] : N;
    t.la[s] = on && lin->r > 0 ? static_cast<const uint4*>(lin->lora_a[s]) : nullptr;
    t.lb[s] = on && lin->r > 0 ? static_cast<const uint16_t*>(lin->lora_b[s]) : nullptr;
    t.bias[s] = on ? static_cast<const uint16_t*>(lin->bias[s]) : nullptr;
  }
  t.scaling = lin->scaling;
  t.tsrc = tgiven ? lin->lora_t : nullptr;
  t.tparts = tgiven ? lin->lora_t_parts : 1;
  t.y = static_cast<uint16_t*>(y);
  t.ldy = ldy;
  return GRPO_OK;
}

}  // namespace

extern "C" int grpo_nf4_tile_supported(int M, int N, int K, int r, int nseg, int blocksize) {
  return plan_tile(M, N, K, r, nseg, blocksize).ok ? 1 : 0;
}

extern "C" int grpo_nf4_tile_norm_supported(int M, int N, int K, int r, int nseg,
                                            int blocksize) {
  const TilePlan pl = plan_tile(M, N, K, r, nseg, blocksize, true);
  return pl.ok && M <= 4 * (pl.WD + pl.WL) * pl.MT ? 1 : 0;
}

extern "C" int grpo_nf4_tile_sumsq_groups(int M, int N, int K, int r, int blocksize) {
  const TilePlan pl = plan_tile(M, N, K, r, 1, blocksize);
  if (!pl.ok) return 0;
  return N / (pl.fold ? 8 : 16);
}

extern "C" size_t grpo_nf4_tile_packed_lora_a_bytes(int K) {
  return K > 0 && K % KSTEP == 0 ? (size_t)(K / KSTEP) * 8 * 64 * 16 : 0;
}

extern "C" int grpo_nf4_tile_pack_lora_a(const void* lora_a, int r, int K, int64_t lda,
                                         void* out, grpo_stream_t stream) {
  if (r < 1 || r > 16 || K < KSTEP || K % KSTEP || lda < K) return einval("bad LoRA A shape");
  if (!lora_a || !out) return einval("null pointer");
  if (!aligned16(lora_a) || lda % 8 || !aligned16(out))
    return einval("lora_a rows and out must be 16-byte aligned");
  const int64_t n = (int64_t)(K / KSTEP) * 8 * 64;
  tile_pack_lora_a_kernel<<<dim3((unsigned)cdiv(n, 256)), 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(lora_a), r, K, lda, static_cast<uint4*>(out));
  return launch_check("tile_pack_lora_a");
}

extern "C" int grpo_nf4_tile_linear(const void* x, int64_t ldx, const uint8_t* w,
                                    const float* absmax, const float* code16, int blocksize,
                                    const grpo_tile_linear_t* lin, void* y, int64_t ldy,
                                    grpo_stream_t stream) {
  TileArgs a;
  TilePlan pl;
  if (int rc = tile_args(lin, x, ldx, w, absmax, code16, blocksize, y, ldy, &a, &pl)) return rc;
  return launch_tile<TX_BF16, TE_OUT>(a, pl, as_stream(stream));
}

extern "C" int grpo_nf4_tile_linear_norm(const void* h, int64_t ldh, const float* sumsq,
                                         int groups, const void* norm_weight, float eps,
                                         const uint8_t* w, const float* absmax,
                                         const float* code16, int blocksize,
                                         const grpo_tile_linear_t* lin, void* y, int64_t ldy,
                                         grpo_stream_t stream) {
  TileArgs a;
  TilePlan pl;
  if (int rc = tile_args(lin, h, ldh, w, absmax, code16, blocksize, y, ldy, &a, &pl, true))
    return rc;
  if (!sumsq || !norm_weight) return einval("null pointer");
  if (groups < 4 || groups > TILE_NORM_MAX_GROUPS || groups % 4)
    return einval("groups must be a multiple of 4 in [4, 256]");
  if (!aligned16(norm_weight) || !aligned16(sumsq))
    return einval("norm_weight and sumsq must be 16-byte aligned");
  if (lin->M > 4 * (pl.WD + pl.WL) * pl.MT) {  // 16 threads per row, MT rows per thread
    set_error("the RMSNorm staging takes at most 4 rows per wave and row tile");
    return GRPO_EUNSUPPORTED;
  }
  a.nss = sumsq;
  a.nG = groups;
  a.nw = static_cast<const uint16_t*>(norm_weight);
  a.neps = eps;
  return launch_tile<TX_NORM, TE_OUT>(a, pl, as_stream(stream));
}

extern "C" int grpo_nf4_tile_linear_residual(const void* x, int64_t ldx, const uint8_t* w,
                                             const float* absmax, const float* code16,
                                             int blocksize, const grpo_tile_linear_t* lin,
                                             const void* residual, void* h_out, int64_t ld,
                                             float* sumsq, grpo_stream_t stream) {
  TileArgs a;
  TilePlan pl;
  if (int rc = tile_args(lin, x, ldx, w, absmax, code16, blocksize, h_out, ld, &a, &pl))
    return rc;
  if (!residual || !sumsq) return einval("null pointer");
  a.res = static_cast<const uint16_t*>(residual);
  a.ss = sumsq;
  return launch_tile<TX_BF16, TE_RES>(a, pl, as_stream(stream));
}
