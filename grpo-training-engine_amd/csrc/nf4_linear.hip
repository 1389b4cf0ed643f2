// NF4 dequantization and the fused NF4 + LoRA linear for gfx950.
//
// Weight format (bitsandbytes Params4bit, read by the reference in
// src/triton_kernels/lora_forward.py:171-206): W[N,K] flattened row-major,
// element e = n*K + k, byte e/2, even e = high nibble; one float32 absmax per
// `blocksize` flat elements; value = bf16_rne(code[q] * absmax).
//
// Fast linear path (M <= 64, K % 256 == 0, K <= 32768, N % 16 == 0,
// blocksize % 64 == 0, r <= 16): D = A*B on v_mfma_f32_16x16x32_bf16 with
// A = x (rows m) and B = W^T (columns n).
//
//  * Work unit: one wave = one 16-row n-tile x up to 4 k-steps of 256.  Lane
//    (n = lane%16, group g = lane/16) owns the 64-element chunk
//    [kstep*256 + 64g, +64) of row n: two 16-byte loads per k-step.  A wave
//    issues ALL its weight and absmax loads before decoding anything, so the
//    memory latency is paid once per wave, not once per k-step.
//  * Decode: per chunk a 16-entry bf16 codebook of bf16(code[j] * absmax) is
//    built in registers and nibbles are expanded with v_perm byte lookups, so
//    every product is exactly the reference's bf16(code*absmax) * x.  decode8
//    emits a dword's eight elements in the order [0,2,4,6,1,3,5,7]; x is
//    permuted the same way, so MFMA sums matching pairs.
//  * Split-K stays inside one workgroup: a workgroup has ntw n-tiles x kw
//    k-groups of waves (<= 16 waves); the kw partial sums are added through
//    LDS in fixed order, so results are deterministic and no cross-workgroup
//    synchronisation (device-scope fences) is ever needed.
//  * x is staged in LDS once per workgroup when it fits (gfx950 allows 160 KiB
//    per workgroup), otherwise each wave reads its own x fragments from L2.
//  * LoRA: x A^T is one more 16-column MFMA tile (A is bf16); the tile of
//    k-group kg is computed by the wave of n-tile kg % ntw, so the extra work
//    is spread over the workgroup; the epilogue applies the reference's
//    rounding points (lora_forward.py:243-257).
#include "common.hpp"

using namespace grpo;

namespace {

constexpr int KSTEP = 256;         // k elements per step: 4 lane groups x 64
constexpr int KPW_MAX = 8;         // k-steps per wave (all loads in flight at once)
constexpr int MAX_WAVES = 16;      // waves per workgroup (1024 threads)
constexpr int LDS_BYTES = 163840;  // gfx950: 160 KiB of LDS per workgroup
constexpr int TARGET_WAVES = 4096; // launch-shape heuristic (4 per SIMD on 256 CUs)
constexpr int MAXSEG = 4;

// ------------------------------------------------------------- dequant --

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
      o[j] = pack_bf2(hi, lo);
    }
    out[2 * i] = make_uint4(o[0], o[1], o[2], o[3]);
    out[2 * i + 1] = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

__global__ void __launch_bounds__(256) nf4_dequant_scalar(const uint8_t* __restrict__ w,
                                                          const float* __restrict__ absmax,
                                                          const float* __restrict__ code16,
                                                          uint16_t* __restrict__ out,
                                                          int64_t numel, int blocksize) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < numel; e += stride) {
    const uint32_t byte = w[e >> 1];
    const uint32_t q = (e & 1) ? (byte & 15u) : (byte >> 4);
    out[e] = f2bf(code16[q] * absmax[e / blocksize]);
  }
}

// ------------------------------------------------------- nibble decode --

__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
  return (m & a) | (~m & b);
}

// 16-entry bf16 codebook of one absmax block, split into high bytes (hb) and
// low bytes (lb): hb[i] byte j = high byte of bf16(code[4i+j] * a).
struct Lut {
  uint32_t hb[4], lb[4];
};

__device__ __forceinline__ Lut make_lut(const float (&code)[16], float a) {
  Lut t;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t p01 = pack_bf2(code[4 * i] * a, code[4 * i + 1] * a);
    const uint32_t p23 = pack_bf2(code[4 * i + 2] * a, code[4 * i + 3] * a);
    t.hb[i] = perm(p23, p01, 0x07050301u);
    t.lb[i] = perm(p23, p01, 0x06040200u);
  }
  return t;
}

// Eight nibbles of one little-endian dword (bytes b0..b3; element 2i = high
// nibble of b_i) -> eight bf16 as 4 dwords in element order [0,2,4,6,1,3,5,7].
__device__ __forceinline__ uint4 decode8(uint32_t wd, const Lut& t) {
  const uint32_t sh = (wd >> 4) & 0x07070707u;               // low 3 bits, even elements
  const uint32_t sl = wd & 0x07070707u;                      // low 3 bits, odd elements
  const uint32_t mh = perm(wd << 8, wd, 0x090B080Au);        // 0xFF where nibble bit 3 set
  const uint32_t ml = perm(wd << 12, wd << 4, 0x090B080Au);
  const uint32_t Hh = bfi(mh, perm(t.hb[3], t.hb[2], sh), perm(t.hb[1], t.hb[0], sh));
  const uint32_t Lh = bfi(mh, perm(t.lb[3], t.lb[2], sh), perm(t.lb[1], t.lb[0], sh));
  const uint32_t Hl = bfi(ml, perm(t.hb[3], t.hb[2], sl), perm(t.hb[1], t.hb[0], sl));
  const uint32_t Ll = bfi(ml, perm(t.lb[3], t.lb[2], sl), perm(t.lb[1], t.lb[0], sl));
  return make_uint4(perm(Hh, Lh, 0x05010400u), perm(Hh, Lh, 0x07030602u),
                    perm(Hl, Ll, 0x05010400u), perm(Hl, Ll, 0x07030602u));
}

// Eight bf16 in natural order (4 dwords) -> the decode8 order [0,2,4,6,1,3,5,7].
__device__ __forceinline__ uint4 deinterleave8(uint4 v) {
  return make_uint4(perm(v.y, v.x, 0x05040100u), perm(v.w, v.z, 0x05040100u),
                    perm(v.y, v.x, 0x07060302u), perm(v.w, v.z, 0x07060302u));
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// ---------------------------------------------------------- arguments --

// Output rows [seg_end[s-1], seg_end[s]) form segment s, with its own bias,
// LoRA A [r, K] and LoRA B [rows_s, r] (one segment for a plain projection;
// q|k|v or gate|up stacked into one weight for a grouped launch).
struct LinearArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  const float* absmax;
  const float* code16;
  int blocksize;
  int nseg;
  int seg_end[MAXSEG];
  const uint16_t* bias[MAXSEG];
  const uint16_t* la[MAXSEG];  // lora A [r, K] per segment
  const uint16_t* lb[MAXSEG];  // lora B [rows_s, r] per segment
  int r;
  float scaling;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int ntw, kw, kpw;  // n-tiles per workgroup, k-groups per workgroup, k-steps per wave
  int bs_shift;      // log2(blocksize) (power-of-two blocksizes on the fast path)
  int xstride;       // LDS row stride of staged x (elements)
  int off_red, off_redt, off_tsum;  // LDS byte offsets of the reduction areas
};

struct LinearPlan {
  int MT, KS, NT, ntw, kw, kpw, grid;
  bool xlds;
  int xstride, off_red, off_redt, off_tsum;
  size_t lds;
};

__host__ __device__ inline bool aligned16(const void* ptr) {
  return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0;
}

bool segments_aligned(const LinearArgs& a, int rows) {
  for (int s = 0; s + 1 < a.nseg; ++s)
    if (a.seg_end[s] % rows != 0) return false;
  return true;
}

LinearPlan plan_linear(const LinearArgs& a) {
  LinearPlan p{};
  p.MT = (a.M + 15) / 16;
  if (p.MT == 3) p.MT = 4;  // launched as the MT = 4 kernel (sizes below must match)
  p.KS = a.K / KSTEP;
  p.NT = a.N / 16;
  int kw = (TARGET_WAVES + p.NT - 1) / p.NT;
  if (kw > p.KS) kw = p.KS;
  if (kw < 1) kw = 1;
  int kpw = (p.KS + kw - 1) / kw;
  const int kpw_min = (p.KS + MAX_WAVES - 1) / MAX_WAVES;  // at most 16 k-groups
  if (kpw < kpw_min) kpw = kpw_min;
  // LoRA waves also hold a LoRA-A chunk: keep their prefetch depth at <= 2
  // k-steps so 16-wave workgroups fit in 128 registers per lane.
  const int kpw_max = a.r > 0 ? 2 : KPW_MAX;
  if (kpw > kpw_max) kpw = kpw_max;
  kw = (p.KS + kpw - 1) / kpw;
  int ntw = MAX_WAVES / kw;
  ntw = ntw >= 4 ? 4 : (ntw >= 2 ? 2 : 1);
  while (ntw > 1 && !segments_aligned(a, 16 * ntw)) ntw /= 2;
  p.kw = kw;
  p.kpw = kpw;
  p.ntw = ntw;
  p.grid = (p.NT + ntw - 1) / ntw;
  const int red = (kw - 1) * ntw * p.MT * 256 * 4;
  const int redt = a.r > 0 ? kw * p.MT * 256 * 4 : 0;
  const int tsum = a.r > 0 ? p.MT * 16 * 16 * 4 : 0;
  const int xbytes = ((a.M * (a.K + 8) * 2) + 15) & ~15;
  p.xlds = xbytes + red + redt + tsum <= LDS_BYTES;
  p.xstride = a.K + 8;
  const int xb = p.xlds ? xbytes : 0;
  p.off_red = xb;
  p.off_redt = xb + red;
  p.off_tsum = xb + red + redt;
  p.lds = (size_t)xb + red + redt + tsum;
  return p;
}

// x fragment for MFMA: lane (m = mt*16 + lane%16) holds x[m][kcol .. kcol+8) in
// decode8 order; rows >= M are zero.
template <bool XLDS>
__device__ __forceinline__ uint4 xfrag(const LinearArgs& p, const uint16_t* xs, int m, int kcol) {
  if (m >= p.M) return make_uint4(0, 0, 0, 0);
  if (XLDS) return *reinterpret_cast<const uint4*>(xs + m * p.xstride + kcol);
  return deinterleave8(*reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + kcol));
}

// ------------------------------------------------------ fast linear --

template <int MT, bool LORA, bool XLDS, int KPW>
__global__ void __launch_bounds__(1024) nf4_linear_mfma(LinearArgs p) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int nt_local = wave % p.ntw, kg = wave / p.ntw;
  const int ntile = blockIdx.x * p.ntw + nt_local;
  const int KS = p.K / KSTEP;
  const int ks0 = kg * p.kpw;
  const int nk = max(0, min(p.kpw, KS - ks0));
  const int n_row = ntile * 16 + ln;
  const bool row_ok = n_row < p.N;

  // Segment of this workgroup (the host keeps workgroups inside one segment).
  const int wg_row0 = blockIdx.x * p.ntw * 16;
  int seg = 0;
  while (seg + 1 < p.nseg && wg_row0 >= p.seg_end[seg]) ++seg;
  const int seg_begin = seg > 0 ? p.seg_end[seg - 1] : 0;

  // The LoRA-A tile of k-group kg is computed once, by the wave of n-tile kg % ntw.
  const bool do_t = LORA && nt_local == kg % p.ntw;
  const uint16_t* seg_la = p.la[seg];
  const bool r_ok = ln < p.r;
  const bool epi = kg == 0 && row_ok;  // waves of k-group 0 write the outputs
  const int n_loc = n_row - seg_begin;

  // 1. Every global load of the wave is issued before anything waits on one
  //    (one memory round trip): weights + absmax of all its k-steps, the
  //    LoRA-A chunk of its first k-step, the epilogue's bias and LoRA-B row,
  //    and then the x staging loads.
  uint4 wv[2 * KPW];
  float av[KPW];
  {
    const uint8_t* wrow = p.w + (int64_t)(row_ok ? n_row : 0) * (p.K / 2);
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      wv[2 * i] = make_uint4(0, 0, 0, 0);
      wv[2 * i + 1] = make_uint4(0, 0, 0, 0);
      av[i] = 0.f;
      if (i < nk && row_ok) {
        const int kc = (ks0 + i) * KSTEP + 64 * lg;
        const uint4* wp = reinterpret_cast<const uint4*>(wrow + kc / 2);
        wv[2 * i] = wp[0];
        wv[2 * i + 1] = wp[1];
        av[i] = p.absmax[((int64_t)n_row * p.K + kc) >> p.bs_shift];
      }
    }
  }
  uint4 av4[8];  // LoRA-A chunk of the current k-step
  if (do_t && nk > 0) {
    const uint16_t* arow = seg_la + (int64_t)(r_ok ? ln : 0) * p.K + ks0 * KSTEP + 64 * lg;
#pragma unroll
    for (int j = 0; j < 8; ++j)
      av4[j] = r_ok ? *reinterpret_cast<const uint4*>(arow + 8 * j) : make_uint4(0, 0, 0, 0);
  }
  const uint16_t* seg_bias = p.bias[seg];
  const float bias = epi && seg_bias ? bf2f(seg_bias[n_loc]) : 0.f;
  float bl[16];
  if (LORA) {
    const uint16_t* brow = p.lb[seg] + (int64_t)n_loc * p.r;
    if (epi && p.r == 16 && aligned16(brow)) {
      const uint4 b0 = reinterpret_cast<const uint4*>(brow)[0];
      const uint4 b1 = reinterpret_cast<const uint4*>(brow)[1];
      const uint32_t bw8[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        bl[2 * q] = bf_lo(bw8[q]);
        bl[2 * q + 1] = bf_hi(bw8[q]);
      }
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) bl[q] = epi && q < p.r ? bf2f(brow[q]) : 0.f;
    }
  }

  // 2. Stage x (all K) in LDS in decode8 order: loads batched 4 per thread.
  const uint16_t* xs = reinterpret_cast<const uint16_t*>(smem);
  if (XLDS) {
    uint16_t* xw = reinterpret_cast<uint16_t*>(smem);
    const int chunks = p.K / 8;
    const int total = p.M * chunks;
    for (int base = 0; base < total; base += 4 * (int)blockDim.x) {
      uint4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = base + u * (int)blockDim.x + tid;
        if (i < total) {
          const int m = i / chunks, c = i - m * chunks;
          v[u] = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + c * 8);
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = base + u * (int)blockDim.x + tid;
        if (i < total) {
          const int m = i / chunks, c = i - m * chunks;
          *reinterpret_cast<uint4*>(xw + m * p.xstride + c * 8) = deinterleave8(v[u]);
        }
      }
    }
    __syncthreads();
  }
  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];

  f32x4_t acc[MT];
  f32x4_t tacc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    tacc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // 3. Decode + MFMA, one k-step at a time.
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    if (i >= nk) break;
    const int kc = (ks0 + i) * KSTEP + 64 * lg;
    if (do_t && i > 0) {  // later LoRA-A chunks; latency overlaps the decode below
      const uint16_t* arow = seg_la + (int64_t)(r_ok ? ln : 0) * p.K + kc;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        av4[j] = r_ok ? *reinterpret_cast<const uint4*>(arow + 8 * j) : make_uint4(0, 0, 0, 0);
    }
    // x fragments of this k-step, read ahead of the decode (one m-tile).
    uint4 xf[8];
    constexpr bool PRE = MT == 1 && KPW <= 4;
    if (PRE) {
#pragma unroll
      for (int j = 0; j < 8; ++j) xf[j] = xfrag<XLDS>(p, xs, ln, kc + 8 * j);
    }
    const Lut t = make_lut(code, av[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint4 bw = decode8(word(wv[2 * i + (j >> 2)], j & 3), t);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = mfma16x16x32(PRE ? xf[j] : xfrag<XLDS>(p, xs, mt * 16 + ln, kc + 8 * j), bw,
                               acc[mt]);
    }
    if (do_t) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const uint4 bv = deinterleave8(av4[j]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          tacc[mt] = mfma16x16x32(PRE ? xf[j] : xfrag<XLDS>(p, xs, mt * 16 + ln, kc + 8 * j),
                                  bv, tacc[mt]);
      }
    }
  }

  // 4. Reduce the kw k-groups (fixed order) and the LoRA-A partials.
  float* red = reinterpret_cast<float*>(smem + p.off_red);    // [kw-1][ntw][MT][256]
  float* redt = reinterpret_cast<float*>(smem + p.off_redt);  // [kw][MT][256]
  float* tsum = reinterpret_cast<float*>(smem + p.off_tsum);  // [MT*16][16]
  if (p.kw > 1 && kg > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      *reinterpret_cast<float4*>(red + (((kg - 1) * p.ntw + nt_local) * MT + mt) * 256 + lane * 4) =
          make_float4(acc[mt][0], acc[mt][1], acc[mt][2], acc[mt][3]);
  }
  if (do_t) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      *reinterpret_cast<float4*>(redt + (kg * MT + mt) * 256 + lane * 4) =
          make_float4(tacc[mt][0], tacc[mt][1], tacc[mt][2], tacc[mt][3]);
  }
  if (p.kw > 1 || LORA) __syncthreads();
  if (LORA) {
    // tacc lane (r = lane%16, g) slot q holds T[m = mt*16 + 4g + q][r]
    for (int i = tid; i < MT * 256; i += blockDim.x) {
      const int mt = i >> 8, idx = i & 255, l = idx >> 2, q = idx & 3;
      float s = 0.f;
      for (int k = 0; k < p.kw; ++k) s += redt[(k * MT + mt) * 256 + idx];
      tsum[(mt * 16 + 4 * (l >> 4) + q) * 16 + (l & 15)] = round_bf(s);
    }
    __syncthreads();
  }
  if (kg != 0 || !row_ok) return;
  for (int k = 1; k < p.kw; ++k) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float4 v = *reinterpret_cast<const float4*>(
          red + (((k - 1) * p.ntw + nt_local) * MT + mt) * 256 + lane * 4);
      acc[mt][0] += v.x;
      acc[mt][1] += v.y;
      acc[mt][2] += v.z;
      acc[mt][3] += v.w;
    }
  }

  // 5. Epilogue: y = bf16(bf16(bf16(acc) + bias) + bf16(bf16(bf16(T) B^T) * bf16(s))).
  const float sc = round_bf(p.scaling);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = mt * 16 + 4 * lg + q;
      if (m >= p.M) continue;
      float v = round_bf(acc[mt][q]);
      if (seg_bias) v = round_bf(v + bias);
      if (LORA) {
        const float* tr = tsum + m * 16;
        float u = 0.f;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) u += tr[rr] * bl[rr];
        u = round_bf(round_bf(u) * sc);
        v = round_bf(v + u);
      }
      p.y[(int64_t)m * p.ldy + n_row] = f2bf(v);
    }
}

// ---------------------------------------------------- generic linear --
// Any shape: one thread per output; the reference arithmetic spelled out.
__global__ void __launch_bounds__(256) nf4_linear_generic(LinearArgs p) {
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

bool use_fast_linear(const LinearArgs& a) {
  if ((a.blocksize & (a.blocksize - 1)) != 0) return false;
  if (!(a.M >= 1 && a.M <= 64 && a.K > 0 && a.K % KSTEP == 0 &&
        a.K <= MAX_WAVES * (a.r > 0 ? 2 : KPW_MAX) * KSTEP && a.N % 16 == 0 && a.blocksize % 64 == 0 &&
        a.r <= 16 && a.ldx % 8 == 0 && aligned16(a.x) && aligned16(a.w) &&
        segments_aligned(a, 16)))
    return false;
  for (int s = 0; s < a.nseg; ++s)
    if (a.r > 0 && !aligned16(a.la[s])) return false;
  return true;
}

// Allows a kernel more than the default dynamic LDS (once per instantiation).
template <typename K>
int allow_lds(K kernel) {
  static int rc = -1;
  if (rc < 0)
    rc = hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES),
                   "hipFuncSetAttribute");
  return rc;
}

template <int MT, bool LORA, int KPW>
int launch_kpw(LinearArgs& a, const LinearPlan& plan, hipStream_t st) {
  dim3 grid(plan.grid), block(64 * plan.ntw * plan.kw);
  if (plan.xlds) {
    if (int rc = allow_lds(nf4_linear_mfma<MT, LORA, true, KPW>)) return rc;
    nf4_linear_mfma<MT, LORA, true, KPW><<<grid, block, plan.lds, st>>>(a);
  } else {
    if (int rc = allow_lds(nf4_linear_mfma<MT, LORA, false, KPW>)) return rc;
    nf4_linear_mfma<MT, LORA, false, KPW><<<grid, block, plan.lds, st>>>(a);
  }
  return launch_check("nf4_linear_mfma");
}

template <int MT>
int launch_fast(LinearArgs& a, const LinearPlan& plan, hipStream_t st) {
  if (a.r > 0)
    return plan.kpw <= 1 ? launch_kpw<MT, true, 1>(a, plan, st)
                         : launch_kpw<MT, true, 2>(a, plan, st);
  if (plan.kpw <= 1) return launch_kpw<MT, false, 1>(a, plan, st);
  if (plan.kpw <= 2) return launch_kpw<MT, false, 2>(a, plan, st);
  if (plan.kpw <= 4) return launch_kpw<MT, false, 4>(a, plan, st);
  return launch_kpw<MT, false, 8>(a, plan, st);
}

int run_linear(LinearArgs& a, hipStream_t st) {
  if (use_fast_linear(a)) {
    const LinearPlan plan = plan_linear(a);
    a.ntw = plan.ntw;
    a.kw = plan.kw;
    a.kpw = plan.kpw;
    a.bs_shift = __builtin_ctz((unsigned)a.blocksize);
    a.xstride = plan.xstride;
    a.off_red = plan.off_red;
    a.off_redt = plan.off_redt;
    a.off_tsum = plan.off_tsum;
    switch (plan.MT) {
      case 1: return launch_fast<1>(a, plan, st);
      case 2: return launch_fast<2>(a, plan, st);
      default: return launch_fast<4>(a, plan, st);  // M in (32, 64]: one zero m-tile at most
    }
  }
  const int64_t total = (int64_t)a.M * a.N;
  nf4_linear_generic<<<dim3((unsigned)cdiv(total, 256)), 256, 0, st>>>(a);
  return launch_check("nf4_linear_generic");
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

extern "C" int grpo_nf4_dequant(const uint8_t* w, const float* absmax, const float* code16,
                                void* out, int64_t numel, int blocksize, grpo_stream_t stream) {
  if (numel < 0) return einval("numel < 0");
  if (blocksize <= 0) return einval("blocksize must be > 0");
  if (numel == 0) return GRPO_OK;
  if (!w || !absmax || !code16 || !out) return einval("null pointer");
  hipStream_t st = as_stream(stream);
  if (numel % 16 == 0 && blocksize % 16 == 0 && (reinterpret_cast<uintptr_t>(w) & 7u) == 0 &&
      aligned16(out)) {
    const int64_t nvec = numel / 16;
    const int64_t blocks = std::min<int64_t>(cdiv(nvec, 256), 8192);
    nf4_dequant_vec<<<dim3((unsigned)blocks), 256, 0, st>>>(
        reinterpret_cast<const uint2*>(w), absmax, code16, reinterpret_cast<uint4*>(out), nvec,
        blocksize);
  } else {
    const int64_t blocks = std::min<int64_t>(cdiv(numel, 256), 8192);
    nf4_dequant_scalar<<<dim3((unsigned)blocks), 256, 0, st>>>(
        w, absmax, code16, reinterpret_cast<uint16_t*>(out), numel, blocksize);
  }
  return launch_check("nf4_dequant");
}

extern "C" int grpo_nf4_lora_linear(const void* x, int64_t ldx, const uint8_t* w,
                                    const float* absmax, const float* code16, int blocksize,
                                    const void* bias, const void* lora_a, const void* lora_b, int r,
                                    float scaling, void* y, int64_t ldy, int M, int N, int K,
                                    grpo_stream_t stream) {
  if (int rc = check_common(x, ldx, w, absmax, code16, blocksize, r, y, ldy, M, N, K)) return rc;
  if (M == 0 || N == 0) return GRPO_OK;
  if (r > 0 && (!lora_a || !lora_b)) return einval("r > 0 needs lora_a and lora_b");
  LinearArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = w;
  a.absmax = absmax;
  a.code16 = code16;
  a.blocksize = blocksize;
  a.nseg = 1;
  a.seg_end[0] = N;
  a.bias[0] = static_cast<const uint16_t*>(bias);
  a.la[0] = static_cast<const uint16_t*>(lora_a);
  a.lb[0] = static_cast<const uint16_t*>(lora_b);
  a.r = r;
  a.scaling = scaling;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  return run_linear(a, as_stream(stream));
}

extern "C" int grpo_nf4_lora_linear_grouped(const void* x, int64_t ldx, const uint8_t* w,
                                            const float* absmax, const float* code16,
                                            int blocksize, int nseg, const int* seg_rows,
                                            const void* const* bias, const void* const* lora_a,
                                            const void* const* lora_b, int r, float scaling,
                                            void* y, int64_t ldy, int M, int K,
                                            grpo_stream_t stream) {
  if (nseg < 1 || nseg > MAXSEG) return einval("nseg must be in [1, 4]");
  if (!seg_rows) return einval("null seg_rows");
  int N = 0;
  for (int s = 0; s < nseg; ++s) {
    if (seg_rows[s] <= 0) return einval("segment with no rows");
    N += seg_rows[s];
  }
  if (int rc = check_common(x, ldx, w, absmax, code16, blocksize, r, y, ldy, M, N, K)) return rc;
  if (M == 0) return GRPO_OK;
  LinearArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = w;
  a.absmax = absmax;
  a.code16 = code16;
  a.blocksize = blocksize;
  a.nseg = nseg;
  int end = 0;
  for (int s = 0; s < nseg; ++s) {
    end += seg_rows[s];
    a.seg_end[s] = end;
    a.bias[s] = bias ? static_cast<const uint16_t*>(bias[s]) : nullptr;
    a.la[s] = r > 0 && lora_a ? static_cast<const uint16_t*>(lora_a[s]) : nullptr;
    a.lb[s] = r > 0 && lora_b ? static_cast<const uint16_t*>(lora_b[s]) : nullptr;
    if (r > 0 && (!a.la[s] || !a.lb[s])) return einval("r > 0 needs lora_a and lora_b per segment");
    if (nseg > 1 && (int64_t)seg_rows[s] * K % blocksize != 0)
      return einval("every segment must hold whole absmax blocks");
  }
  a.r = r;
  a.scaling = scaling;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  return run_linear(a, as_stream(stream));
}
