// Input gradient of the NF4 linear for gfx950 (the training side of the fused
// NF4 + LoRA linear): out[m, k] = bf16(sum_n g[m, n] * W[n, k]), optionally
// out = bf16(out + addend[m, k]).  Restates _lora_grad_x_base_kernel
// (src/triton_kernels/lora_forward.py:262-348): W = bf16_rne(code[q] * absmax)
// exactly as the forward dequantizes it, float32 accumulation over the N
// output features, one bf16 rounding; the addend is the reference's
// `grad_x_base + grad_x_lora` (:873) folded into the store.
//
//  * Tile: a workgroup of 8 waves owns 128 rows m x 128 columns k; wave
//    (wm, wk) owns 64 rows x 32 columns as 4 x 2 tiles of
//    v_mfma_f32_16x16x32_bf16 (A = g rows m, B = W columns k, reduction over
//    n): 16 MFMAs per wave per 64-row chunk of W, two waves per SIMD.
//  * Per chunk the workgroup reads g[128, 64] (two 16-byte loads per thread)
//    and 64 x 128 nibbles of W (per thread 8 consecutive k of rows n and n + 1,
//    each inside one absmax block), decodes W and writes it to LDS transposed
//    ([k][n], an (n, n + 1) pair per dword), so every MFMA operand is one
//    16-byte LDS read.  The next chunk's global loads are issued before the
//    current chunk's MFMAs.  A last chunk past N (N % 64 == 32) reads zeros.
//  * Rows m >= M read row M - 1 and are not stored.
#include "common.hpp"

using namespace grpo;

namespace {

constexpr int GX_TM = 128;      // rows m per workgroup
constexpr int GX_TK = 128;      // columns k per workgroup
constexpr int GX_TN = 64;       // reduction chunk (rows n of W)
constexpr int GX_T = 512;       // threads
constexpr int GX_LD = GX_TN + 8;  // LDS row stride (bf16) of both tiles: 144 bytes

struct GradXArgs {
  const uint16_t* g;
  int64_t ldg;
  const uint8_t* w;
  const float* absmax;
  const float* code;
  int bs;
  const uint16_t* add;
  int64_t lda;
  uint16_t* out;
  int64_t ldo;
  int M, N, K;
};

struct GradXChunk {  // one thread's global loads of one chunk
  uint4 g0, g1;       // g rows gr and gr + 64, 8 columns
  uint32_t w0, w1;    // 8 nibbles of W rows n and n + 1
  float a0, a1;       // their absmax
};

__device__ __forceinline__ void gx_load(const GradXArgs& p, const uint16_t* g0p,
                                        const uint16_t* g1p, int gcol, int64_t e0, int wrow,
                                        int n0, GradXChunk& c) {
  // N % 32 == 0: the 8 columns of g and the row pair of W are in or out together
  const uint4 z = make_uint4(0, 0, 0, 0);
  c.g0 = n0 + gcol < p.N ? *reinterpret_cast<const uint4*>(g0p + n0) : z;
  c.g1 = n0 + gcol < p.N ? *reinterpret_cast<const uint4*>(g1p + n0) : z;
  c.w0 = c.w1 = 0;
  c.a0 = c.a1 = 0.f;
  if (n0 + wrow < p.N) {
    const int64_t e = e0 + (int64_t)n0 * p.K;  // flat element of row n, a multiple of 8
    c.w0 = *reinterpret_cast<const uint32_t*>(p.w + e / 2);
    c.w1 = *reinterpret_cast<const uint32_t*>(p.w + (e + p.K) / 2);
    c.a0 = p.absmax[e / p.bs];
    c.a1 = p.absmax[(e + p.K) / p.bs];
  }
}

__global__ void __launch_bounds__(GX_T) nf4_grad_x_kernel(GradXArgs p) {
  __shared__ __align__(16) uint16_t sg[GX_TM * GX_LD];  // g chunk [m][n]
  __shared__ __align__(16) uint16_t sw[GX_TK * GX_LD];  // W chunk transposed [k][n]
  __shared__ float scode[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int wm = wave >> 2, wk = wave & 3;
  const int k0 = blockIdx.x * GX_TK, m0 = blockIdx.y * GX_TM;
  if (tid < 16) scode[tid] = p.code[tid];
  // g loader: rows tid / 8 and tid / 8 + 64 of the tile, columns 8 (tid % 8) .. + 7
  const int gr = tid >> 3, gc = (tid & 7) * 8;
  const uint16_t* g0p = p.g + (int64_t)min(m0 + gr, p.M - 1) * p.ldg + gc;
  const uint16_t* g1p = p.g + (int64_t)min(m0 + gr + 64, p.M - 1) * p.ldg + gc;
  // W loader: rows 2 (tid % 32) and + 1 of the chunk, columns k0 + 8 (tid / 32) .. + 7
  const int wr = (tid & 31) * 2, wc = (tid >> 5) * 8;
  const int64_t e0 = (int64_t)wr * p.K + k0 + wc;
  f32x4_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  GradXChunk c;
  gx_load(p, g0p, g1p, gc, e0, wr, 0, c);
  __syncthreads();  // codebook
  for (int n0 = 0; n0 < p.N; n0 += GX_TN) {
    __syncthreads();  // the previous chunk's MFMAs have read both tiles
    *reinterpret_cast<uint4*>(sg + gr * GX_LD + gc) = c.g0;
    *reinterpret_cast<uint4*>(sg + (gr + 64) * GX_LD + gc) = c.g1;
    // byte j holds elements 2j (high nibble) and 2j + 1 (low nibble) of the 8
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t b0 = (c.w0 >> (8 * j)) & 0xFFu, b1 = (c.w1 >> (8 * j)) & 0xFFu;
      *reinterpret_cast<uint32_t*>(sw + (wc + 2 * j) * GX_LD + wr) =
          (uint32_t)f2bf(scode[b0 >> 4] * c.a0) | ((uint32_t)f2bf(scode[b1 >> 4] * c.a1) << 16);
      *reinterpret_cast<uint32_t*>(sw + (wc + 2 * j + 1) * GX_LD + wr) =
          (uint32_t)f2bf(scode[b0 & 15u] * c.a0) |
          ((uint32_t)f2bf(scode[b1 & 15u] * c.a1) << 16);
    }
    __syncthreads();
    if (n0 + GX_TN < p.N) gx_load(p, g0p, g1p, gc, e0, wr, n0 + GX_TN, c);
#pragma unroll
    for (int ks = 0; ks < GX_TN / 32; ++ks) {
      uint4 b[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
        b[kt] = *reinterpret_cast<const uint4*>(sw + (wk * 32 + kt * 16 + ln) * GX_LD +
                                                ks * 32 + 8 * lg);
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const uint4 a = *reinterpret_cast<const uint4*>(sg + (wm * 64 + mt * 16 + ln) * GX_LD +
                                                        ks * 32 + 8 * lg);
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) acc[mt][kt] = mfma16x16x32(a, b[kt], acc[mt][kt]);
      }
    }
  }
  // lane (ln, lg) holds D[4 lg + q][ln] of each 16 x 16 tile
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + wm * 64 + mt * 16 + 4 * lg + q;
        const int k = k0 + wk * 32 + kt * 16 + ln;
        if (m < p.M) {
          uint16_t v = f2bf(acc[mt][kt][q]);
          if (p.add) v = f2bf(bf2f(v) + bf2f(p.add[(int64_t)m * p.lda + k]));
          p.out[(int64_t)m * p.ldo + k] = v;
        }
      }
}

}  // namespace

extern "C" int grpo_nf4_grad_x(const void* grad, int64_t ldg, const uint8_t* w,
                               const float* absmax, const float* code16, int blocksize, int M,
                               int N, int K, const void* addend, int64_t ld_add, void* out,
                               int64_t ldo, grpo_stream_t stream) {
  if (M < 0 || N <= 0 || K <= 0) return einval("M >= 0, N > 0 and K > 0 required");
  if (N % 32) return einval("N must be a multiple of 32");
  if (K % GX_TK) return einval("K must be a multiple of 128");
  if (blocksize <= 0 || blocksize % 8) return einval("blocksize must be a positive multiple of 8");
  if (M == 0) return GRPO_OK;
  if (!grad || !w || !absmax || !code16 || !out) return einval("null pointer");
  if (ldg < N || ldg % 8 || reinterpret_cast<uintptr_t>(grad) % 16)
    return einval("grad rows must be 16-byte aligned with ld >= N");
  if (reinterpret_cast<uintptr_t>(w) % 4) return einval("packed weight must be 4-byte aligned");
  if (ldo < K || (addend && ld_add < K)) return einval("ld >= K required");
  GradXArgs a{static_cast<const uint16_t*>(grad), ldg, w, absmax, code16, blocksize,
              static_cast<const uint16_t*>(addend), ld_add, static_cast<uint16_t*>(out), ldo,
              M, N, K};
  const dim3 grid(K / GX_TK, (M + GX_TM - 1) / GX_TM);
  nf4_grad_x_kernel<<<grid, GX_T, 0, as_stream(stream)>>>(a);
  return launch_check("nf4_grad_x");
}
