// NF4 dequantization and the fused NF4 + LoRA linear for gfx950.
//
// Weight format (bitsandbytes Params4bit, read by the reference in
// src/triton_kernels/lora_forward.py:171-206): W[N,K] flattened row-major,
// element e = n*K + k, byte e/2, even e = high nibble; one float32 absmax per
// `blocksize` flat elements; value = bf16_rne(code[q] * absmax).
//
// Fast linear path (M <= 64, K % 256 == 0, N % 16 == 0, blocksize % 64 == 0,
// r <= 16): D = A*B on v_mfma_f32_16x16x32_bf16 with A = x (rows m) and
// B = W^T (columns n).  Each lane owns one 64-element chunk of one weight row
// per 256-wide k-step (32 bytes, two 16-byte loads), builds a 16-entry bf16
// codebook for that chunk's absmax block in registers (so every product is
// exactly the reference's bf16(code*absmax) * x), and expands nibbles with
// v_perm byte lookups.  The decode emits each dword's eight elements in the
// order [0,2,4,6,1,3,5,7]; x is staged in LDS in that same order, so MFMA sums
// the right pairs.  The LoRA-A product x*A^T is one more 16-column MFMA tile of
// the same k-loop (A is bf16, no decode).  Split-K across workgroups reduces
// through a caller workspace; the last workgroup of each 64-row group (found
// with a device-scope counter, no spinning) sums the partials in split order
// and runs the epilogue, so results do not depend on arrival order.
#include "common.hpp"

using namespace grpo;

namespace {

constexpr int KSTEP = 256;       // k elements per step: 4 lane groups x 64
constexpr int WG_ROWS = 64;      // weight rows per workgroup: 4 waves x 16
constexpr int LDS_BYTES = 65536;
constexpr int TARGET_WGS = 512;  // launch-shape heuristic (2 per CU on 256 CUs)
constexpr size_t COUNTER_BYTES = 65536;  // split-K group counters: up to 16384 groups of 64 rows

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

// ------------------------------------------------------ fast linear --

struct LinearArgs {
  const uint16_t* x;
  int64_t ldx;
  const uint8_t* w;
  const float* absmax;
  const float* code16;
  int blocksize;
  const uint16_t* bias;
  const uint16_t* la;  // lora A [r, K]
  const uint16_t* lb;  // lora B [N, r]
  int r;
  float scaling;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int S, kps;      // k-splits and k-steps per split
  float* ws_acc;   // [S][M][N]
  float* ws_t;     // [NG][S][M][16]
  int* ws_cnt;     // [NG]
};

struct LinearPlan {
  int MT, KS, NG, S, kps;
  size_t off_cnt, off_acc, off_t, bytes;
};

LinearPlan plan_linear(int M, int N, int K, int r) {
  LinearPlan p{};
  p.MT = (M + 15) / 16;
  p.KS = K / KSTEP;
  p.NG = (N + WG_ROWS - 1) / WG_ROWS;
  const int tred = 4 * p.MT * 16 * 16 * 4;
  int kps_lds = ((LDS_BYTES - tred - 256) / (M * 2) - 8) / KSTEP;
  if (kps_lds < 1) kps_lds = 1;
  int S = (TARGET_WGS + p.NG - 1) / p.NG;
  if (S > p.KS) S = p.KS;
  if (S < 1) S = 1;
  int kps = (p.KS + S - 1) / S;
  if (kps > kps_lds) kps = kps_lds;
  S = (p.KS + kps - 1) / kps;
  p.S = S;
  p.kps = kps;
  if (S > 1) {
    // Counters live at a fixed offset (0) for every shape: a workspace reused
    // across shapes then always finds them where the last call left them (zero),
    // never on top of another shape's partial sums.
    auto align = [](size_t v) { return (v + 255) & ~(size_t)255; };
    size_t acc = align((size_t)S * M * N * 4);
    size_t tb = r > 0 ? align((size_t)p.NG * S * M * 16 * 4) : 0;
    p.off_cnt = 0;
    p.off_acc = COUNTER_BYTES;
    p.off_t = COUNTER_BYTES + acc;
    p.bytes = COUNTER_BYTES + acc + tb;
  }
  return p;
}

template <int MT, bool LORA>
__global__ void __launch_bounds__(256) nf4_linear_mfma(LinearArgs p) {
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int ng = blockIdx.x, s = blockIdx.y;
  const int KS = p.K / KSTEP;
  const int ks0 = s * p.kps;
  const int ks1 = min(ks0 + p.kps, KS);
  const int nsteps = ks1 - ks0;
  const int xstride = p.kps * KSTEP + 8;  // LDS row stride in elements (16B pad)
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* tred = reinterpret_cast<float*>(smem + (size_t)p.M * xstride * 2);  // [4][MT*16][16]
  int* flag = reinterpret_cast<int*>(tred + 4 * MT * 16 * 16);

  // Stage x[0:M, ks0*256 : ks1*256] into LDS, 8 elements per 16 bytes,
  // deinterleaved to the decode8 order.
  {
    const int chunks = nsteps * (KSTEP / 8);
    const int total = p.M * chunks;
    const int kg = ks0 * KSTEP;
    for (int i = tid; i < total; i += 256) {
      const int m = i / chunks, c = i - m * chunks;
      const uint4 v = *reinterpret_cast<const uint4*>(p.x + (int64_t)m * p.ldx + kg + c * 8);
      *reinterpret_cast<uint4*>(xs + m * xstride + c * 8) = deinterleave8(v);
    }
  }
  float code[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) code[j] = p.code16[j];
  __syncthreads();

  const int n_row = ng * WG_ROWS + wave * 16 + ln;
  const bool row_ok = n_row < p.N;
  const uint8_t* wrow = p.w + (int64_t)(row_ok ? n_row : 0) * (p.K / 2);
  f32x4_t acc[MT];
  f32x4_t tacc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    tacc[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  for (int it = 0; it < nsteps; ++it) {
    const int kc = (ks0 + it) * KSTEP + 64 * lg;  // this lane's chunk (global k)
    const int kl = it * KSTEP + 64 * lg;           // same chunk in LDS
    uint4 w0 = make_uint4(0, 0, 0, 0), w1 = w0;
    float a = 0.f;
    if (row_ok) {
      const uint4* wp = reinterpret_cast<const uint4*>(wrow + kc / 2);
      w0 = wp[0];
      w1 = wp[1];
      a = p.absmax[((int64_t)n_row * p.K + kc) / p.blocksize];
    }
    const Lut t = make_lut(code, a);
    const uint32_t wd[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint4 bw = decode8(wd[j], t);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + ln;
        uint4 ax = make_uint4(0, 0, 0, 0);
        if (m < p.M) ax = *reinterpret_cast<const uint4*>(xs + m * xstride + kl + 8 * j);
        acc[mt] = mfma16x16x32(ax, bw, acc[mt]);
      }
    }
    if (LORA && (it & 3) == wave) {
      // LoRA-A tile: columns are the r rows of A (rows >= r read as zero).
      const bool r_ok = ln < p.r;
      const uint16_t* arow = p.la + (int64_t)(r_ok ? ln : 0) * p.K + kc;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint4 bv = make_uint4(0, 0, 0, 0);
        if (r_ok) bv = deinterleave8(*reinterpret_cast<const uint4*>(arow + 8 * j));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = mt * 16 + ln;
          uint4 ax = make_uint4(0, 0, 0, 0);
          if (m < p.M) ax = *reinterpret_cast<const uint4*>(xs + m * xstride + kl + 8 * j);
          tacc[mt] = mfma16x16x32(ax, bv, tacc[mt]);
        }
      }
    }
  }

  // Sum the four waves' LoRA-A partials: tred[wave][m][r].
  if (LORA) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        tred[(wave * MT * 16 + mt * 16 + 4 * lg + q) * 16 + ln] = tacc[mt][q];
    __syncthreads();
    for (int i = tid; i < MT * 16 * 16; i += 256)
      tred[i] = tred[i] + tred[MT * 256 + i] + tred[2 * MT * 256 + i] + tred[3 * MT * 256 + i];
    __syncthreads();
  }

  if (p.S > 1) {
    // Publish this split's partials, then let the last split of the group finish.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mt * 16 + 4 * lg + q;
        if (m < p.M && row_ok) p.ws_acc[((int64_t)s * p.M + m) * p.N + n_row] = acc[mt][q];
      }
    if (LORA) {
      float* dst = p.ws_t + ((int64_t)ng * p.S + s) * p.M * 16;
      for (int i = tid; i < p.M * 16; i += 256) dst[i] = tred[i];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const int old = atomicAdd(p.ws_cnt + ng, 1);
      *flag = (old == p.S - 1);
    }
    __syncthreads();
    if (!*flag) return;
    __threadfence();
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = mt * 16 + 4 * lg + q;
        float v = 0.f;
        if (m < p.M && row_ok)
          for (int ss = 0; ss < p.S; ++ss) v += p.ws_acc[((int64_t)ss * p.M + m) * p.N + n_row];
        acc[mt][q] = v;
      }
    if (LORA) {
      const float* src = p.ws_t + (int64_t)ng * p.S * p.M * 16;
      for (int i = tid; i < p.M * 16; i += 256) {
        float v = 0.f;
        for (int ss = 0; ss < p.S; ++ss) v += src[(int64_t)ss * p.M * 16 + i];
        tred[i] = v;
      }
    }
    if (tid == 0) p.ws_cnt[ng] = 0;
    __syncthreads();
  }

  // Epilogue: y = bf16(bf16(bf16(acc) + bias) + bf16(bf16(bf16(T) B^T) * bf16(s))).
  if (LORA) {
    for (int i = tid; i < p.M * 16; i += 256) tred[i] = round_bf(tred[i]);
    __syncthreads();
  }
  if (!row_ok) return;
  const float bias = p.bias ? bf2f(p.bias[n_row]) : 0.f;
  float bl[16];
  if (LORA) {
#pragma unroll
    for (int q = 0; q < 16; ++q) bl[q] = q < p.r ? bf2f(p.lb[(int64_t)n_row * p.r + q]) : 0.f;
  }
  const float sc = round_bf(p.scaling);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int m = mt * 16 + 4 * lg + q;
      if (m >= p.M) continue;
      float v = round_bf(acc[mt][q]);
      if (p.bias) v = round_bf(v + bias);
      if (LORA) {
        const float* tr = tred + m * 16;
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
  if (p.bias) v = round_bf(v + bf2f(p.bias[n]));
  if (p.r > 0) {
    float u = 0.f;
    for (int rr = 0; rr < p.r; ++rr) {
      const uint16_t* ar = p.la + (int64_t)rr * p.K;
      float t = 0.f;
      for (int k = 0; k < p.K; ++k) t += bf2f(xr[k]) * bf2f(ar[k]);
      u += round_bf(t) * bf2f(p.lb[(int64_t)n * p.r + rr]);
    }
    u = round_bf(round_bf(u) * round_bf(p.scaling));
    v = round_bf(v + u);
  }
  p.y[(int64_t)m * p.ldy + n] = f2bf(v);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

bool use_fast_linear(const LinearArgs& a) {
  return a.M <= 64 && a.K % KSTEP == 0 && a.N % 16 == 0 && a.blocksize % 64 == 0 && a.r <= 16 &&
         (a.N + WG_ROWS - 1) / WG_ROWS <= (int)(COUNTER_BYTES / 4) &&
         a.ldx % 8 == 0 && aligned16(a.x) && aligned16(a.w) && (a.r == 0 || a.K % 8 == 0) &&
         (a.r == 0 || aligned16(a.la));
}

template <int MT>
int launch_fast(const LinearArgs& a, const LinearPlan& plan, hipStream_t st) {
  const size_t lds = (size_t)a.M * (plan.kps * KSTEP + 8) * 2 + 4 * MT * 16 * 16 * 4 + 16;
  dim3 grid(plan.NG, plan.S);
  if (a.r > 0)
    nf4_linear_mfma<MT, true><<<grid, 256, lds, st>>>(a);
  else
    nf4_linear_mfma<MT, false><<<grid, 256, lds, st>>>(a);
  return launch_check("nf4_linear_mfma");
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

extern "C" size_t grpo_nf4_lora_linear_workspace_bytes(int M, int N, int K, int r) {
  if (M <= 0 || N <= 0 || K <= 0 || M > 64 || K % KSTEP != 0 || N % 16 != 0 || r > 16) return 0;
  if ((N + WG_ROWS - 1) / WG_ROWS > (int)(COUNTER_BYTES / 4)) return 0;
  return plan_linear(M, N, K, r).bytes;
}

extern "C" int grpo_nf4_lora_linear(const void* x, int64_t ldx, const uint8_t* w,
                                    const float* absmax, const float* code16, int blocksize,
                                    const void* bias, const void* lora_a, const void* lora_b, int r,
                                    float scaling, void* y, int64_t ldy, int M, int N, int K,
                                    void* workspace, size_t workspace_bytes,
                                    grpo_stream_t stream) {
  if (M < 0 || N < 0 || K < 0) return einval("negative dimension");
  if (r < 0) return einval("r < 0");
  if (blocksize <= 0) return einval("blocksize must be > 0");
  if (M == 0 || N == 0) return GRPO_OK;
  if (!x || !w || !absmax || !code16 || !y) return einval("null pointer");
  if (r > 0 && (!lora_a || !lora_b)) return einval("r > 0 needs lora_a and lora_b");
  if (ldx < K || ldy < N) return einval("row stride smaller than the row");
  LinearArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.w = w;
  a.absmax = absmax;
  a.code16 = code16;
  a.blocksize = blocksize;
  a.bias = static_cast<const uint16_t*>(bias);
  a.la = static_cast<const uint16_t*>(lora_a);
  a.lb = static_cast<const uint16_t*>(lora_b);
  a.r = r;
  a.scaling = scaling;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  hipStream_t st = as_stream(stream);
  if (K > 0 && use_fast_linear(a)) {
    const LinearPlan plan = plan_linear(M, N, K, r);
    a.S = plan.S;
    a.kps = plan.kps;
    if (plan.S > 1) {
      if (!workspace || workspace_bytes < plan.bytes) {
        set_error("invalid argument: workspace of %zu bytes needed, %zu given", plan.bytes,
                  workspace_bytes);
        return GRPO_EWORKSPACE;
      }
      uint8_t* ws = static_cast<uint8_t*>(workspace);
      a.ws_cnt = reinterpret_cast<int*>(ws + plan.off_cnt);
      a.ws_acc = reinterpret_cast<float*>(ws + plan.off_acc);
      a.ws_t = reinterpret_cast<float*>(ws + plan.off_t);
    }
    switch (plan.MT) {
      case 1: return launch_fast<1>(a, plan, st);
      case 2: return launch_fast<2>(a, plan, st);
      case 3: return launch_fast<3>(a, plan, st);
      default: return launch_fast<4>(a, plan, st);
    }
  }
  const int64_t total = (int64_t)M * N;
  nf4_linear_generic<<<dim3((unsigned)cdiv(total, 256)), 256, 0, st>>>(a);
  return launch_check("nf4_linear_generic");
}
