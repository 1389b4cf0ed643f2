// Temperature / top-p sampling of one token per row from bf16 logits, and the
// sampled decode step's row bookkeeping: the reference's fused_logits_sampling
// (src/triton_kernels/fused_ops.py:236-248) and _sample_tokens
// (src/triton_kernels/paged_kv.py:437-450) followed by the row update of
// paged_kv.py:800-820, :938, :978.
//
// The reference sorts the whole vocabulary per row.  Here no sort is needed:
// the distinct bf16 values of a row are counted, and the counts in descending
// value order ARE the sorted vocabulary in runs of equal values.  Each row is
// cut into S slices (S * rows ~ 256 workgroups, so the passes over the row use
// the whole chip); five launches:
//   K0 smp_max     (slice, row): the slice's maximum scaled value
//                  (scaled = bf16(logit * (1/T)), as order-preserving 16-bit
//                  keys of the bf16 bit patterns).
//   K1 smp_hist    (slice, row; coarser slices): counts per distinct value within 86 of the row
//                  maximum m in LDS (bin = key(m) - key; at most 33906 values;
//                  tokens further down have exp(s - m) < 2^-124, probability 0
//                  in bf16), added into the row's bins in the workspace.
//   K2 smp_scan    (row): takes the row's bins into LDS (clearing them).  Per bin: e =
//                  exp(v - m); Z = sum count * e (exact fixed point); p =
//                  bf16(e / Z); the exact running sum of p (2^-62 units) in
//                  descending order locates the cut: the bin where the sum
//                  passes the keep bound and how many of its tied tokens
//                  (lowest indices first) stay.  Then Z' over the kept tokens,
//                  q = bf16(e / Z'), and the draw: t = floor(r * W / 2^64), W
//                  the fixed-point total of the kept q, located in the kept
//                  tokens taken in sorted order (value descending, index
//                  ascending): a value and the rank of the token among that
//                  value's tokens.
//   K3 smp_count   (slice, row): tokens of that value per slice.
//   K4 smp_pick    (row): the slice and position of the rank-th such token;
//                  the token; the row bookkeeping.
// Every rounding point is fixed (a bespoke exp with no fused multiply-adds,
// exact integer sums, correctly rounded float32 division), so the token is a
// deterministic function of (logits, T, top_p, r) that a float32 host
// restatement reproduces bit for bit.  The workspace's bins are zero between
// calls (K2 clears what K1 added), so no memset is ever issued: the five
// launches can be captured into a HIP graph and replayed.

#include <math.h>

#include "common.hpp"
#include "decode_state.hpp"

namespace grpo {
namespace {

constexpr int SMP_KEYS = 34816;            // LDS bins (>= 33906 values in the window)
constexpr int SMP_SMAX = 32;               // slices per row at most
constexpr int SMP_T1 = 256;                // threads of the slice kernels K0, K3
constexpr int SMP_TH = 512;                // threads of the histogram kernel K1
constexpr int SMP_T = 1024;                // threads of the row kernels K2, K4
constexpr int SMP_KPT = SMP_KEYS / SMP_T;  // bins per K2 thread
constexpr size_t SMP_LDS = (size_t)SMP_KEYS * 4;
constexpr float EXP_MIN_X = -86.0f;
constexpr int SMP_U = 8;  // 16-byte group loads in flight per thread in the row passes
constexpr int SMP_CMAX = SMP_KEYS / 2;                // entries of the compacted bins
constexpr int SMP_EPT = (SMP_CMAX + SMP_T - 1) / SMP_T;  // entries per thread at most
static_assert(SMP_KEYS % SMP_T == 0 && SMP_KEYS % 4 == 0, "bins must split evenly");

// Per-row workspace.
struct RowWs {
  uint32_t slice_max[SMP_SMAX];  // K0
  uint32_t slice_cnt[SMP_SMAX];  // K3
  int64_t sel_key;               // K2: the drawn token's value (as a key)
  int64_t sel_rank;              // K2: its rank among that value's tokens, index order
  int64_t nkept;                 // K2: tokens in the top-p set
  int64_t pad;
  uint32_t bins[SMP_KEYS];       // K1 adds, K2 reads and clears: zero between calls
};
static_assert(sizeof(RowWs) % 16 == 0, "row workspaces must stay 16-byte aligned");

struct SampleArgs {
  const uint16_t* logits;
  int64_t ld;
  int M, V;
  int S, SG;         // slices per row, 8-token groups per slice (K0, K3)
  int SH, SGH;       // the same for the histogram kernel K1
  float inv_t;       // float32(1 / max(T, 1e-6))
  int nofilter;      // top_p >= 1: no cut
  int64_t keep;      // keep a token while the running sum (2^-62 units) <= keep
  const uint64_t* draws;  // [M] uniforms, or null: SplitMix64 of (seed, row, count[row])
  uint64_t seed;
  RowWs* ws;
  int64_t* out_tokens;    // [M] or null
  int32_t* out_kept;      // [M] or null
  // decode bookkeeping (tokens == null: sampling only)
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

// Order-preserving key of a bf16 bit pattern (a larger value has a larger key).
__device__ __forceinline__ uint32_t okey(uint32_t b) {
  return (b & 0x8000u) ? (b ^ 0xFFFFu) : (b ^ 0x8000u);
}
__device__ __forceinline__ uint32_t key_bits(uint32_t k) {
  return (k & 0x8000u) ? (k ^ 0x8000u) : (k ^ 0xFFFFu);
}

// exp(x) for x <= 0: Cody-Waite reduction x = n*ln2 + r (ln2 split into a
// 14-bit head, so n * head is exact, and a tail), exp(r) by its degree-7 Taylor
// polynomial (|r| <= ln2/2: truncation below 6e-9), scaled by 2^n.  Every
// operation rounds once (no contraction into fused multiply-adds), so a float32
// host restatement reproduces each bit.  x <= -86 gives 0 (exp < 2^-124).
__device__ __forceinline__ float exp_nonpos(float x) {
#pragma clang fp contract(off)
  if (!(x > EXP_MIN_X)) return 0.0f;
  const float n = rintf(x * 1.4426950408889634f);
  const float r = (x - n * 0.693145751953125f) - n * 1.4286068203094173e-06f;
  float p = 1.0f / 5040.0f;
  p = p * r + 1.0f / 720.0f;
  p = p * r + 1.0f / 120.0f;
  p = p * r + 1.0f / 24.0f;
  p = p * r + 1.0f / 6.0f;
  p = p * r + 1.0f / 2.0f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  return ldexpf(p, (int)n);
}

__device__ __forceinline__ uint64_t to_fixed(float v, float scale) {
  return (uint64_t)(v * scale);  // v >= 0; exact power-of-two scaling, truncation
}
constexpr float TWO44 = 17592186044416.0f;
constexpr float TWO62 = 4611686018427387904.0f;
constexpr float TWO_M44 = 5.684341886080802e-14f;

// SplitMix64 output function (Steele, Lea and Flood, OOPSLA 2014).
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Block-wide sum / max over NW waves through one LDS slot per wave.  Every
// thread gets the result; the trailing barrier lets the slots be reused.
template <int NW, typename T>
__device__ __forceinline__ T block_sum(T v, T* slots) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
  __syncthreads();
  T s = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) s += slots[w];
  __syncthreads();
  return s;
}
template <int NW>
__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t* slots) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) s = max(s, slots[w]);
  __syncthreads();
  return s;
}

// Exclusive prefix over the block (thread order) of a (u64, u32) pair.
__device__ __forceinline__ void block_excl_scan(uint64_t& a, uint32_t& b, uint64_t* sa,
                                                uint32_t* sb) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t ia = a;
  uint32_t ib = b;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint64_t ta = __shfl_up(ia, o);
    const uint32_t tb = __shfl_up(ib, o);
    if (lane >= o) {
      ia += ta;
      ib += tb;
    }
  }
  if (lane == 63) {
    sa[wave] = ia;
    sb[wave] = ib;
  }
  __syncthreads();
  uint64_t pa = 0;
  uint32_t pb = 0;
  for (int w = 0; w < wave; ++w) {
    pa += sa[w];
    pb += sb[w];
  }
  __syncthreads();
  a = pa + ia - a;
  b = pb + ib - b;
}

// Calls f(group index, its 16 bytes) for the groups first, first + stride, ...
// below end, with SMP_U loads issued before any is used (clamped addresses, so
// every load is unconditional and in bounds).
template <typename F>
__device__ __forceinline__ void for_groups(const uint16_t* row, int end, int first, int stride,
                                           F&& f) {
  for (int g = first; g < end; g += SMP_U * stride) {
    uint4 v[SMP_U];
#pragma unroll
    for (int u = 0; u < SMP_U; ++u)
      v[u] = *reinterpret_cast<const uint4*>(row + 8 * (int64_t)min(g + u * stride, end - 1));
#pragma unroll
    for (int u = 0; u < SMP_U; ++u)
      if (g + u * stride < end) f(g + u * stride, v[u]);
  }
}

// 8 scaled keys of one 16-byte group of logits.
__device__ __forceinline__ void keys_of(const uint4& v, float inv_t, uint32_t (&k)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k[2 * i] = okey(f2bf(bf_lo(w[i]) * inv_t));
    k[2 * i + 1] = okey(f2bf(bf_hi(w[i]) * inv_t));
  }
}

__device__ __forceinline__ bool row_stopped(const SampleArgs& a, int m) {
  return a.tokens != nullptr && !a.active[m];
}
__device__ __forceinline__ uint32_t row_max_key(const SampleArgs& a, const RowWs& w) {
  uint32_t k = 0;
  for (int i = 0; i < a.S; ++i) k = max(k, w.slice_max[i]);
  return k;
}

// K0: the slice's maximum key.
__global__ void __launch_bounds__(SMP_T1) smp_max_kernel(SampleArgs a) {
  touch_kernargs<sizeof(SampleArgs)>();
  __shared__ uint32_t s32[SMP_T1 / 64];
  const int s = blockIdx.x, m = blockIdx.y;
  if (row_stopped(a, m)) return;
  const uint16_t* row = a.logits + (int64_t)m * a.ld;
  const int G = a.V >> 3, g0 = min(G, s * a.SG), g1 = min(G, g0 + a.SG);
  const float inv_t = a.inv_t;
  uint32_t kmax = 0;
  for_groups(row, g1, g0 + (int)threadIdx.x, SMP_T1, [&](int, const uint4& v) {
    uint32_t k[8];
    keys_of(v, inv_t, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) kmax = max(kmax, k[i]);
  });
  kmax = block_max<SMP_T1 / 64>(kmax, s32);
  if (threadIdx.x == 0) a.ws[m].slice_max[s] = kmax;
}

// K1: the slice's counts per value within the window, added into the row's bins.
__global__ void __launch_bounds__(SMP_TH) smp_hist_kernel(SampleArgs a) {
  touch_kernargs<sizeof(SampleArgs)>();
  extern __shared__ uint32_t hist[];  // [SMP_KEYS]
  const int s = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
  if (row_stopped(a, m)) return;
  RowWs& w = a.ws[m];
  const uint32_t kmax = row_max_key(a, w);
  const float mf = bf2f((uint16_t)key_bits(kmax));
  if (!isfinite(mf)) return;  // no distribution: K2 picks the first maximum
  {
    uint4* h4 = reinterpret_cast<uint4*>(hist);
#pragma unroll
    for (int k = 0; k < (SMP_KEYS / 4 + SMP_TH - 1) / SMP_TH; ++k)
      if (tid + k * SMP_TH < SMP_KEYS / 4) h4[tid + k * SMP_TH] = make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  const uint16_t* row = a.logits + (int64_t)m * a.ld;
  const int G = a.V >> 3, g0 = min(G, s * a.SGH), g1 = min(G, g0 + a.SGH);
  const float inv_t = a.inv_t;
  for_groups(row, g1, g0 + tid, SMP_TH, [&](int, const uint4& v) {
    uint32_t k[8];
    keys_of(v, inv_t, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = bf2f((uint16_t)key_bits(k[i])) - mf;
      if (x > EXP_MIN_X) atomicAdd(&hist[kmax - k[i]], 1u);
    }
  });
  __syncthreads();
  {
    const uint4* h4 = reinterpret_cast<const uint4*>(hist);
#pragma unroll 4
    for (int k = 0; k < (SMP_KEYS / 4 + SMP_TH - 1) / SMP_TH; ++k) {
      const int i4 = tid + k * SMP_TH;
      if (i4 >= SMP_KEYS / 4) break;
      const uint4 c = h4[i4];
      if (c.x) atomicAdd(&w.bins[4 * i4], c.x);
      if (c.y) atomicAdd(&w.bins[4 * i4 + 1], c.y);
      if (c.z) atomicAdd(&w.bins[4 * i4 + 2], c.z);
      if (c.w) atomicAdd(&w.bins[4 * i4 + 3], c.w);
    }
  }
}

// The row's counts from the workspace into LDS (16-byte loads, all issued
// before the stores), the workspace copy cleared for the next call, then a
// barrier.
__device__ __forceinline__ void take_counts(uint32_t* bins, uint32_t* lds) {
  constexpr int N4 = SMP_KEYS / 4, PER = (N4 + SMP_T - 1) / SMP_T;
  uint4* src = reinterpret_cast<uint4*>(bins);
  uint4* dst = reinterpret_cast<uint4*>(lds);
  uint4 v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) v[k] = src[min((int)threadIdx.x + k * SMP_T, N4 - 1)];
#pragma unroll
  for (int k = 0; k < PER; ++k)
    if ((int)threadIdx.x + k * SMP_T < N4) {
      dst[threadIdx.x + k * SMP_T] = v[k];
      src[threadIdx.x + k * SMP_T] = make_uint4(0, 0, 0, 0);
    }
  __syncthreads();
}

// LDS word of a bin: count in bits 0..17 (V < 2^18), and a probability in
// [0, 1] as bf16 bits (at most 0x3F80, 14 bits) in bits 18..31.
constexpr uint32_t CNT_MASK = (1u << 18) - 1;
__device__ __forceinline__ uint32_t cnt_of(uint32_t w) { return w & CNT_MASK; }
__device__ __forceinline__ uint64_t prob62(uint32_t w) {
  return to_fixed(bf2f((uint16_t)(w >> 18)), TWO62);
}

// K2: the row's bin scan: cut, kept probabilities, draw (value and rank).
// The per-bin arithmetic (exp, divisions) runs in balanced passes, thread t
// taking bins t, t + 1024, ... (the populated bins cluster near the top of the
// window); the ordered prefixes run over contiguous ranges, thread t taking
// bins [34t, 34t + 34).  Everything after the first read lives in LDS.
__global__ void __launch_bounds__(SMP_T) smp_scan_kernel(SampleArgs a) {
  touch_kernargs<sizeof(SampleArgs)>();
  extern __shared__ uint32_t lds[];  // [SMP_KEYS] packed (count, p or q) words
  __shared__ uint64_t s64[SMP_T / 64];
  __shared__ uint32_t s32[SMP_T / 64];
  __shared__ int64_t s_cut[3];  // cut bin, its tied tokens kept, tokens above it
  __shared__ int64_t s_sel[2];  // drawn bin, rank within it
  __shared__ uint64_t s_w;
  const int tid = threadIdx.x;
  const int m = blockIdx.x;
  if (row_stopped(a, m)) return;
  RowWs& ws = a.ws[m];
  const uint32_t kmax = row_max_key(a, ws);
  const float mf = bf2f((uint16_t)key_bits(kmax));
  if (!isfinite(mf)) {  // +inf or NaN maximum: the first index holding it
    if (tid == 0) {
      ws.sel_key = kmax;
      ws.sel_rank = 0;
      ws.nkept = 1;
    }
    return;
  }
  if (tid == 0) {
    s_cut[0] = SMP_KEYS;
    s_cut[1] = 0;
    s_cut[2] = 0;
    s_sel[0] = 0;
    s_sel[1] = 0;
  }
  take_counts(ws.bins, lds);
  // e of a bin.  Each pass takes its own opaque copy of (kmax, m): otherwise
  // the compiler keeps every bin's exponent argument live from pass to pass.
  uint32_t km = kmax;
  float mfv = mf;
  auto fresh = [&]() { asm volatile("" : "+v"(km), "+v"(mfv)); };
  auto e_of = [&](int bin) {
    return exp_nonpos(bf2f((uint16_t)key_bits(km - (uint32_t)bin)) - mfv);
  };

  // Compaction: the non-empty bins, in sorted order, as entries (count, bin,
  // probability) so that every pass below takes ~N/1024 consecutive entries
  // per thread instead of 34 mostly-empty bins.  Rows with more than
  // SMP_CMAX distinct values in the window keep the bin-wise passes.
  {
    const int c0 = tid * SMP_KPT;
    uint64_t nzmask = 0;
#pragma unroll
    for (int j = 0; j < SMP_KPT; ++j) nzmask |= (uint64_t)(lds[c0 + j] != 0u) << j;
    const uint64_t mine = (uint64_t)__popcll(nzmask);
    uint64_t off = mine;
    uint32_t unused = 0;
    block_excl_scan(off, unused, s64, s32);
    if (tid == SMP_T - 1) s_w = off + mine;
    __syncthreads();
    const uint32_t N = (uint32_t)s_w;
    if (N <= (uint32_t)SMP_CMAX) {
      uint32_t* ccnt = lds;                                         // [SMP_CMAX]
      uint16_t* cbin = reinterpret_cast<uint16_t*>(lds + SMP_CMAX);  // [SMP_CMAX]
      uint16_t* cprob = cbin + SMP_CMAX;                             // [SMP_CMAX]
      {
        uint32_t c[SMP_KPT];
#pragma unroll
        for (int j = 0; j < SMP_KPT; ++j) c[j] = lds[c0 + j];
        __syncthreads();  // every count is in registers before the entries overwrite them
        uint32_t k = (uint32_t)off;
#pragma unroll
        for (int j = 0; j < SMP_KPT; ++j)
          if (c[j]) {
            ccnt[k] = c[j];
            cbin[k] = (uint16_t)(c0 + j);
            ++k;
          }
      }
      __syncthreads();
      const uint32_t ept = (N + SMP_T - 1) / SMP_T;  // entries per thread (<= SMP_EPT)
      const uint32_t k0 = tid * ept;
      float ev[SMP_EPT];
      // A: e per entry, Z
      fresh();
      uint64_t zc = 0;
#pragma unroll
      for (int i = 0; i < SMP_EPT; ++i) {
        const uint32_t k = k0 + i;
        ev[i] = 0.0f;
        if (i < (int)ept && k < N) {
          ev[i] = e_of(cbin[k]);
          zc += (uint64_t)ccnt[k] * to_fixed(ev[i], TWO44);
        }
      }
      const float zcf = (float)block_sum<SMP_T / 64>(zc, s64) * TWO_M44;
      // B, C: p per entry; running sum in sorted order; the cut (as an entry index)
      uint64_t mass = 0;
      uint32_t ntok = 0;
#pragma unroll
      for (int i = 0; i < SMP_EPT; ++i) {
        const uint32_t k = k0 + i;
        if (i < (int)ept && k < N) {
          const uint16_t pb = f2bf(ev[i] / zcf);
          cprob[k] = pb;
          mass += (uint64_t)ccnt[k] * to_fixed(bf2f(pb), TWO62);
          ntok += ccnt[k];
        }
      }
      uint64_t cum = mass;
      uint32_t above = ntok;
      block_excl_scan(cum, above, s64, s32);
      if (tid == 0) {
        s_cut[0] = N;  // no cut: every entry kept
        s_cut[1] = 0;
        s_cut[2] = 0;
      }
      __syncthreads();
      if (!a.nofilter) {
        if (a.keep < 0) {
          if (tid == 0) {  // entry 0 is bin 0 (the maximum): its first token only
            s_cut[0] = 0;
            s_cut[1] = 1;
            s_cut[2] = 0;
          }
        } else if ((int64_t)cum <= a.keep && (int64_t)(cum + mass) > a.keep) {
          for (uint32_t k = k0; k < min(N, k0 + ept); ++k) {  // this thread holds the crossing
            const uint32_t ck = ccnt[k];
            const uint64_t pk = to_fixed(bf2f(cprob[k]), TWO62);
            const uint64_t end = cum + (uint64_t)ck * pk;
            if ((int64_t)end > a.keep) {
              const int64_t kt = (int64_t)min((uint64_t)ck, ((uint64_t)a.keep - cum) / pk);
              s_cut[0] = k;
              s_cut[1] = (k == 0 && kt == 0) ? 1 : kt;
              s_cut[2] = above;
              break;
            }
            cum = end;
            above += ck;
          }
        }
      }
      __syncthreads();
      const uint32_t kc = (uint32_t)s_cut[0];
      const int64_t kt_c = s_cut[1];
      const int64_t nk = kc < N ? s_cut[2] + kt_c : a.V;
      auto kept_e = [&](uint32_t k) -> uint64_t {
        return k < kc ? ccnt[k] : (k == kc ? (uint64_t)kt_c : 0);
      };
      // D: Z' over the kept entries
      uint64_t zkc = 0;
#pragma unroll
      for (int i = 0; i < SMP_EPT; ++i) {
        const uint32_t k = k0 + i;
        if (i < (int)ept && k < N) zkc += kept_e(k) * to_fixed(ev[i], TWO44);
      }
      const float zkcf = (float)block_sum<SMP_T / 64>(zkc, s64) * TWO_M44;
      // E, F: q per kept entry; kept mass in sorted order; W; the draw
      uint64_t w = 0;
#pragma unroll
      for (int i = 0; i < SMP_EPT; ++i) {
        const uint32_t k = k0 + i;
        if (i < (int)ept && k < N) {
          const uint64_t n = kept_e(k);
          const uint16_t qb = n ? f2bf(ev[i] / zkcf) : (uint16_t)0;
          cprob[k] = qb;
          w += n * to_fixed(bf2f(qb), TWO62);
        }
      }
      uint64_t wpre = w;
      block_excl_scan(wpre, unused, s64, s32);
      if (tid == SMP_T - 1) s_w = wpre + w;
      __syncthreads();
      const uint64_t W = s_w;
      uint64_t r;
      if (a.draws) {
        r = a.draws[m];
      } else {
        const uint32_t step = a.tokens ? (uint32_t)a.count[m] : 0u;
        r = splitmix64(a.seed + splitmix64(((uint64_t)(uint32_t)m << 32) | step));
      }
      const uint64_t t = __umul64hi(r, W);
      if (t >= wpre && t < wpre + w) {  // t lies in this thread's entries
        uint64_t acc = wpre;
        for (uint32_t k = k0; k < min(N, k0 + ept); ++k) {
          const uint64_t n = kept_e(k);
          if (!n) continue;
          const uint64_t q62 = to_fixed(bf2f(cprob[k]), TWO62);
          if (t < acc + n * q62) {  // (then q62 > 0)
            s_sel[0] = cbin[k];
            s_sel[1] = (int64_t)((t - acc) / q62);
            break;
          }
          acc += n * q62;
        }
      }
      __syncthreads();
      if (tid == 0) {
        ws.sel_key = kmax - (uint32_t)s_sel[0];
        ws.sel_rank = s_sel[1];
        ws.nkept = nk;
      }
      return;
    }
  }

  // A (balanced): Z = sum count * e over the bins (2^-44 units)
  uint64_t z = 0;
  fresh();
#pragma unroll
  for (int j = 0; j < SMP_KPT; ++j) {
    const int bin = tid + j * SMP_T;
    const uint32_t c = lds[bin];
    if (c) z += (uint64_t)c * to_fixed(e_of(bin), TWO44);
    if (j & 1) __builtin_amdgcn_sched_barrier(0);  // two exp chains at a time
  }
  const float zf = (float)block_sum<SMP_T / 64>(z, s64) * TWO_M44;
  // B (balanced): p = bf16(e / Z) packed beside the count
  fresh();
#pragma unroll
  for (int j = 0; j < SMP_KPT; ++j) {
    const int bin = tid + j * SMP_T;
    const uint32_t c = lds[bin];
    if (c) lds[bin] = c | ((uint32_t)f2bf(e_of(bin) / zf) << 18);
    if (j & 1) __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();
  // C (contiguous): running sum of p in sorted order; the cut
  const int b0 = tid * SMP_KPT;
  {
    uint64_t mass = 0;
    uint32_t ntok = 0;
#pragma unroll
    for (int j = 0; j < SMP_KPT; ++j) {
      const uint32_t w = lds[b0 + j];
      mass += (uint64_t)cnt_of(w) * prob62(w);
      ntok += cnt_of(w);
      if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    uint64_t cum = mass;
    uint32_t above = ntok;
    block_excl_scan(cum, above, s64, s32);
    // the first bin whose last token's running sum passes the bound, and how
    // many of its tied tokens stay (the first token always stays)
    if (!a.nofilter) {
      if (a.keep < 0) {
        if (tid == 0) {
          s_cut[0] = 0;
          s_cut[1] = 1;
          s_cut[2] = 0;
        }
      } else if ((int64_t)cum <= a.keep && (int64_t)(cum + mass) > a.keep) {
        for (int j = 0; j < SMP_KPT; ++j) {  // this thread's bins hold the crossing
          const uint32_t w = lds[b0 + j];
          const uint32_t cj = cnt_of(w);
          if (!cj) continue;
          const uint64_t pj = prob62(w);
          const uint64_t end = cum + (uint64_t)cj * pj;
          if ((int64_t)end > a.keep) {
            const int64_t kt = (int64_t)min((uint64_t)cj, ((uint64_t)a.keep - cum) / pj);
            s_cut[0] = b0 + j;
            s_cut[1] = (b0 + j == 0 && kt == 0) ? 1 : kt;
            s_cut[2] = above;
            break;
          }
          cum = end;
          above += cj;
        }
      }
    }
  }
  __syncthreads();
  const uint32_t gcut = (uint32_t)s_cut[0];
  const int64_t kties = s_cut[1];
  const int64_t nkept = gcut < (uint32_t)SMP_KEYS ? s_cut[2] + kties : a.V;
  auto kept = [&](uint32_t bin, uint32_t c) -> uint64_t {
    return bin < gcut ? c : (bin == gcut ? (uint64_t)kties : 0);
  };

  // D (balanced): Z' = sum kept * e
  uint64_t zk = 0;
  fresh();
#pragma unroll
  for (int j = 0; j < SMP_KPT; ++j) {
    const int bin = tid + j * SMP_T;
    const uint64_t n = kept((uint32_t)bin, cnt_of(lds[bin]));
    if (n) zk += n * to_fixed(e_of(bin), TWO44);
    if (j & 1) __builtin_amdgcn_sched_barrier(0);
  }
  const float zkf = (float)block_sum<SMP_T / 64>(zk, s64) * TWO_M44;
  // E (balanced): q = bf16(e / Z') of the kept bins in place of p (0 elsewhere)
  fresh();
#pragma unroll
  for (int j = 0; j < SMP_KPT; ++j) {
    const int bin = tid + j * SMP_T;
    const uint32_t c = cnt_of(lds[bin]);
    const uint32_t qb = kept((uint32_t)bin, c) ? f2bf(e_of(bin) / zkf) : 0u;
    lds[bin] = c | (qb << 18);
    if (j & 1) __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();
  // F (contiguous): the kept mass in sorted order, W, and the draw
  {
    uint64_t w = 0;
#pragma unroll
    for (int j = 0; j < SMP_KPT; ++j) {
      const uint32_t v = lds[b0 + j];
      w += kept((uint32_t)(b0 + j), cnt_of(v)) * prob62(v);
      if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    uint64_t wpre = w;
    uint32_t unused = 0;
    block_excl_scan(wpre, unused, s64, s32);
    if (tid == SMP_T - 1) s_w = wpre + w;  // W: the last thread's inclusive prefix
    __syncthreads();
    const uint64_t W = s_w;
    uint64_t r;
    if (a.draws) {
      r = a.draws[m];
    } else {
      const uint32_t step = a.tokens ? (uint32_t)a.count[m] : 0u;
      r = splitmix64(a.seed + splitmix64(((uint64_t)(uint32_t)m << 32) | step));
    }
    const uint64_t t = __umul64hi(r, W);
    if (t >= wpre && t < wpre + w) {  // t lies in this thread's bins
      uint64_t acc = wpre;
      for (int j = 0; j < SMP_KPT; ++j) {
        const uint32_t v = lds[b0 + j];
        const uint64_t n = kept((uint32_t)(b0 + j), cnt_of(v));
        if (!n) continue;
        const uint64_t q62 = prob62(v);
        if (t < acc + n * q62) {  // (then q62 > 0)
          s_sel[0] = b0 + j;
          s_sel[1] = (int64_t)((t - acc) / q62);
          break;
        }
        acc += n * q62;
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    ws.sel_key = kmax - (uint32_t)s_sel[0];
    ws.sel_rank = s_sel[1];
    ws.nkept = nkept;
  }
}

// K3: tokens of the drawn value per slice.
__global__ void __launch_bounds__(SMP_T1) smp_count_kernel(SampleArgs a) {
  touch_kernargs<sizeof(SampleArgs)>();
  __shared__ uint32_t s32[SMP_T1 / 64];
  const int s = blockIdx.x, m = blockIdx.y;
  if (row_stopped(a, m)) return;
  const uint32_t key = (uint32_t)a.ws[m].sel_key;
  const uint16_t* row = a.logits + (int64_t)m * a.ld;
  const int G = a.V >> 3, g0 = min(G, s * a.SG), g1 = min(G, g0 + a.SG);
  const float inv_t = a.inv_t;
  uint32_t c = 0;
  for_groups(row, g1, g0 + (int)threadIdx.x, SMP_T1, [&](int, const uint4& v) {
    uint32_t k[8];
    keys_of(v, inv_t, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) c += k[i] == key ? 1u : 0u;
  });
  c = block_sum<SMP_T1 / 64>(c, s32);
  if (threadIdx.x == 0) a.ws[m].slice_cnt[s] = c;
}

// K4: the rank-th token of the drawn value (index order), and the row update.
__global__ void __launch_bounds__(SMP_T) smp_pick_kernel(SampleArgs a) {
  touch_kernargs<sizeof(SampleArgs)>();
  __shared__ uint64_t s64[SMP_T / 64];
  __shared__ uint32_t s32[SMP_T / 64];
  __shared__ int64_t s_token;
  __shared__ uint64_t s_round;
  const int tid = threadIdx.x, m = blockIdx.x;
  if (row_stopped(a, m)) {  // stopped row: no draw, the row state stays put
    if (tid == 0) {
      const int64_t g = a.tokens[m];
      if (a.out_tokens) a.out_tokens[m] = g;
      advance_row(m, g, a.tokens, a.pos, a.count, a.limit, a.active, a.eos, a.generated,
                  a.gen_ld, a.append_pos, a.attn_len);
    }
    return;
  }
  const RowWs& ws = a.ws[m];
  const uint32_t key = (uint32_t)ws.sel_key;
  int64_t rank = ws.sel_rank;
  int hold = a.S - 1;
  for (int s = 0; s < a.S; ++s) {
    const int64_t c = ws.slice_cnt[s];
    if (rank < c) {
      hold = s;
      break;
    }
    rank -= c;
  }
  if (tid == 0) s_token = -1;
  __syncthreads();
  const uint16_t* row = a.logits + (int64_t)m * a.ld;
  const int G = a.V >> 3, g0 = min(G, hold * a.SG), g1 = min(G, g0 + a.SG);
  const float inv_t = a.inv_t;
  for (int gr = g0; gr < g1; gr += SMP_T) {
    const int g = gr + tid;
    const bool valid = g < g1;
    const uint4 v = *reinterpret_cast<const uint4*>(row + 8 * (int64_t)min(g, G - 1));
    uint32_t k[8];
    keys_of(v, inv_t, k);
    uint32_t hits = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) hits |= (valid && k[i] == key) ? (1u << i) : 0u;
    const uint64_t mine = (uint64_t)__popc(hits);
    uint64_t ex = mine;
    uint32_t unused = 0;
    block_excl_scan(ex, unused, s64, s32);
    if ((int64_t)ex <= rank && rank < (int64_t)(ex + mine)) {
      int left = (int)(rank - (int64_t)ex);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (hits & (1u << i)) {
          if (left == 0) {
            s_token = 8 * (int64_t)g + i;
            break;
          }
          --left;
        }
    }
    if (tid == SMP_T - 1) s_round = ex + mine;  // tokens of the value in this round
    __syncthreads();
    const int64_t found = s_token;
    rank -= (int64_t)s_round;
    __syncthreads();
    if (found >= 0) break;
  }
  int64_t token = s_token;
  if (token < 0 || token >= a.V) token = 0;  // unreachable: the rank lies in the row
  if (tid == 0) {
    if (a.out_tokens) a.out_tokens[m] = token;
    if (a.out_kept) a.out_kept[m] = (int32_t)ws.nkept;
    if (a.tokens)
      advance_row(m, token, a.tokens, a.pos, a.count, a.limit, a.active, a.eos, a.generated,
                  a.gen_ld, a.append_pos, a.attn_len);
  }
}

// Keep bound of the reference's `cumulative > top_p` in bf16: the largest
// running sum (2^-62 units) whose bf16 rounding is <= bf16(top_p).
int64_t keep_bound(double top_p) {
  const uint32_t fb = __builtin_bit_cast(uint32_t, (float)top_p);
  uint32_t b = (fb + 0x7FFFu + ((fb >> 16) & 1u)) >> 16;  // bf16 round-to-nearest-even
  const float bval = __builtin_bit_cast(float, b << 16);
  if (!(bval > 0.0f)) return -1;
  int e;
  frexpf(bval, &e);  // bval = f * 2^e, f in [0.5, 1): spacing above bval is 2^(e-8)
  const double mid = ldexp((double)bval + ldexp(1.0, e - 9), 62);
  const int64_t bound = (int64_t)mid;
  return (b & 1u) ? bound - 1 : bound;
}

template <typename K>
int allow_lds(K kernel) {
  return hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)SMP_LDS),
                   "hipFuncSetAttribute");
}

int launch(SampleArgs a, grpo_stream_t stream) {
  static const int rc = allow_lds(smp_hist_kernel) ? 1 : allow_lds(smp_scan_kernel);
  if (rc) return rc;
  const int G = a.V / 8;
  a.S = max(1, min(SMP_SMAX, 256 / a.M));
  a.SG = (G + a.S - 1) / a.S;
  // fewer, larger histogram slices: each adds its distinct values once into
  // the row's bins, and a slice's fixed cost is clearing and reading 34816 bins
  a.SH = max(1, min(SMP_SMAX, 64 / a.M));
  a.SGH = (G + a.SH - 1) / a.SH;
  hipStream_t st = as_stream(stream);
  const dim3 slices((unsigned)a.S, (unsigned)a.M);
  smp_max_kernel<<<slices, SMP_T1, 0, st>>>(a);
  smp_hist_kernel<<<dim3((unsigned)a.SH, (unsigned)a.M), SMP_TH, SMP_LDS, st>>>(a);
  smp_scan_kernel<<<dim3(a.M), SMP_T, SMP_LDS, st>>>(a);
  smp_count_kernel<<<slices, SMP_T1, 0, st>>>(a);
  smp_pick_kernel<<<dim3(a.M), SMP_T, 0, st>>>(a);
  return launch_check("sample_top_p");
}

int check_common(const void* logits, int64_t ld, int M, int V, float temperature,
                 const void* workspace, size_t workspace_bytes) {
  if (M <= 0 || V <= 0) return einval("bad sampling dimensions");
  if (V % 8 || ld % 8 || ld < V) return einval("sampling needs V % 8 == 0 and ld % 8 == 0, ld >= V");
  if (V >= (1 << 18)) return einval("sampling supports V < 262144");
  if (!logits || !aligned16(logits)) return einval("logits must be 16-byte aligned");
  if (!(temperature > 0.0f)) return einval("temperature must be > 0 (greedy decoding otherwise)");
  if (!workspace || !aligned16(workspace)) return einval("workspace must be 16-byte aligned");
  if (workspace_bytes < (size_t)M * sizeof(RowWs)) return einval("sampling workspace too small");
  return GRPO_OK;
}

SampleArgs make_args(const void* logits, int64_t ld, int M, int V, float temperature,
                     double top_p, void* workspace) {
  SampleArgs a = {};
  a.logits = static_cast<const uint16_t*>(logits);
  a.ld = ld;
  a.M = M;
  a.V = V;
  a.inv_t = 1.0f / fmaxf(temperature, 1e-6f);
  a.nofilter = top_p >= 1.0 ? 1 : 0;
  a.keep = a.nofilter ? INT64_MAX : keep_bound(top_p);
  a.ws = static_cast<RowWs*>(workspace);
  return a;
}

}  // namespace
}  // namespace grpo

using namespace grpo;

extern "C" size_t grpo_sample_workspace_bytes(int M, int V) {
  if (M <= 0 || V <= 0) return 0;
  return (size_t)M * sizeof(RowWs);
}

extern "C" int grpo_sample_top_p(const void* logits, int64_t ld_logits, int M, int V,
                                 float temperature, double top_p, const uint64_t* draws,
                                 int64_t* tokens_out, int32_t* kept_out, void* workspace,
                                 size_t workspace_bytes, grpo_stream_t stream) {
  if (int rc = check_common(logits, ld_logits, M, V, temperature, workspace, workspace_bytes))
    return rc;
  if (!draws || !tokens_out) return einval("null draws or tokens");
  SampleArgs a = make_args(logits, ld_logits, M, V, temperature, top_p, workspace);
  a.draws = draws;
  a.out_tokens = tokens_out;
  a.out_kept = kept_out;
  return launch(a, stream);
}

extern "C" int grpo_sample_advance(const void* logits, int64_t ld_logits, int M, int V,
                                   float temperature, double top_p, uint64_t seed,
                                   int64_t* next_tokens, int64_t* tokens, int32_t* pos,
                                   int32_t* count, const int32_t* limit, uint8_t* active,
                                   const int64_t* eos, int64_t* generated, int64_t gen_ld,
                                   int32_t* append_pos, int32_t* attn_len, void* workspace,
                                   size_t workspace_bytes, grpo_stream_t stream) {
  if (int rc = check_common(logits, ld_logits, M, V, temperature, workspace, workspace_bytes))
    return rc;
  if (!tokens || !pos || !count || !limit || !active || !eos || !append_pos || !attn_len)
    return einval("null row state");
  if (generated && gen_ld <= 0) return einval("gen_ld must be > 0");
  SampleArgs a = make_args(logits, ld_logits, M, V, temperature, top_p, workspace);
  a.seed = seed;
  a.out_tokens = next_tokens;
  a.tokens = tokens;
  a.pos = pos;
  a.count = count;
  a.limit = limit;
  a.active = active;
  a.eos = eos;
  a.generated = generated;
  a.gen_ld = gen_ld;
  a.append_pos = append_pos;
  a.attn_len = attn_len;
  return launch(a, stream);
}
