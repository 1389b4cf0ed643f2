// Temperature / top-p sampling of one token per row from bf16 logits, and the
// sampled decode step's row bookkeeping: the reference's fused_logits_sampling
// (src/triton_kernels/fused_ops.py:236-248) and _sample_tokens
// (src/triton_kernels/paged_kv.py:437-450) followed by the row update of
// paged_kv.py:800-820, :938, :978.
//
// The reference sorts the whole vocabulary per row.  This kernel needs no sort:
// one workgroup per row, 1024 threads.
//   1. max: scaled = bf16(logit * (1/T)); the row maximum m of the scaled values
//      (as order-preserving 16-bit keys of their bf16 bit patterns).
//   2. histogram: every token whose scaled value lies within 86 of m gets
//      counted in an LDS bin per distinct bf16 value (bin = key(m) - key); the
//      86-wide window holds at most 33906 distinct bf16 values.  Tokens further
//      down have exp(s - m) < 2^-124, i.e. probability 0 in bf16.
//   3. bin scan: the bins in descending value order are the sorted vocabulary
//      in runs of equal values.  Per bin: e = exp(v - m); Z = sum of count * e
//      (exact fixed-point sum); p = bf16(e / Z); the running sum of p in sorted
//      order (exact, 2^-62 units) locates the cut: the bin where the running sum
//      passes the keep bound and how many of its tied tokens (lowest indices
//      first) stay.  Then Z' over the kept tokens, q = bf16(e / Z') per bin,
//      and W = the fixed-point total of the kept q.
//   4. draw: t = floor(r * W / 2^64) for the row's 64-bit uniform r; the token
//      is the first index whose running sum of kept q (index order) exceeds t.
//      Each wave sums the kept mass of its slice of the row, the wave holding t
//      walks its slice.
// Every rounding point is fixed (a bespoke exp with no fused multiply-adds,
// exact integer sums, correctly rounded float32 division), so the result is a
// deterministic function of (logits, T, top_p, r) that a float32 host
// restatement reproduces bit for bit.

#include <math.h>

#include "common.hpp"
#include "decode_state.hpp"

namespace grpo {
namespace {

constexpr int SMP_T = 1024;                // threads per workgroup
constexpr int SMP_W = SMP_T / 64;          // waves per workgroup
constexpr int SMP_KEYS = 34816;            // LDS bins (>= 33906 values in the window)
constexpr int SMP_KPT = SMP_KEYS / SMP_T;  // bins per thread
constexpr size_t SMP_LDS = (size_t)SMP_KEYS * 4;
constexpr float EXP_MIN_X = -86.0f;
static_assert(SMP_KEYS % SMP_T == 0, "bins must split evenly over the threads");

struct SampleArgs {
  const uint16_t* logits;
  int64_t ld;
  int M, V;
  float inv_t;       // float32(1 / max(T, 1e-6))
  int nofilter;      // top_p >= 1: no cut
  int64_t keep;      // keep a token while the running sum (2^-62 units) <= keep
  const uint64_t* draws;  // [M] uniforms, or null: SplitMix64 of (seed, row, count[row])
  uint64_t seed;
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

// Block-wide sum / max / min through one LDS slot per wave.  Every thread gets
// the result; the trailing barrier lets the slots be reused at once.
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* slots) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
  __syncthreads();
  T s = 0;
#pragma unroll
  for (int w = 0; w < SMP_W; ++w) s += slots[w];
  __syncthreads();
  return s;
}
__device__ __forceinline__ uint32_t block_max(uint32_t v, uint32_t* slots) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, (uint32_t)__shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t s = 0;
#pragma unroll
  for (int w = 0; w < SMP_W; ++w) s = max(s, slots[w]);
  __syncthreads();
  return s;
}
__device__ __forceinline__ uint32_t block_min(uint32_t v, uint32_t* slots) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor(v, o));
  if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t s = 0xFFFFFFFFu;
#pragma unroll
  for (int w = 0; w < SMP_W; ++w) s = min(s, slots[w]);
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

constexpr int SMP_U = 8;     // 16-byte group loads in flight per thread in the row passes
constexpr int SMP_RMAX = 64; // rounds (64 groups each) per wave slice: V <= 16 * 64 * 64 * 8

// Calls f(group index, its 16 bytes) for the groups first, first + stride, ...
// below G, with SMP_U loads issued before any is used (clamped addresses, so
// every load is unconditional and in bounds).
template <typename F>
__device__ __forceinline__ void for_groups(const uint16_t* row, int G, int first, int stride,
                                           F&& f) {
  for (int g = first; g < G; g += SMP_U * stride) {
    uint4 v[SMP_U];
#pragma unroll
    for (int u = 0; u < SMP_U; ++u)
      v[u] = *reinterpret_cast<const uint4*>(row + 8 * (int64_t)min(g + u * stride, G - 1));
#pragma unroll
    for (int u = 0; u < SMP_U; ++u)
      if (g + u * stride < G) f(g + u * stride, v[u]);
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

__global__ void __launch_bounds__(SMP_T) sample_top_p_kernel(SampleArgs a) {
  touch_kernargs<sizeof(SampleArgs)>();
  extern __shared__ uint32_t hist[];  // [SMP_KEYS]: counts, then e (float), then kept q (bf16)
  __shared__ uint64_t s64[SMP_W];
  __shared__ uint32_t s32[SMP_W];
  __shared__ uint64_t wmass[SMP_W];
  __shared__ uint32_t wties[SMP_W];
  __shared__ uint64_t rmass[SMP_W][SMP_RMAX];  // per wave and round: kept mass w/o cut ties
  __shared__ uint32_t rties[SMP_W][SMP_RMAX];  // per wave and round: tokens in the cut bin
  __shared__ int64_t s_cut[4];  // cut bin, its tied tokens kept, tokens above it, its q (2^-62)
  __shared__ int64_t s_token;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m = blockIdx.x;
  const bool bookkeeping = a.tokens != nullptr;
  if (bookkeeping && !a.active[m]) {  // stopped row: no draw, the row state stays put
    if (tid == 0) {
      const int64_t g = a.tokens[m];
      if (a.out_tokens) a.out_tokens[m] = g;
      advance_row(m, g, a.tokens, a.pos, a.count, a.limit, a.active, a.eos, a.generated,
                  a.gen_ld, a.append_pos, a.attn_len);
    }
    return;
  }
  const uint16_t* row = a.logits + (int64_t)m * a.ld;
  const int G = a.V >> 3;
  const float inv_t = a.inv_t;
  for (int i = tid; i < SMP_KEYS; i += SMP_T) hist[i] = 0;
  if (tid == 0) {
    s_cut[0] = SMP_KEYS;
    s_cut[1] = 0;
    s_cut[2] = 0;
    s_cut[3] = 0;
    s_token = -1;
  }

  // 1. row maximum of the scaled values
  uint32_t kmax = 0;
  for_groups(row, G, tid, SMP_T, [&](int, const uint4& v) {
    uint32_t k[8];
    keys_of(v, inv_t, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) kmax = max(kmax, k[i]);
  });
  kmax = block_max(kmax, s32);  // (its barriers also order the clear above)
  const float mf = bf2f((uint16_t)key_bits(kmax));
  int64_t token = 0;
  int64_t nkept = 1;
  if (!isfinite(mf)) {
    // +inf or NaN maximum: the first index holding it (no distribution exists)
    uint32_t first = 0xFFFFFFFFu;
    for_groups(row, G, tid, SMP_T, [&](int g, const uint4& v) {
      uint32_t k[8];
      keys_of(v, inv_t, k);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k[i] == kmax) first = min(first, (uint32_t)(8 * g + i));
    });
    first = block_min(first, s32);
    token = first < (uint32_t)a.V ? first : 0;
  } else {
    // 2. counts per distinct value within the window
    for_groups(row, G, tid, SMP_T, [&](int, const uint4& v) {
      uint32_t k[8];
      keys_of(v, inv_t, k);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = bf2f((uint16_t)key_bits(k[i])) - mf;
        if (x > EXP_MIN_X) atomicAdd(&hist[kmax - k[i]], 1u);
      }
    });
    __syncthreads();

    // 3. bin scan; thread t holds bins [t*KPT, (t+1)*KPT) (descending values).
    // Counts move to registers; each non-empty bin's e is computed once and
    // parked in its LDS slot.
    const int b0 = tid * SMP_KPT;
    uint32_t cnt[SMP_KPT];
#pragma unroll
    for (int j = 0; j < SMP_KPT; ++j) cnt[j] = hist[b0 + j];
    uint64_t z = 0;
#pragma unroll
    for (int j = 0; j < SMP_KPT; ++j) {
      float e = 0.0f;
      if (cnt[j]) {
        e = exp_nonpos(bf2f((uint16_t)key_bits(kmax - (uint32_t)(b0 + j))) - mf);
        z += (uint64_t)cnt[j] * to_fixed(e, 17592186044416.0f);  // 2^44
      }
      hist[b0 + j] = __float_as_uint(e);
      if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    const float zf = (float)block_sum(z, s64) * 5.684341886080802e-14f;  // 2^-44
    // p = bf16(e / Z) in 2^-62 units
    auto p62 = [&](int j) {
      return to_fixed(bf2f(f2bf(__uint_as_float(hist[b0 + j]) / zf)), 4611686018427387904.0f);
    };
    uint64_t mass = 0;
    uint32_t ntok = 0;
#pragma unroll
    for (int j = 0; j < SMP_KPT; ++j) {
      if (cnt[j]) mass += (uint64_t)cnt[j] * p62(j);
      ntok += cnt[j];
      if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // bound the hoisted LDS reads
    }
    uint64_t cum = mass;
    uint32_t above = ntok;
    block_excl_scan(cum, above, s64, s32);
    // The cut: the first bin whose last token's running sum passes the bound,
    // and how many of its tied tokens stay (the first token always stays).
    if (!a.nofilter) {
      if (a.keep < 0) {
        if (tid == 0) {
          s_cut[0] = 0;
          s_cut[1] = 1;
          s_cut[2] = 0;
        }
      } else if ((int64_t)cum <= a.keep && (int64_t)(cum + mass) > a.keep) {
        // this thread's range holds the crossing
        for (int j = 0; j < SMP_KPT; ++j) {
          if (!cnt[j]) continue;
          const uint64_t pj = p62(j);
          const uint64_t end = cum + (uint64_t)cnt[j] * pj;
          if ((int64_t)end > a.keep) {
            const int64_t kt =
                (int64_t)min((uint64_t)cnt[j], ((uint64_t)a.keep - cum) / pj);
            s_cut[0] = b0 + j;
            s_cut[1] = (b0 + j == 0 && kt == 0) ? 1 : kt;
            s_cut[2] = above;
            break;
          }
          cum = end;
          above += cnt[j];
        }
      }
    }
    __syncthreads();
    const uint32_t gcut = (uint32_t)s_cut[0];
    const int64_t kties = s_cut[1];
    nkept = gcut < (uint32_t)SMP_KEYS ? s_cut[2] + kties : a.V;

    // Z' over the kept tokens, their bf16 probabilities q and total W
    auto kept_n = [&](int j) -> uint64_t {
      const uint32_t bin = b0 + j;
      return bin < gcut ? cnt[j] : (bin == gcut ? (uint64_t)kties : 0);
    };
    uint64_t zk = 0;
#pragma unroll
    for (int j = 0; j < SMP_KPT; ++j) {
      const uint64_t n = kept_n(j);
      if (n) zk += n * to_fixed(__uint_as_float(hist[b0 + j]), 17592186044416.0f);
      if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    const float zkf = (float)block_sum(zk, s64) * 5.684341886080802e-14f;
    uint64_t w = 0;
#pragma unroll
    for (int j = 0; j < SMP_KPT; ++j) {
      const uint32_t bin = b0 + j;
      const uint16_t qb =
          (bin <= gcut && cnt[j]) ? f2bf(__uint_as_float(hist[bin]) / zkf) : (uint16_t)0;
      const uint64_t q62 = to_fixed(bf2f(qb), 4611686018427387904.0f);
      w += kept_n(j) * q62;
      hist[bin] = qb;
      if (bin == gcut) s_cut[3] = (int64_t)q62;
      if ((j & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    const uint64_t W = block_sum(w, s64);  // (its barriers publish hist and s_cut[3])
    const uint64_t qcut = gcut < (uint32_t)SMP_KEYS ? (uint64_t)s_cut[3] : 0;

    // 4. draw
    uint64_t r;
    if (a.draws) {
      r = a.draws[m];
    } else {
      const uint32_t step = bookkeeping ? (uint32_t)a.count[m] : 0u;
      r = splitmix64(a.seed + splitmix64(((uint64_t)(uint32_t)m << 32) | step));
    }
    const uint64_t t = __umul64hi(r, W);
    const int GW = (G + SMP_W - 1) / SMP_W;  // groups per wave slice
    const int g0 = min(G, wave * GW), g1 = min(G, g0 + GW);
    const int R = (g1 - g0 + 63) / 64;      // rounds of 64 groups in this slice
    // per round: kept mass outside the cut bin, and tokens in the cut bin
    auto group_q = [&](const uint4& v, uint64_t& km, uint32_t& tc) {
      uint32_t k[8];
      keys_of(v, inv_t, k);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t bin = kmax - k[i];
        if (bin == gcut) {
          ++tc;
        } else if (bin < (uint32_t)SMP_KEYS) {
          km += to_fixed(bf2f((uint16_t)hist[bin]), 4611686018427387904.0f);
        }
      }
    };
    uint64_t wkm = 0;
    uint32_t wtc = 0;
    for (int rb = 0; rb < R; rb += SMP_U) {
      uint4 v[SMP_U];
#pragma unroll
      for (int u = 0; u < SMP_U; ++u)
        v[u] = *reinterpret_cast<const uint4*>(
            row + 8 * (int64_t)min(g0 + (rb + u) * 64 + lane, G - 1));
#pragma unroll
      for (int u = 0; u < SMP_U; ++u) {
        if (rb + u >= R) break;  // wave-uniform
        uint64_t km = 0;
        uint32_t tc = 0;
        if (g0 + (rb + u) * 64 + lane < g1) group_q(v[u], km, tc);
        km = wave_sum(km);
        tc = wave_sum(tc);
        if (lane == 0) {
          rmass[wave][rb + u] = km;
          rties[wave][rb + u] = tc;
        }
        wkm += km;
        wtc += tc;
      }
    }
    if (lane == 0) {
      wmass[wave] = wkm;
      wties[wave] = wtc;
    }
    __syncthreads();
    // the wave whose slice holds t (each thread finds it from the 16 totals)
    uint64_t base = 0;
    int64_t ties_before = 0;
    int hold = SMP_W - 1;
    for (int v = 0; v < SMP_W; ++v) {
      const int64_t kt = min((int64_t)wties[v], max((int64_t)0, kties - ties_before));
      const uint64_t kmv = wmass[v] + (uint64_t)kt * qcut;
      if (t < base + kmv) {
        hold = v;
        break;
      }
      base += kmv;
      ties_before += wties[v];
    }
    if (wave == hold) {
      // the round holding t: lane l looks at round l of the slice
      const uint64_t rm = lane < R ? rmass[wave][lane] : 0;
      const uint32_t rt = lane < R ? rties[wave][lane] : 0;
      uint32_t it = rt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t x = __shfl_up(it, o);
        if (lane >= o) it += x;
      }
      const int64_t tb_round = ties_before + (it - rt);  // cut ties before this round
      const int64_t kt = min((int64_t)rt, max((int64_t)0, kties - tb_round));
      const uint64_t rk = rm + (uint64_t)kt * qcut;
      uint64_t im = rk;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint64_t x = __shfl_up(im, o);
        if (lane >= o) im += x;
      }
      const uint64_t hitr = __ballot(lane < R && base + im > t);
      const int rsel = hitr ? __ffsll((unsigned long long)hitr) - 1 : R - 1;
      const uint64_t rbase = base + __shfl(im - rk, rsel);
      const int64_t rties0 = __shfl(tb_round, rsel);
      // that round: one group per lane
      const int g = g0 + rsel * 64 + lane;
      const bool valid = g < g1;
      const uint4 v = *reinterpret_cast<const uint4*>(row + 8 * (int64_t)min(g, G - 1));
      uint32_t k[8];
      keys_of(v, inv_t, k);
      uint32_t lt = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) lt += (valid && kmax - k[i] == gcut) ? 1u : 0u;
      uint32_t il = lt;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t x = __shfl_up(il, o);
        if (lane >= o) il += x;
      }
      int64_t rank = rties0 + (il - lt);  // tie rank of this lane's first cut-bin token
      uint64_t wq[8];
      uint64_t lm = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t bin = kmax - k[i];
        uint64_t q = 0;
        if (valid) {
          if (bin == gcut) {
            q = rank < kties ? qcut : 0;
            ++rank;
          } else if (bin < (uint32_t)SMP_KEYS) {
            q = to_fixed(bf2f((uint16_t)hist[bin]), 4611686018427387904.0f);
          }
        }
        wq[i] = q;
        lm += q;
      }
      uint64_t ig = lm;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint64_t x = __shfl_up(ig, o);
        if (lane >= o) ig += x;
      }
      const uint64_t hit = __ballot(valid && rbase + ig > t);
      if (hit && lane == __ffsll((unsigned long long)hit) - 1) {
        uint64_t acc = rbase + ig - lm;
        int64_t tok = 8 * (int64_t)g + 7;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (acc + wq[i] > t) {
            tok = 8 * (int64_t)g + i;
            break;
          }
          acc += wq[i];
        }
        s_token = tok;
      }
    }
    __syncthreads();
    token = s_token;
    if (token < 0 || token >= a.V) token = 0;  // unreachable: t < W always lands
  }
  if (tid == 0) {
    if (a.out_tokens) a.out_tokens[m] = token;
    if (a.out_kept) a.out_kept[m] = (int32_t)nkept;
    if (bookkeeping)
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

int launch(const SampleArgs& a, grpo_stream_t stream) {
  static const int rc = hip_check(
      hipFuncSetAttribute(reinterpret_cast<const void*>(sample_top_p_kernel),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)SMP_LDS),
      "hipFuncSetAttribute");
  if (rc) return rc;
  sample_top_p_kernel<<<dim3(a.M), SMP_T, SMP_LDS, as_stream(stream)>>>(a);
  return launch_check("sample_top_p");
}

int check_common(const void* logits, int64_t ld, int M, int V, float temperature) {
  if (M <= 0 || V <= 0) return einval("bad sampling dimensions");
  if (V % 8 || ld % 8 || ld < V) return einval("sampling needs V % 8 == 0 and ld % 8 == 0, ld >= V");
  if (V > SMP_W * SMP_RMAX * 64 * 8) return einval("sampling supports V <= 524288");
  if (!logits || !aligned16(logits)) return einval("logits must be 16-byte aligned");
  if (!(temperature > 0.0f)) return einval("temperature must be > 0 (greedy decoding otherwise)");
  return GRPO_OK;
}

SampleArgs make_args(const void* logits, int64_t ld, int M, int V, float temperature,
                     double top_p) {
  SampleArgs a = {};
  a.logits = static_cast<const uint16_t*>(logits);
  a.ld = ld;
  a.M = M;
  a.V = V;
  a.inv_t = 1.0f / fmaxf(temperature, 1e-6f);
  a.nofilter = top_p >= 1.0 ? 1 : 0;
  a.keep = a.nofilter ? INT64_MAX : keep_bound(top_p);
  return a;
}

}  // namespace
}  // namespace grpo

using namespace grpo;

extern "C" int grpo_sample_top_p(const void* logits, int64_t ld_logits, int M, int V,
                                 float temperature, double top_p, const uint64_t* draws,
                                 int64_t* tokens_out, int32_t* kept_out, grpo_stream_t stream) {
  if (int rc = check_common(logits, ld_logits, M, V, temperature)) return rc;
  if (!draws || !tokens_out) return einval("null draws or tokens");
  SampleArgs a = make_args(logits, ld_logits, M, V, temperature, top_p);
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
                                   int32_t* append_pos, int32_t* attn_len, grpo_stream_t stream) {
  if (int rc = check_common(logits, ld_logits, M, V, temperature)) return rc;
  if (!tokens || !pos || !count || !limit || !active || !eos || !append_pos || !attn_len)
    return einval("null row state");
  if (generated && gen_ld <= 0) return einval("gen_ld must be > 0");
  SampleArgs a = make_args(logits, ld_logits, M, V, temperature, top_p);
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
