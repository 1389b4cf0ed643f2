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

// 8 scaled keys of one 16-byte group of logits.
__device__ __forceinline__ void group_keys(const uint16_t* p, float inv_t, uint32_t (&k)[8]) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k[2 * i] = okey(f2bf(bf_lo(w[i]) * inv_t));
    k[2 * i + 1] = okey(f2bf(bf_hi(w[i]) * inv_t));
  }
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

__global__ void __launch_bounds__(SMP_T) sample_top_p_kernel(SampleArgs a) {
  touch_kernargs<sizeof(SampleArgs)>();
  extern __shared__ uint32_t hist[];  // [SMP_KEYS] counts, later kept bf16 q bits
  __shared__ uint64_t s64[SMP_W];
  __shared__ uint32_t s32[SMP_W];
  __shared__ uint64_t wmass[SMP_W];
  __shared__ uint32_t wties[SMP_W];
  __shared__ int64_t s_cut[4];  // bin, tied tokens kept, tokens above the bin, q62 of the bin
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
  for (int i = tid; i < SMP_KEYS; i += SMP_T) hist[i] = 0;

  // 1. row maximum of the scaled values
  uint32_t kmax = 0;
  for (int g = tid; g < G; g += SMP_T) {
    uint32_t k[8];
    group_keys(row + 8 * (int64_t)g, a.inv_t, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) kmax = max(kmax, k[i]);
  }
  kmax = block_max(kmax, s32);  // (its barriers also order the histogram clear)
  const float mf = bf2f((uint16_t)key_bits(kmax));
  int64_t token = 0;
  int64_t nkept = 1;
  if (!isfinite(mf)) {
    // +inf or NaN maximum: the first index holding it (no distribution exists)
    uint32_t first = 0xFFFFFFFFu;
    for (int g = tid; g < G; g += SMP_T) {
      uint32_t k[8];
      group_keys(row + 8 * (int64_t)g, a.inv_t, k);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (k[i] == kmax) first = min(first, (uint32_t)(8 * g + i));
    }
    first = block_min(first, s32);
    token = first < (uint32_t)a.V ? first : 0;
  } else {
    // 2. counts per distinct value within the window
    for (int g = tid; g < G; g += SMP_T) {
      uint32_t k[8];
      group_keys(row + 8 * (int64_t)g, a.inv_t, k);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float x = bf2f((uint16_t)key_bits(k[i])) - mf;
        if (x > EXP_MIN_X) atomicAdd(&hist[kmax - k[i]], 1u);
      }
    }
    __syncthreads();

    // 3. bin scan; thread t holds bins [t*KPT, (t+1)*KPT) (descending values)
    // (counts stay in LDS and are re-read per phase; e is recomputed for
    // non-empty bins only, which keeps the phase cost at one wave's bins)
    const int b0 = tid * SMP_KPT;
    auto e_of = [&](int bin) {
      return exp_nonpos(bf2f((uint16_t)key_bits(kmax - (uint32_t)bin)) - mf);
    };
    uint64_t z = 0;
    for (int j = 0; j < SMP_KPT; ++j) {
      const uint32_t c = hist[b0 + j];
      if (c) z += (uint64_t)c * to_fixed(e_of(b0 + j), 17592186044416.0f);  // 2^44
    }
    const float zf = (float)block_sum(z, s64) * 5.684341886080802e-14f;  // 2^-44
    // p = bf16(e / Z) in 2^-62 units (recomputed below rather than held)
    auto p62 = [&](int bin) {
      return to_fixed(bf2f(f2bf(e_of(bin) / zf)), 4611686018427387904.0f);
    };
    uint64_t mass = 0;
    uint32_t ntok = 0;
    for (int j = 0; j < SMP_KPT; ++j) {
      const uint32_t c = hist[b0 + j];
      if (c) mass += (uint64_t)c * p62(b0 + j);
      ntok += c;
    }
    uint64_t cum = mass;
    uint32_t above = ntok;
    block_excl_scan(cum, above, s64, s32);
    // first bin whose last token passes the bound, and how many of its ties stay
    uint32_t cut = SMP_KEYS;
    int64_t keep_ties = 0, above_cut = 0;
    if (!a.nofilter) {
      for (int j = 0; j < SMP_KPT && cut == SMP_KEYS; ++j) {
        const uint32_t c = hist[b0 + j];
        if (!c) continue;
        const uint64_t pj = p62(b0 + j);
        const uint64_t end = cum + (uint64_t)c * pj;
        if ((int64_t)end > a.keep) {
          cut = b0 + j;
          above_cut = above;
          keep_ties = a.keep < (int64_t)cum
                          ? 0
                          : (int64_t)min((uint64_t)c, ((uint64_t)a.keep - cum) / pj);
        }
        cum = end;
        above += c;
      }
    }
    const uint32_t gcut = block_min(cut, s32);
    if (cut == gcut && gcut < SMP_KEYS) {
      // the first token in sorted order is always kept
      s_cut[1] = (gcut == 0 && keep_ties == 0) ? 1 : keep_ties;
      s_cut[2] = above_cut;
    }
    __syncthreads();
    const int64_t kties = gcut < SMP_KEYS ? s_cut[1] : 0;
    nkept = gcut < SMP_KEYS ? s_cut[2] + kties : a.V;

    // Z' over the kept tokens, their bf16 probabilities and fixed-point total
    uint64_t zk = 0;
    for (int j = 0; j < SMP_KPT; ++j) {
      const uint32_t bin = b0 + j;
      const uint64_t n = bin < gcut ? hist[bin] : (bin == gcut ? (uint64_t)kties : 0);
      if (n) zk += n * to_fixed(e_of(bin), 17592186044416.0f);
    }
    const float zkf = (float)block_sum(zk, s64) * 5.684341886080802e-14f;
    uint64_t w = 0;
    for (int j = 0; j < SMP_KPT; ++j) {
      const uint32_t bin = b0 + j;
      const uint32_t c = hist[bin];
      const uint16_t qb = (bin <= gcut && c) ? f2bf(e_of(bin) / zkf) : (uint16_t)0;
      const uint64_t q62 = to_fixed(bf2f(qb), 4611686018427387904.0f);
      const uint64_t n = bin < gcut ? c : (bin == gcut ? (uint64_t)kties : 0);
      w += n * q62;
      hist[bin] = qb;
      if (bin == gcut) s_cut[3] = (int64_t)q62;
    }
    const uint64_t W = block_sum(w, s64);  // (its barriers publish hist and s_cut[3])
    const uint64_t qcut = gcut < SMP_KEYS ? (uint64_t)s_cut[3] : 0;

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
    const int g0 = wave * GW, g1 = min(G, g0 + GW);
    // kept mass (excluding the cut bin's ties) and cut-bin ties of this wave's slice
    uint64_t km = 0;
    uint32_t tc = 0;
    for (int g = g0 + lane; g < g1; g += 64) {
      uint32_t k[8];
      group_keys(row + 8 * (int64_t)g, a.inv_t, k);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t bin = kmax - k[i];
        if (bin == gcut) {
          ++tc;
        } else if (bin < (uint32_t)SMP_KEYS) {
          km += to_fixed(bf2f((uint16_t)hist[bin]), 4611686018427387904.0f);
        }
      }
    }
    km = wave_sum(km);
    tc = wave_sum(tc);
    if (lane == 0) {
      wmass[wave] = km;
      wties[wave] = tc;
    }
    if (tid == 0) s_token = -1;
    __syncthreads();
    // the wave whose slice holds t; each thread finds it from the 16 totals
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
      for (int gr = g0; gr < g1; gr += 64) {
        const int g = gr + lane;
        uint32_t k[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        bool valid = g < g1;
        if (valid) group_keys(row + 8 * (int64_t)g, a.inv_t, k);
        uint32_t lt = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) lt += (valid && kmax - k[i] == gcut) ? 1u : 0u;
        uint32_t it = lt;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t x = __shfl_up(it, o);
          if (lane >= o) it += x;
        }
        int64_t rank = ties_before + (it - lt);  // tie rank of this lane's first tie
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
        uint64_t im = lm;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint64_t x = __shfl_up(im, o);
          if (lane >= o) im += x;
        }
        const uint64_t hit = __ballot(base + im > t);
        if (hit) {
          if (lane == __ffsll((unsigned long long)hit) - 1) {
            uint64_t acc = base + im - lm;
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
          break;
        }
        base += __shfl(im, 63);
        ties_before += __shfl(it, 63);
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
