// Paged KV append and single-query (decode) paged attention with GQA, gfx950.
//
// Cache: bf16 [num_blocks, Hkv, block_size, D]; block_tables int32 [B, max_blocks];
// context_lens int32 [B] (device-resident, read-only here).
//
// Fast decode path (D == 128, block_size == 16, Hq/Hkv <= 8): grid
// (context split, KV head, sequence), 4 waves per workgroup; every wave walks
// its share of the split's 16-token blocks.  Per block the 4 KB K tile is read
// with 16-byte loads straight into the A operand of v_mfma_f32_16x16x32_bf16
// (rows = tokens) against the B operand Q^T of all query heads of the GQA group
// (columns = heads), giving S^T[token][head] in 4 MFMAs.  The online softmax
// runs in the exp2 domain; P and the per-head rescale go through a per-wave LDS
// slot; P.V runs on VALU with every V element loaded once and applied to all
// heads of the group.  Waves merge through LDS; sequences needing several
// splits write (max, sum, unnormalised O) partials that a second kernel merges
// with log-sum-exp weights.  K and V of a KV head are therefore read once per
// step, not once per query head.
#include <math.h>

#include "common.hpp"

using namespace grpo;

namespace {

constexpr int FD = 128;  // fast-path head dim
constexpr int FBS = 16;  // fast-path block size
constexpr int TARGET_WAVES = 1024;
constexpr float LOG2E = 1.4426950408889634f;

struct AttnArgs {
  const uint16_t* q;
  int64_t qsb, qsh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t num_blocks;
  const int32_t* bt;
  int64_t bts;
  const int32_t* cl;
  void* out;
  int out_bf16;
  int B, Hq, Hkv, D, BS, max_blocks;
  float scale;
  int bps;       // blocks per split
  int S;         // splits allocated in the workspace
  float* ws_o;   // [B][Hq][S][D]
  float* ws_ml;  // [B][Hq][S][2]
};

struct AttnPlan {
  bool fast;
  int bps, S;
  size_t bytes;
};

AttnPlan plan_attn(int B, int Hq, int Hkv, int D, int BS, int max_blocks) {
  AttnPlan p{};
  p.fast = D == FD && BS == FBS && Hkv > 0 && Hq % Hkv == 0 && Hq / Hkv <= 8;
  if (!p.fast) {
    p.bps = max_blocks > 0 ? max_blocks : 1;
    p.S = 1;
    return p;
  }
  const int64_t total = (int64_t)B * Hkv * max_blocks;
  int64_t bpw = total / TARGET_WAVES;
  if (bpw < 1) bpw = 1;
  p.bps = (int)(4 * bpw);
  p.S = max_blocks > 0 ? (int)cdiv(max_blocks, p.bps) : 1;
  if (p.S > 1) p.bytes = (size_t)B * Hq * p.S * (D + 2) * 4;
  return p;
}

__device__ __forceinline__ int seq_ctx(const AttnArgs& p, int b) {
  int c = p.cl[b];
  const int cap = p.max_blocks * p.BS;
  return c < 0 ? 0 : (c > cap ? cap : c);
}

__device__ __forceinline__ void store_out(const AttnArgs& p, int64_t idx, float v) {
  if (p.out_bf16)
    static_cast<uint16_t*>(p.out)[idx] = f2bf(v);
  else
    static_cast<float*>(p.out)[idx] = v;
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int GQ>
__global__ void __launch_bounds__(256) paged_attn_mfma(AttnArgs p) {
  const int s = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int ctx = seq_ctx(p, b);
  const int nblk = (ctx + FBS - 1) / FBS;
  const int nsplit = nblk > 0 ? (nblk + p.bps - 1) / p.bps : 1;
  if (s >= nsplit) return;
  const int blk0 = s * p.bps;
  const int blk1 = min(blk0 + p.bps, nblk);

  __shared__ __align__(16) float sP[4][16][16];
  __shared__ float sC[4][16];
  __shared__ float sM[4][16];
  __shared__ float sL[4][16];
  __shared__ __align__(16) float sO[4][GQ][FD];

  // Q^T as the MFMA B operand: lane (head ln, group lg) holds
  // Q[head][8*lg + 32*i + 0..7] for MFMA i.
  uint4 qf[4];
  {
    const bool hv = ln < GQ;
    const uint16_t* qrow =
        p.q + (int64_t)b * p.qsb + (int64_t)(kvh * GQ + (hv ? ln : 0)) * p.qsh;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      qf[i] = hv ? *reinterpret_cast<const uint4*>(qrow + 8 * lg + 32 * i) : make_uint4(0, 0, 0, 0);
  }
  const float sl2 = p.scale * LOG2E;
  float m_run = -INFINITY, l_run = 0.f;  // softmax state of head ln
  float o[GQ][8];
#pragma unroll
  for (int h = 0; h < GQ; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) o[h][j] = 0.f;

  const int64_t head_stride = (int64_t)FBS * FD;
  for (int blk = blk0 + wave; blk < blk1; blk += 4) {
    const int phys = p.bt[(int64_t)b * p.bts + blk];
    if (phys < 0 || phys >= p.num_blocks) continue;
    const uint16_t* kb = p.kc + ((int64_t)phys * p.Hkv + kvh) * head_stride;
    const uint16_t* vb = p.vc + ((int64_t)phys * p.Hkv + kvh) * head_stride;
    uint4 kf[4], vf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) kf[i] = *reinterpret_cast<const uint4*>(kb + ln * FD + 8 * lg + 32 * i);
#pragma unroll
    for (int i = 0; i < 4; ++i) vf[i] = *reinterpret_cast<const uint4*>(vb + (4 * lg + i) * FD + 8 * ln);

    f32x4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) sacc = mfma16x16x32(kf[i], qf[i], sacc);
    // lane (head ln, lg) now holds S[token 4*lg + r][head ln], r = 0..3.
    float sv[4];
    float bmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = blk * FBS + 4 * lg + r;
      sv[r] = t < ctx ? sacc[r] * sl2 : -INFINITY;
      bmax = fmaxf(bmax, sv[r]);
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
    const float m_new = fmaxf(m_run, bmax);  // finite: token blk*16 < ctx
    const float corr = exp2f(m_run - m_new);
    float pv[4];
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pv[r] = exp2f(sv[r] - m_new);
      ps += pv[r];
    }
    ps += __shfl_xor(ps, 16);
    ps += __shfl_xor(ps, 32);
    l_run = l_run * corr + ps;
    m_run = m_new;
    *reinterpret_cast<float4*>(&sP[wave][ln][4 * lg]) = make_float4(pv[0], pv[1], pv[2], pv[3]);
    if (lg == 0) sC[wave][ln] = corr;
    wave_sync();
    // P.V: lane (token group lg, d chunk ln) owns O[h][8*ln + j] over tokens 4*lg..4*lg+3.
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      const float c = sC[wave][h];
      const float4 ph = *reinterpret_cast<const float4*>(&sP[wave][h][4 * lg]);
      const float pr[4] = {ph.x, ph.y, ph.z, ph.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) o[h][j] *= c;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t vw[4] = {vf[r].x, vf[r].y, vf[r].z, vf[r].w};
#pragma unroll
        for (int c2 = 0; c2 < 4; ++c2) {
          o[h][2 * c2] += pr[r] * bf_lo(vw[c2]);
          o[h][2 * c2 + 1] += pr[r] * bf_hi(vw[c2]);
        }
      }
    }
    wave_sync();
  }

  // Sum the four token groups of the wave, then merge the four waves.
#pragma unroll
  for (int h = 0; h < GQ; ++h)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      o[h][j] += __shfl_xor(o[h][j], 16);
      o[h][j] += __shfl_xor(o[h][j], 32);
    }
  if (lg == 0) {
    sM[wave][ln] = m_run;
    sL[wave][ln] = l_run;
#pragma unroll
    for (int h = 0; h < GQ; ++h) {
      *reinterpret_cast<float4*>(&sO[wave][h][8 * ln]) =
          make_float4(o[h][0], o[h][1], o[h][2], o[h][3]);
      *reinterpret_cast<float4*>(&sO[wave][h][8 * ln + 4]) =
          make_float4(o[h][4], o[h][5], o[h][6], o[h][7]);
    }
  }
  __syncthreads();
  for (int i = tid; i < GQ * FD; i += 256) {
    const int h = i / FD, d = i - h * FD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, sM[w][h]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = exp2f(sM[w][h] - M);
        L += f * sL[w][h];
        O += f * sO[w][h][d];
      }
    }
    const int hq = kvh * GQ + h;
    if (nsplit == 1) {
      store_out(p, ((int64_t)b * p.Hq + hq) * FD + d, O / fmaxf(L, 1e-6f));
    } else {
      const int64_t slot = ((int64_t)b * p.Hq + hq) * p.S + s;
      p.ws_o[slot * FD + d] = O;
      if (d == 0) {
        p.ws_ml[slot * 2] = M;
        p.ws_ml[slot * 2 + 1] = L;
      }
    }
  }
}

// Combine split partials: out = sum_s 2^(m_s - M) O_s / max(sum_s 2^(m_s - M) l_s, 1e-6).
__global__ void __launch_bounds__(128) paged_attn_merge(AttnArgs p) {
  const int hq = blockIdx.x, b = blockIdx.y;
  const int ctx = seq_ctx(p, b);
  const int nblk = (ctx + p.BS - 1) / p.BS;
  const int nsplit = nblk > 0 ? (nblk + p.bps - 1) / p.bps : 1;
  if (nsplit <= 1) return;
  const int64_t base = ((int64_t)b * p.Hq + hq) * p.S;
  float M = -INFINITY;
  for (int s = 0; s < nsplit; ++s) M = fmaxf(M, p.ws_ml[(base + s) * 2]);
  const bool any = M != -INFINITY;  // false only if every block id was invalid
  float L = 0.f;
  if (any)
    for (int s = 0; s < nsplit; ++s)
      L += exp2f(p.ws_ml[(base + s) * 2] - M) * p.ws_ml[(base + s) * 2 + 1];
  const float inv = 1.f / fmaxf(L, 1e-6f);
  for (int d = threadIdx.x; d < p.D; d += blockDim.x) {
    float O = 0.f;
    if (any)
      for (int s = 0; s < nsplit; ++s)
        O += exp2f(p.ws_ml[(base + s) * 2] - M) * p.ws_o[(base + s) * p.D + d];
    store_out(p, ((int64_t)b * p.Hq + hq) * p.D + d, O * inv);
  }
}

// Any D (<= 512) / block size / GQA ratio: one workgroup per (sequence, query
// head); chunks of 256 tokens, online softmax, float32 throughout.
constexpr int GEN_T = 128;
constexpr int GEN_CHUNK = 256;
constexpr int GEN_MAXD = 512;

__global__ void __launch_bounds__(GEN_T) paged_attn_generic(AttnArgs p) {
  const int hq = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
  const int kvh = hq / (p.Hq / p.Hkv);
  const int ctx = seq_ctx(p, b);
  __shared__ float sq[GEN_MAXD];
  __shared__ float sp[GEN_CHUNK];
  __shared__ float red[GEN_T];
  const uint16_t* qrow = p.q + (int64_t)b * p.qsb + (int64_t)hq * p.qsh;
  for (int d = tid; d < p.D; d += GEN_T) sq[d] = bf2f(qrow[d]);
  __syncthreads();
  float o[GEN_MAXD / GEN_T];
#pragma unroll
  for (int i = 0; i < GEN_MAXD / GEN_T; ++i) o[i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const int64_t hs = (int64_t)p.BS * p.D;
  for (int c0 = 0; c0 < ctx; c0 += GEN_CHUNK) {
    const int cn = min(GEN_CHUNK, ctx - c0);
    float lmax = -INFINITY;
    for (int i = tid; i < cn; i += GEN_T) {
      const int t = c0 + i;
      const int phys = p.bt[(int64_t)b * p.bts + t / p.BS];
      float logit = -INFINITY;
      if (phys >= 0 && phys < p.num_blocks) {
        const uint16_t* kr = p.kc + ((int64_t)phys * p.Hkv + kvh) * hs + (int64_t)(t % p.BS) * p.D;
        float dot = 0.f;
        for (int d = 0; d < p.D; ++d) dot += sq[d] * bf2f(kr[d]);
        logit = dot * p.scale;
      }
      sp[i] = logit;
      lmax = fmaxf(lmax, logit);
    }
    red[tid] = lmax;
    __syncthreads();
    for (int w = GEN_T / 2; w > 0; w >>= 1) {
      if (tid < w) red[tid] = fmaxf(red[tid], red[tid + w]);
      __syncthreads();
    }
    const float m_new = fmaxf(m_run, red[0]);
    __syncthreads();
    const float corr = m_new == -INFINITY ? 1.f : expf(m_run - m_new);
    float lsum = 0.f;
    for (int i = tid; i < cn; i += GEN_T) {
      const float e = m_new == -INFINITY ? 0.f : expf(sp[i] - m_new);
      sp[i] = e;
      lsum += e;
    }
    red[tid] = lsum;
    __syncthreads();
    for (int w = GEN_T / 2; w > 0; w >>= 1) {
      if (tid < w) red[tid] += red[tid + w];
      __syncthreads();
    }
    l_run = l_run * corr + red[0];
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < GEN_MAXD / GEN_T; ++i) {
      const int d = tid + i * GEN_T;
      if (d >= p.D) break;
      float acc = o[i] * corr;
      for (int j = 0; j < cn; ++j) {
        const int t = c0 + j;
        const int phys = p.bt[(int64_t)b * p.bts + t / p.BS];
        if (phys < 0 || phys >= p.num_blocks) continue;
        const uint16_t* vr = p.vc + ((int64_t)phys * p.Hkv + kvh) * hs + (int64_t)(t % p.BS) * p.D;
        acc += sp[j] * bf2f(vr[d]);
      }
      o[i] = acc;
    }
    __syncthreads();
  }
  const float inv = 1.f / fmaxf(l_run, 1e-6f);
#pragma unroll
  for (int i = 0; i < GEN_MAXD / GEN_T; ++i) {
    const int d = tid + i * GEN_T;
    if (d >= p.D) break;
    store_out(p, ((int64_t)b * p.Hq + hq) * p.D + d, o[i] * inv);
  }
}

__global__ void __launch_bounds__(128) paged_kv_append_kernel(
    const uint16_t* __restrict__ kn, const uint16_t* __restrict__ vn, int64_t ksb, int64_t ksh,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t num_blocks,
    const int32_t* __restrict__ bt, int64_t bts, const int32_t* __restrict__ cl, int Hkv, int D,
    int BS, int max_blocks) {
  const int b = blockIdx.x;
  const int pos = cl[b];
  if (pos < 0 || pos >= max_blocks * BS) return;
  const int phys = bt[(int64_t)b * bts + pos / BS];
  if (phys < 0 || phys >= num_blocks) return;
  const int off = pos % BS;
  for (int i = threadIdx.x; i < Hkv * D; i += blockDim.x) {
    const int h = i / D, d = i - h * D;
    const int64_t dst = (((int64_t)phys * Hkv + h) * BS + off) * D + d;
    const int64_t src = (int64_t)b * ksb + (int64_t)h * ksh + d;
    kc[dst] = kn[src];
    vc[dst] = vn[src];
  }
}

template <int GQ>
int launch_fast_attn(const AttnArgs& a, hipStream_t st) {
  dim3 grid(a.S, a.Hkv, a.B);
  paged_attn_mfma<GQ><<<grid, 256, 0, st>>>(a);
  return launch_check("paged_attn_mfma");
}

}  // namespace

extern "C" int grpo_paged_kv_append(const void* k_new, const void* v_new, int64_t kn_stride_b,
                                    int64_t kn_stride_h, void* k_cache, void* v_cache,
                                    int64_t num_blocks, const int32_t* block_tables,
                                    int64_t bt_stride, const int32_t* context_lens, int B, int Hkv,
                                    int D, int block_size, int max_blocks, grpo_stream_t stream) {
  if (B < 0 || Hkv <= 0 || D <= 0 || block_size <= 0 || max_blocks < 0 || num_blocks < 0)
    return einval("bad append dimensions");
  if (B == 0 || max_blocks == 0) return GRPO_OK;
  if (!k_new || !v_new || !k_cache || !v_cache || !block_tables || !context_lens)
    return einval("null pointer");
  paged_kv_append_kernel<<<dim3(B), 128, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(k_new), static_cast<const uint16_t*>(v_new), kn_stride_b,
      kn_stride_h, static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), num_blocks,
      block_tables, bt_stride, context_lens, Hkv, D, block_size, max_blocks);
  return launch_check("paged_kv_append");
}

extern "C" size_t grpo_paged_attn_workspace_bytes(int B, int Hq, int Hkv, int D, int block_size,
                                                  int max_blocks) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || block_size <= 0 || max_blocks <= 0) return 0;
  return plan_attn(B, Hq, Hkv, D, block_size, max_blocks).bytes;
}

extern "C" int grpo_paged_attn_decode(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                      const void* k_cache, const void* v_cache, int64_t num_blocks,
                                      const int32_t* block_tables, int64_t bt_stride,
                                      const int32_t* context_lens, void* out, int out_bf16, int B,
                                      int Hq, int Hkv, int D, int block_size, int max_blocks,
                                      float scale, void* workspace, size_t workspace_bytes,
                                      grpo_stream_t stream) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || block_size <= 0 || max_blocks < 0 ||
      num_blocks < 0)
    return einval("bad attention dimensions");
  if (Hq % Hkv != 0) return einval("Hq must be a multiple of Hkv");
  if (D > GEN_MAXD) return einval("head_dim > 512 is not supported");
  if (B == 0) return GRPO_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out)
    return einval("null pointer");
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qsb = q_stride_b;
  a.qsh = q_stride_h;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.num_blocks = num_blocks;
  a.bt = block_tables;
  a.bts = bt_stride;
  a.cl = context_lens;
  a.out = out;
  a.out_bf16 = out_bf16;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.D = D;
  a.BS = block_size;
  a.max_blocks = max_blocks;
  a.scale = scale;
  hipStream_t st = as_stream(stream);
  const AttnPlan plan = plan_attn(B, Hq, Hkv, D, block_size, max_blocks);
  const bool aligned = (reinterpret_cast<uintptr_t>(q) & 15u) == 0 && q_stride_b % 8 == 0 &&
                       q_stride_h % 8 == 0 && (reinterpret_cast<uintptr_t>(k_cache) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(v_cache) & 15u) == 0;
  if (plan.fast && aligned && max_blocks > 0) {
    a.bps = plan.bps;
    a.S = plan.S;
    if (plan.S > 1) {
      if (!workspace || workspace_bytes < plan.bytes) {
        set_error("invalid argument: workspace of %zu bytes needed, %zu given", plan.bytes,
                  workspace_bytes);
        return GRPO_EWORKSPACE;
      }
      a.ws_o = static_cast<float*>(workspace);
      a.ws_ml = a.ws_o + (size_t)B * Hq * plan.S * D;
    }
    int rc = GRPO_OK;
    switch (Hq / Hkv) {
      case 1: rc = launch_fast_attn<1>(a, st); break;
      case 2: rc = launch_fast_attn<2>(a, st); break;
      case 3: rc = launch_fast_attn<3>(a, st); break;
      case 4: rc = launch_fast_attn<4>(a, st); break;
      case 5: rc = launch_fast_attn<5>(a, st); break;
      case 6: rc = launch_fast_attn<6>(a, st); break;
      case 7: rc = launch_fast_attn<7>(a, st); break;
      default: rc = launch_fast_attn<8>(a, st); break;
    }
    if (rc != GRPO_OK || plan.S <= 1) return rc;
    paged_attn_merge<<<dim3(Hq, B), 128, 0, st>>>(a);
    return launch_check("paged_attn_merge");
  }
  a.bps = max_blocks > 0 ? max_blocks : 1;
  a.S = 1;
  paged_attn_generic<<<dim3(Hq, B), GEN_T, 0, st>>>(a);
  return launch_check("paged_attn_generic");
}
