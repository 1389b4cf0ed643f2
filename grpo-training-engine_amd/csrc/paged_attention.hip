// Paged KV append and single-query (decode) paged attention with GQA, gfx950.
//
// Cache: bf16 [num_blocks, Hkv, block_size, D]; block_tables int32 [B, max_blocks];
// context_lens int32 [B] (device-resident, read-only here).
//
// Fast decode path (D == 128, block_size == 16, Hq/Hkv <= 8): grid
// (context split, KV head, sequence) with at most 8 splits; 8 waves per
// workgroup, each wave walking every 8th 16-token block of its split (the next
// block's K/V loads are issued before the current block is processed).  Per
// block the 4 KB K tile is read with 16-byte loads straight into the A operand
// of v_mfma_f32_16x16x32_bf16 (rows = tokens) against the B operand Q^T of all
// query heads of the GQA group (columns = heads), giving S^T[token][head] in 4
// MFMAs.  The online softmax runs in the exp2 domain; P goes through a
// per-wave LDS slot; P.V runs on bf16 MFMA with P split into two bf16 terms
// (v_mfma_f32_16x16x16_bf16: O^T tiles of 16 head-dimension rows x 16 heads),
// every V element loaded once and applied to all heads of the group, each lane
// ending with distinct outputs (no cross-lane sums).  The 8 waves
// merge through LDS and every split writes (max, sum, unnormalised O): the
// standalone entry point merges them in a second kernel, the decode step merges
// them while the o_proj kernel stages its input (linear_parts.hpp, nf4_linear.hip).
// K and V of a KV head are read once per step, not once per query head.
//
// The decode step's variant also finishes the q|k|v projection from its split-K
// partial sums, applies RoPE to q and k, and appends the new token's K/V to the
// cache (the split holding the slot does it before it reads the cache), so
// neither q nor the RoPE + append needs a launch of its own.
#include <math.h>

#include <mutex>

#include "linear_parts.hpp"

using namespace grpo;

namespace {

constexpr int FD = 128;        // fast-path head dim
constexpr int FBS = 16;        // fast-path block size
constexpr int AW = 8;          // waves per workgroup
constexpr int AT = 64 * AW;    // threads per workgroup
constexpr int MAX_SPLITS = ATTN_MAX_SPLITS;  // context splits per (sequence, KV head)
constexpr float LOG2E = 1.4426950408889634f;
constexpr int ATTN_DEVICE_CUS = 256;  // MI355X
// One merge counter per 128-byte line (a line is touched only by the splits
// of one pair, which run on one XCD).
constexpr int MERGE_CNT_STRIDE = 32;
constexpr int NUM_XCD = 8;
// K/V blocks: read once per launch, loaded with the non-temporal hint (see
// load_w in nf4_linear.hip).
__device__ __forceinline__ uint4 load_kv16(const uint16_t* p) { return load_stream(p); }

struct AttnArgs {
  const uint16_t* q;
  int64_t qsb, qsh;
  uint16_t* kc;
  uint16_t* vc;
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
  float* ws_ml;  // [B][Hq][S][2]: max (log2 domain), sum
  // fused q|k|v finish + RoPE + append (decode step)
  LinParts qkv;
  const uint16_t* cos_t;
  const uint16_t* sin_t;
  int max_pos;
  const int32_t* append_pos;
  // one split per (sequence, KV head): the split writes the normalised bf16
  // output [B][Hq][D] here instead of partials (null otherwise)
  uint16_t* direct_out;
  // In-kernel merge (decode step, null otherwise): the split of each
  // (sequence, KV head) that arrives last merges the pair's splits into the
  // bf16 output mout [B][Hq * D]; counters [B * Hkv * MERGE_CNT_STRIDE]
  // (zero, left zero), xcd_err set when a pair's splits did not share an XCD.
  int* mcnt;
  int* xcd_err;
  uint16_t* mout;
  float* mout_f32;  // float32 merge output [B][Hq * D] instead of mout (plain attention)
  // ... and, with lora_r > 0, the pair's share of the next linear's LoRA-A
  // product: lora_t[b][kvh][r] = sum over the pair's Hq / Hkv heads of
  // mout[b, k] * lora_a[r][k] (float32; the consumer sums the Hkv shares)
  const uint16_t* lora_a;  // [lora_r][Hq * D] bf16
  int lora_r;
  float* lora_t;           // [B][Hkv][16]
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
  const int mb = max_blocks > 0 ? max_blocks : 1;
  // Context splits per (sequence, KV head): up to MAX_SPLITS while the
  // (sequence, KV head) pairs alone leave CUs idle; one split once they fill
  // the device.  The workgroup needs ~150 VGPRs per lane, so one workgroup of
  // 8 waves runs per CU: every extra round of workgroups repeats the
  // prologue and the wave merge, and at B * Hkv >= 256 (config 5: 64 rows x 4
  // KV heads) a single split per pair measured fastest (73 us against 77 at 2
  // splits and 82 at 8, 4096-token contexts).
  const int target = (int64_t)B * Hkv >= ATTN_DEVICE_CUS ? 1 : MAX_SPLITS;
  const int bpw = (int)cdiv(mb, (int64_t)AW * target);
  // one thread per block-table entry of a split: bps <= AT (contexts <= 64K)
  if (AW * bpw > AT) {
    p.fast = false;
    p.bps = mb;
    p.S = 1;
    return p;
  }
  p.bps = AW * bpw;
  p.S = (int)cdiv(mb, p.bps);
  p.bytes = (size_t)B * Hq * p.S * (D + 2) * 4;
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

// Orders a wave's LDS writes before its lanes read each other's values: wait
// for the wave's outstanding LDS operations only (lgkmcnt), with a compiler
// memory barrier.  A memory-model fence would also wait for the wave's
// outstanding global loads, i.e. for the next block's prefetch.
__device__ __forceinline__ void wave_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s16x4_t as_s16x4(uint2 v) { return __builtin_bit_cast(s16x4_t, v); }
__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// K slices of the q|k|v projection the fused prologue reads: MS = 8 covers
// the decode shapes (M = 64 at hidden 3584 plans 7 slices); up to 16 slices
// take the MS = 16 instantiation.
constexpr int QKV_SLICES_SMALL = 8;
constexpr int QKV_SLICES_LARGE = 16;

template <int GQ, bool FUSED, int MS = QKV_SLICES_SMALL>
__global__ void __launch_bounds__(AT) paged_attn_split(AttnArgs p) {
  touch_kernargs<sizeof(AttnArgs)>();
  // grid (pairs padded to a multiple of 8, splits): the splits of a (sequence,
  // KV head) pair have linear ids equal modulo 8, so they run on one XCD
  const int pair = blockIdx.x;
  if (pair >= p.B * p.Hkv) return;
  const int s = blockIdx.y, b = pair / p.Hkv, kvh = pair - b * p.Hkv;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lg = lane >> 4;
  const int blk0 = s * p.bps;  // < max_blocks for every launched split

  extern __shared__ __align__(16) float sO[];  // [AW][GQ][FD]
  __shared__ __align__(16) uint16_t sQ[GQ][FD];
  __shared__ __align__(16) uint16_t sNew[2][FD];  // appended token: rotated K, V
  __shared__ float sTs[MAXSEG * 16];
  // P of the wave's block, [head][token]; rows padded to 20 floats so the
  // P.V operand reads (token 4s + lane group) spread over the banks
  __shared__ __align__(16) float sP[AW][16][20];
  __shared__ float sM[AW][16];
  __shared__ float sL[AW][16];
  int* sBT = reinterpret_cast<int*>(sO + (size_t)AW * GQ * FD);  // the split's table slice

  const int64_t head_stride = (int64_t)FBS * FD;
  // K/V fragments of physical block phys; an invalid id reads block 0 and the
  // block is then skipped.  The loads are unconditional (see below).
  auto load_kv = [&](int phys, uint4 (&kf)[4], uint4 (&vf)[4])
                     __attribute__((always_inline)) -> bool {
    const bool ok = phys >= 0 && phys < p.num_blocks;
    const int64_t ph = ok ? phys : 0;
    const uint16_t* kb = p.kc + (ph * p.Hkv + kvh) * head_stride;
    const uint16_t* vb = p.vc + (ph * p.Hkv + kvh) * head_stride;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kf[i] = load_kv16(kb + ln * FD + 8 * lg + 32 * i);
      vf[i] = load_kv16(vb + (4 * i + lg) * FD + 8 * ln);
    }
    return ok;
  };

  // Load schedule.  Vector loads retire in issue order and the compiler waits
  // for one with s_waitcnt vmcnt(N), N = loads issued after it; after a
  // conditional load it can only assume the fewest loads, so a conditional
  // load makes the waits of the loads issued BEFORE it conservative, never of
  // those after it.  Hence: first the loads only some threads need, each
  // predicated (LoRA t: 12 threads; the q|k|v partial sums of the GQ + 2 rows,
  // or q; the block-table slice), none depending on a loaded value; then one
  // batch of scalar loads brings the context length, the append position and
  // this wave's first block id; then the loads every thread needs,
  // unconditional: the RoPE tables and the first block's K/V (HBM).  Each
  // phase then waits only for its own loads.  The wave whose first block
  // receives the new token loads it before the append and patches the
  // token's row from LDS afterwards.
  const int first = blk0 + wave;
  // Vector loads (VGPR results): kept in VGPRs until the barrier below, so the
  // wait for them and their move to scalar registers come after every load of
  // the prologue has been issued.
  int ctx_v = p.cl[b];
  int pos_v = FUSED ? p.append_pos[b] : -1;
  int phys_v = p.bt[(int64_t)b * p.bts + min(first, p.max_blocks - 1)];
  constexpr int NROW = GQ + 2;  // fused rows: GQ q heads, then k, then v
  static_assert(NROW * (FD / 4) <= AT - 64, "the last wave fetches no q|k|v row");
  const int row = tid / (FD / 4), d4 = 4 * (tid % (FD / 4));
  const int t_item = tid - (AT - 64);  // LoRA t item of a last-wave lane
  Fetch4<MS> f;
  float4 tv[MS];
  uint4 qv = make_uint4(0, 0, 0, 0);
  if constexpr (FUSED) {
    // LoRA t by the last wave (no q|k|v rows; its first K/V is needed only
    // after the prologue): the compiler starts the sum right after these loads,
    // which stalls the fetching wave for one round trip.
    if (t_item >= 0 && t_item < p.qkv.nseg * 4 && p.qkv.r > 0) lin_fetch_t(p.qkv, b, t_item, tv);
    if (row < NROW) {
      const int n0 = row < GQ ? (kvh * GQ + row) * FD
                              : (row == GQ ? (p.Hq + kvh) * FD : (p.Hq + p.Hkv + kvh) * FD);
      lin_fetch4(p.qkv, b, n0 + d4, f);
    }
  } else {
    if (tid < GQ * (FD / 8)) {
      const int h = tid / (FD / 8), c = tid - h * (FD / 8);
      qv = *reinterpret_cast<const uint4*>(p.q + (int64_t)b * p.qsb +
                                           (int64_t)(kvh * GQ + h) * p.qsh + 8 * c);
    }
  }
  int bt_v = 0;
  if (tid < p.bps) bt_v = p.bt[(int64_t)b * p.bts + min(blk0 + tid, p.max_blocks - 1)];
  // The context length, append position and first block id are consumed
  // here, after every prologue load has been issued (without the barrier the
  // compiler moves them to scalar registers right after their loads, which
  // stalls the wave for a round trip before it issues anything else).
  asm volatile("" : "+v"(ctx_v), "+v"(pos_v), "+v"(phys_v));
  const int ctx_raw = __builtin_amdgcn_readfirstlane(ctx_v);
  const int pos = __builtin_amdgcn_readfirstlane(pos_v);
  const int phys0 = __builtin_amdgcn_readfirstlane(phys_v);
  const int ctx = max(0, min(ctx_raw, p.max_blocks * FBS));
  const int nblk = (ctx + FBS - 1) / FBS;
  const int nsplit = nblk > 0 ? (nblk + p.bps - 1) / p.bps : 1;
  if (s >= nsplit) return;
  const int blk1 = min(blk0 + p.bps, nblk);
  const int nb = blk1 - blk0;  // 0 only for an empty context
  const int pblk = pos >= 0 ? pos / FBS : -1;
  const bool app = FUSED && pos >= 0 && pos < p.max_blocks * FBS && pblk >= blk0 && pblk < blk1;
  uint16_t rc0 = 0, rc1 = 0, rs0 = 0, rs1 = 0;  // cos/sin of RoPE pair dimension tid % 64
  if constexpr (FUSED) {
    const int cpos = pos < 0 ? 0 : (pos >= p.max_pos ? p.max_pos - 1 : pos);
    const int d = tid % (FD / 2);
    rc0 = p.cos_t[(int64_t)cpos * FD + d];
    rc1 = p.cos_t[(int64_t)cpos * FD + d + FD / 2];
    rs0 = p.sin_t[(int64_t)cpos * FD + d];
    rs1 = p.sin_t[(int64_t)cpos * FD + d + FD / 2];
  }
  uint4 kn[4], vn[4];
  bool ok_next = load_kv(first < blk1 ? phys0 : -1, kn, vn);

  if constexpr (FUSED) {
    // Phase A: LoRA t and the q|k|v finish (bias, LoRA, bf16) into LDS.
    float* sRaw = sO;  // [GQ + 2][FD], reused by the wave merge later
    if (t_item >= 0) lin_store_t(p.qkv, tv, t_item, sTs);
    if (tid < nb) sBT[tid] = bt_v;
    __syncthreads();
    if (row < NROW) {
      float v[4];
      lin_finish4(p.qkv, sTs, f, v);
      *reinterpret_cast<float4*>(sRaw + row * FD + d4) = make_float4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
    // The new token's cache row: its block id comes from the split's table
    // slice (in LDS since the first barrier).
    const int physA = app ? sBT[pblk - blk0] : -1;
    const int64_t slot = app && physA >= 0 && physA < p.num_blocks
                             ? (((int64_t)physA * p.Hkv + kvh) * FBS + pos % FBS) * FD
                             : -1;
    // Phase B: RoPE pairs (d, d + D/2) of the GQ q rows (+ the k row when
    // appending); the pair index advances by AT, a multiple of D/2, so every
    // pair of a thread uses dimension tid % 64.
    const int npair = (GQ + (app ? 1 : 0)) * (FD / 2);
    const float c0 = bf2f(rc0), c1 = bf2f(rc1), s0 = bf2f(rs0), s1 = bf2f(rs1);
    for (int i = tid; i < npair; i += AT) {
      const int r = i / (FD / 2), d = i % (FD / 2);
      const float x1 = sRaw[r * FD + d], x2 = sRaw[r * FD + d + FD / 2];
      const uint16_t lo = f2bf(round_bf(round_bf(x1 * c0) + round_bf(-x2 * s0)));
      const uint16_t hi = f2bf(round_bf(round_bf(x2 * c1) + round_bf(x1 * s1)));
      if (r < GQ) {
        sQ[r][d] = lo;
        sQ[r][d + FD / 2] = hi;
      } else {
        sNew[0][d] = lo;
        sNew[0][d + FD / 2] = hi;
        if (slot >= 0) {
          p.kc[slot + d] = lo;
          p.kc[slot + d + FD / 2] = hi;
        }
      }
    }
    if (app)
      for (int d = tid; d < FD; d += AT) {
        const uint16_t v = f2bf(sRaw[(GQ + 1) * FD + d]);
        sNew[1][d] = v;
        if (slot >= 0) p.vc[slot + d] = v;
      }
  } else {
    if (tid < GQ * (FD / 8)) {
      const int h = tid / (FD / 8), c = tid - h * (FD / 8);
      *reinterpret_cast<uint4*>(&sQ[h][8 * c]) = qv;
    }
    if (tid < nb) sBT[tid] = bt_v;
  }
  // Orders sQ, sNew, sBT and the reuse of sO before any wave reads them.  (The
  // cache rows written above are read by no wave of this launch: the block
  // holding them is this split's, and its wave patches the row from sNew.)
  __syncthreads();

  if (FUSED && app && first == pblk) {
    // The first block of this wave received the new token at row t.
    const int t = pos % FBS;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (ln == t) kn[i] = *reinterpret_cast<const uint4*>(&sNew[0][8 * lg + 32 * i]);
      if (4 * i + lg == t) vn[i] = *reinterpret_cast<const uint4*>(&sNew[1][8 * ln]);
    }
  }

  // Q^T as the MFMA B operand: lane (head ln, group lg) holds
  // Q[head][8*lg + 32*i + 0..7] for MFMA i.
  uint4 qf[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    qf[i] = ln < GQ ? *reinterpret_cast<const uint4*>(&sQ[ln][8 * lg + 32 * i])
                    : make_uint4(0, 0, 0, 0);
  const float sl2 = p.scale * LOG2E;
  float m_run = -INFINITY, l_run = 0.f;  // softmax state of head ln
  // O^T in eight 16x16 tiles: tile i holds rows d = 8*r + i (r = 0..15) and
  // columns = heads; lane (head ln, group lg) holds O[ln][8*(4*lg + q) + i]
  // in oacc[i][q].
  f32x4_t oacc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // One 16-token block: S^T on MFMA, online softmax, P.V on float32 MFMA.  (Inlined
  // at both call sites: a call would pass every captured variable, the kernel
  // arguments included, through scratch memory.)
  auto block = [&](int blk, const uint4 (&kf)[4], const uint4 (&vf)[4])
                   __attribute__((always_inline)) {
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
    bmax = pair32_max(pair16_max(bmax));
    const float m_new = fmaxf(m_run, bmax);  // finite: token blk*16 < ctx
    const float corr = exp2f(m_run - m_new);
    float pv[4];
    float ps = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pv[r] = exp2f(sv[r] - m_new);
      ps += pv[r];
    }
    ps = pair32_sum(pair16_sum(ps));
    l_run = l_run * corr + ps;
    m_run = m_new;
    *reinterpret_cast<float4*>(&sP[wave][ln][4 * lg]) = make_float4(pv[0], pv[1], pv[2], pv[3]);
    wave_sync();
    // P.V on bf16 MFMA with P split in two bf16 terms, P = P_hi + P_lo + e,
    // |e| <= 2^-17 |P|: V is bf16, so V.P_hi and V.P_lo are exact float32
    // products summed in float32 (the reference's float32 p * v up to e), at
    // 16 v_mfma_f32_16x16x16_bf16 per block instead of 32 float32 16x16x4
    // (an eighth of the matrix-core cycles).  O^T tile i += V^T (16 d x 16
    // tokens) . P (16 tokens x 16 heads); MFMA k = 4*lg + s is token 4s + lg:
    // lane (ln, lg) gives A = V[4s + lg][8*ln + i] (element i of vf[s]) and
    // B = P[4s + lg][head ln], s = 0..3.  The rescale by this lane's head's
    // corr comes first.
    float pb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) pb[q] = sP[wave][ln][4 * q + lg];
    uint2 bh, bl;
    {
      const uint32_t h01 = pack_bf2(pb[0], pb[1]), h23 = pack_bf2(pb[2], pb[3]);
      bh = make_uint2(h01, h23);
      bl = make_uint2(pack_bf2(pb[0] - bf_lo(h01), pb[1] - bf_hi(h01)),
                      pack_bf2(pb[2] - bf_lo(h23), pb[3] - bf_hi(h23)));
    }
    // Rescale only when some head's running max moved in this block (corr is
    // exactly 1 otherwise, so skipping the 32 multiplies changes no bit): a
    // wave-uniform test, true on the first blocks and rarely after.
    if (__builtin_amdgcn_ballot_w64(corr != 1.f)) {
#pragma unroll
      for (int i = 0; i < 8; ++i) oacc[i] *= corr;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t w0 = word(vf[0], i >> 1), w1 = word(vf[1], i >> 1);
      const uint32_t w2 = word(vf[2], i >> 1), w3 = word(vf[3], i >> 1);
      const uint2 a = make_uint2(perm(w1, w0, sel), perm(w3, w2, sel));
      oacc[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(as_s16x4(a), as_s16x4(bh), oacc[i], 0,
                                                          0, 0);
      oacc[i] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(as_s16x4(a), as_s16x4(bl), oacc[i], 0,
                                                          0, 0);
    }
    wave_sync();
  };

  // The wave's blocks first, first + AW, ...: the next block's loads are issued
  // before the current one is processed.  The two branches keep the load count
  // exact (a prefetch issued or not), so the current block waits only for its
  // own loads.
  for (int blk = first; blk < blk1; blk += AW) {
    uint4 kf[4], vf[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kf[i] = kn[i];
      vf[i] = vn[i];
    }
    const bool ok = ok_next;
    const int nxt = blk + AW;
    if (nxt < blk1) {
      ok_next = load_kv(sBT[nxt - blk0], kn, vn);
      if (ok) block(blk, kf, vf);
    } else {
      if (ok) block(blk, kf, vf);
    }
  }

  // Merge the AW waves: each lane of a head column writes its 32 elements of
  // O[head][:] (rows 8*(4*lg + q) + i of the tiles) to the wave's slot.
  if (lg == 0) {
    sM[wave][ln] = m_run;
    sL[wave][ln] = l_run;
  }
  if (ln < GQ) {
    float* dst = sO + ((size_t)wave * GQ + ln) * FD;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int d0 = 8 * (4 * lg + q);
      *reinterpret_cast<float4*>(dst + d0) =
          make_float4(oacc[0][q], oacc[1][q], oacc[2][q], oacc[3][q]);
      *reinterpret_cast<float4*>(dst + d0 + 4) =
          make_float4(oacc[4][q], oacc[5][q], oacc[6][q], oacc[7][q]);
    }
  }
  __syncthreads();
  // In-kernel merge (decode step): a pair whose whole context is this split
  // writes its output directly; otherwise the split arriving last merges.
  const bool merge = p.mcnt != nullptr;
  const bool single = merge && nsplit == 1;
  // LoRA-A rows of this thread's four columns k (the output's columns of
  // head kvh * GQ + h, d4 .. d4 + 3), for the next linear's t: issued before
  // they are needed (ranks past lora_r read rank 0, dropped in the sum)
  const int mh = tid / (FD / 4), md4 = 4 * (tid - mh * (FD / 4));
  const int64_t kcol = (int64_t)(kvh * GQ + mh) * FD + md4;
  const bool lora = merge && p.lora_r > 0 && tid < GQ * (FD / 4);
  uint2 arow[16];
  auto load_lora_a = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      arow[r] = *reinterpret_cast<const uint2*>(p.lora_a + (int64_t)(r < p.lora_r ? r : 0) *
                                                               p.Hq * FD + kcol);
  };
  if (single && lora) load_lora_a();
  float xr[4] = {0.f, 0.f, 0.f, 0.f};  // this thread's bf16 output values (merge)
  // Four columns of one head per thread: the split's max M and the waves'
  // weights 2^(m_w - M) computed by every thread of the head (no second
  // barrier behind a per-head pass), O summed in wave order; the head's first
  // thread writes (M, L).
  for (int i = tid; i < GQ * FD / 4; i += AT) {
    const int h = i / (FD / 4), d4 = 4 * (i - h * (FD / 4));
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < AW; ++w) M = fmaxf(M, sM[w][h]);
    float f[AW];
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < AW; ++w) {
      f[w] = M == -INFINITY ? 0.f : exp2f(sM[w][h] - M);
      L += f[w] * sL[w][h];
    }
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < AW; ++w) {
      const float4 v = *reinterpret_cast<const float4*>(sO + ((size_t)w * GQ + h) * FD + d4);
      O.x += f[w] * v.x;
      O.y += f[w] * v.y;
      O.z += f[w] * v.z;
      O.w += f[w] * v.w;
    }
    if (single && p.mout_f32) {
      // the whole context in this split, float32 output: out = O / max(L, 1e-6)
      const float den = fmaxf(L, 1e-6f);
      *reinterpret_cast<float4*>(p.mout_f32 + ((int64_t)b * p.Hq + kvh * GQ + h) * FD + d4) =
          make_float4(O.x / den, O.y / den, O.z / den, O.w / den);
    } else if (p.direct_out || single) {
      // the whole context in this split: out = O / max(L, 1e-6), bf16
      const float den = fmaxf(L, 1e-6f);
      const uint2 ov = make_uint2(pack_bf2(O.x / den, O.y / den), pack_bf2(O.z / den, O.w / den));
      uint16_t* dst = single ? p.mout : p.direct_out;
      *reinterpret_cast<uint2*>(dst + ((int64_t)b * p.Hq + kvh * GQ + h) * FD + d4) = ov;
      xr[0] = bf_lo(ov.x);
      xr[1] = bf_hi(ov.x);
      xr[2] = bf_lo(ov.y);
      xr[3] = bf_hi(ov.y);
    } else {
      const int64_t slot = ((int64_t)b * p.Hq + kvh * GQ + h) * p.S + s;
      if (d4 == 0) {
        p.ws_ml[slot * 2] = M;
        p.ws_ml[slot * 2 + 1] = L;
      }
      *reinterpret_cast<float4*>(p.ws_o + slot * FD + d4) = O;
    }
  }
  if (!merge) return;
  if (!single) {
    // Arrival: this split's partials are in the XCD's L2 once its stores are
    // acknowledged (the vector L1 writes through); the pair's counter is an
    // L2 atomic (xcd_arrive: checks that the pair's splits share an XCD).
    // The last of the nsplit splits drops its L1 lines and merges:
    // out = sum_s 2^(m_s - M) O_s / max(sum_s 2^(m_s - M) l_s, 1e-6).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ int s_last;
    if (tid == 0)
      s_last = xcd_arrive(p.mcnt + (int64_t)(b * p.Hkv + kvh) * MERGE_CNT_STRIDE, nsplit,
                          p.xcd_err);
    __syncthreads();
    if (!s_last) return;
    asm volatile("buffer_inv sc0" ::: "memory");
    if (tid < GQ * (FD / 4)) {
      const int64_t base = ((int64_t)b * p.Hq + kvh * GQ + mh) * p.S;
      float2 ml[MAX_SPLITS];
      float4 ov[MAX_SPLITS];
#pragma unroll
      for (int q = 0; q < MAX_SPLITS; ++q)
        if (q < nsplit) {
          ml[q] = *reinterpret_cast<const float2*>(p.ws_ml + (base + q) * 2);
          ov[q] = *reinterpret_cast<const float4*>(p.ws_o + (base + q) * FD + md4);
        }
      if (lora) load_lora_a();
      float M = -INFINITY;
#pragma unroll
      for (int q = 0; q < MAX_SPLITS; ++q)
        if (q < nsplit) M = fmaxf(M, ml[q].x);
      float L = 0.f;
      float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
      if (M != -INFINITY) {
#pragma unroll
        for (int q = 0; q < MAX_SPLITS; ++q)
          if (q < nsplit) {
            const float w = exp2f(ml[q].x - M);
            L += w * ml[q].y;
            O.x += w * ov[q].x;
            O.y += w * ov[q].y;
            O.z += w * ov[q].z;
            O.w += w * ov[q].w;
          }
      }
      const float den = fmaxf(L, 1e-6f);
      if (p.mout_f32) {
        *reinterpret_cast<float4*>(p.mout_f32 + ((int64_t)b * p.Hq + kvh * GQ + mh) * FD + md4) =
            make_float4(O.x / den, O.y / den, O.z / den, O.w / den);
      } else {
        const uint2 o2 =
            make_uint2(pack_bf2(O.x / den, O.y / den), pack_bf2(O.z / den, O.w / den));
        *reinterpret_cast<uint2*>(p.mout + ((int64_t)b * p.Hq + kvh * GQ + mh) * FD + md4) = o2;
        xr[0] = bf_lo(o2.x);
        xr[1] = bf_hi(o2.x);
        xr[2] = bf_lo(o2.y);
        xr[3] = bf_hi(o2.y);
      }
    }
  }
  if (p.lora_r <= 0) return;
  // The pair's share of t = out . A^T: per rank, the thread's four products,
  // summed over each wave (DPP) and then over the waves in order.
  __shared__ float sT[AW][16];
  float tp[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float v = 0.f;
    if (lora && r < p.lora_r) {
      v = xr[0] * bf_lo(arow[r].x) + xr[1] * bf_hi(arow[r].x) + xr[2] * bf_lo(arow[r].y) +
          xr[3] * bf_hi(arow[r].y);
    }
    tp[r] = wave_sum_dpp(v);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sT[wave][r] = tp[r];
  }
  __syncthreads();
  if (tid < 16) {
    constexpr int TW = (GQ * (FD / 4) + 63) / 64;  // waves holding columns
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < TW; ++w) t += sT[w][tid];
    p.lora_t[((int64_t)b * p.Hkv + kvh) * 16 + tid] = t;
  }
}

// Combine split partials: out = sum_s 2^(m_s - M) O_s / max(sum_s 2^(m_s - M) l_s, 1e-6).
// Every split's (max, sum) and O values of a thread are loaded before any is
// used (the fast path has at most MAX_SPLITS splits), so the merge is one
// memory round trip.
__global__ void __launch_bounds__(128) paged_attn_merge(AttnArgs p) {
  const int hq = blockIdx.x, b = blockIdx.y;
  const int ctx = seq_ctx(p, b);
  const int nblk = (ctx + p.BS - 1) / p.BS;
  const int nsplit = min(nblk > 0 ? (nblk + p.bps - 1) / p.bps : 1, MAX_SPLITS);
  const int64_t base = ((int64_t)b * p.Hq + hq) * p.S;
  float2 ml[MAX_SPLITS];
  float ov[MAX_SPLITS];
  const int d0 = threadIdx.x;
#pragma unroll
  for (int s = 0; s < MAX_SPLITS; ++s)
    if (s < nsplit) {
      ml[s] = *reinterpret_cast<const float2*>(p.ws_ml + (base + s) * 2);
      if (d0 < p.D) ov[s] = p.ws_o[(base + s) * p.D + d0];
    }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < MAX_SPLITS; ++s)
    if (s < nsplit) M = fmaxf(M, ml[s].x);
  const bool any = M != -INFINITY;  // false only if every block id was invalid
  float L = 0.f, w[MAX_SPLITS];
#pragma unroll
  for (int s = 0; s < MAX_SPLITS; ++s) {
    w[s] = any && s < nsplit ? exp2f(ml[s].x - M) : 0.f;
    if (s < nsplit) L += w[s] * ml[s].y;
  }
  const float den = fmaxf(L, 1e-6f);
  for (int d = d0; d < p.D; d += blockDim.x) {
    float O = 0.f;
#pragma unroll
    for (int s = 0; s < MAX_SPLITS; ++s)
      if (s < nsplit) O += w[s] * (d == d0 ? ov[s] : p.ws_o[(base + s) * p.D + d]);
    store_out(p, ((int64_t)b * p.Hq + hq) * p.D + d, O / den);
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

template <int GQ, bool FUSED>
int launch_split(const AttnArgs& a, hipStream_t st) {
  // wave merge [AW][GQ][FD] floats (the fused prologue reuses it as [GQ + 2][FD]),
  // then the split's block-table slice
  const size_t lds = (size_t)AW * GQ * FD * sizeof(float) + (size_t)a.bps * sizeof(int);
  if (lds > 65536) return einval("context too long for the split attention kernel");
  const dim3 grid((unsigned)(cdiv((int64_t)a.B * a.Hkv, NUM_XCD) * NUM_XCD), (unsigned)a.S);
  if constexpr (FUSED) {
    if (a.qkv.S > QKV_SLICES_SMALL) {
      paged_attn_split<GQ, FUSED, QKV_SLICES_LARGE><<<grid, AT, lds, st>>>(a);
      return launch_check("paged_attn_split");
    }
  }
  paged_attn_split<GQ, FUSED><<<grid, AT, lds, st>>>(a);
  return launch_check("paged_attn_split");
}

template <bool FUSED>
int launch_split_gq(const AttnArgs& a, hipStream_t st) {
  switch (a.Hq / a.Hkv) {
    case 1: return launch_split<1, FUSED>(a, st);
    case 2: return launch_split<2, FUSED>(a, st);
    case 3: return launch_split<3, FUSED>(a, st);
    case 4: return launch_split<4, FUSED>(a, st);
    case 5: return launch_split<5, FUSED>(a, st);
    case 6: return launch_split<6, FUSED>(a, st);
    case 7: return launch_split<7, FUSED>(a, st);
    default: return launch_split<8, FUSED>(a, st);
  }
}

int use_workspace(AttnArgs& a, const AttnPlan& plan, void* workspace, size_t workspace_bytes) {
  if (!workspace || workspace_bytes < plan.bytes) {
    set_error("invalid argument: workspace of %zu bytes needed, %zu given", plan.bytes,
              workspace_bytes);
    return GRPO_EWORKSPACE;
  }
  if ((reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
    return einval("attention workspace must be 16-byte aligned");
  a.bps = plan.bps;
  a.S = plan.S;
  a.ws_o = static_cast<float*>(workspace);
  a.ws_ml = a.ws_o + (size_t)a.B * a.Hq * plan.S * a.D;
  return GRPO_OK;
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
  a.kc = static_cast<uint16_t*>(const_cast<void*>(k_cache));
  a.vc = static_cast<uint16_t*>(const_cast<void*>(v_cache));
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
    if (int rc = use_workspace(a, plan, workspace, workspace_bytes)) return rc;
    if (int rc = launch_split_gq<false>(a, st)) return rc;
    paged_attn_merge<<<dim3(Hq, B), 128, 0, st>>>(a);
    return launch_check("paged_attn_merge");
  }
  a.bps = max_blocks > 0 ? max_blocks : 1;
  a.S = 1;
  paged_attn_generic<<<dim3(Hq, B), GEN_T, 0, st>>>(a);
  return launch_check("paged_attn_generic");
}

extern "C" int grpo_paged_attn_decode_merged(
    const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
    const void* v_cache, int64_t num_blocks, const int32_t* block_tables, int64_t bt_stride,
    const int32_t* context_lens, void* out, int out_bf16, int B, int Hq, int Hkv, int D,
    int block_size, int max_blocks, float scale, void* workspace, size_t workspace_bytes,
    int* counters, int* xcd_err, grpo_stream_t stream) {
  const AttnPlan plan = plan_attn(B > 0 ? B : 1, Hq > 0 ? Hq : 1, Hkv > 0 ? Hkv : 1,
                                  D > 0 ? D : 1, block_size > 0 ? block_size : 1, max_blocks);
  const bool aligned = (reinterpret_cast<uintptr_t>(q) & 15u) == 0 && q_stride_b % 8 == 0 &&
                       q_stride_h % 8 == 0 && (reinterpret_cast<uintptr_t>(k_cache) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(v_cache) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || !plan.fast || !aligned ||
      max_blocks <= 0 || !q || !k_cache || !v_cache || !block_tables || !context_lens || !out)
    // one launch already (the generic kernel), or an argument error it reports
    return grpo_paged_attn_decode(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                                  block_tables, bt_stride, context_lens, out, out_bf16, B, Hq,
                                  Hkv, D, block_size, max_blocks, scale, workspace,
                                  workspace_bytes, stream);
  if (num_blocks < 0) return einval("bad attention dimensions");
  if (!counters || !xcd_err) return einval("the in-kernel merge needs its counters and error word");
  if ((reinterpret_cast<uintptr_t>(counters) & 127u) != 0)
    return einval("merge counters must be 128-byte aligned");
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.qsb = q_stride_b;
  a.qsh = q_stride_h;
  a.kc = static_cast<uint16_t*>(const_cast<void*>(k_cache));
  a.vc = static_cast<uint16_t*>(const_cast<void*>(v_cache));
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
  if (int rc = use_workspace(a, plan, workspace, workspace_bytes)) return rc;
  a.mcnt = counters;
  a.xcd_err = xcd_err;
  if (out_bf16)
    a.mout = static_cast<uint16_t*>(out);
  else
    a.mout_f32 = static_cast<float*>(out);
  return launch_split_gq<false>(a, as_stream(stream));
}

namespace {

// In-kernel merge target of the decode-step attention (all-null: none).
struct MergeTarget {
  int* cnt = nullptr;
  int* err = nullptr;
  uint16_t* out = nullptr;
  const uint16_t* lora_a = nullptr;
  int lora_r = 0;
  float* lora_t = nullptr;
};

int run_attn_qkv(const grpo_linear_parts_t* qkv, int Hq, int Hkv, int D, const void* cos_table,
                 const void* sin_table, int max_pos, const int32_t* append_pos,
                 const int32_t* context_lens, void* k_cache, void* v_cache, int64_t num_blocks,
                 const int32_t* block_tables, int64_t bt_stride, int block_size, int max_blocks,
                 float scale, void* workspace, size_t workspace_bytes, void* out,
                 const MergeTarget& mg, grpo_stream_t stream) {
  AttnArgs a{};
  if (int rc = make_parts(qkv, &a.qkv)) return rc;
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || max_blocks <= 0 || num_blocks < 0 || max_pos <= 0)
    return einval("bad attention dimensions");
  const AttnPlan plan = plan_attn(a.qkv.M, Hq, Hkv, D, block_size, max_blocks);
  if (!plan.fast) {
    set_error("fused q|k|v attention needs head_dim 128, block size 16, Hq/Hkv <= 8");
    return GRPO_EUNSUPPORTED;
  }
  if (a.qkv.N != (Hq + 2 * Hkv) * D) return einval("qkv width must be (Hq + 2 Hkv) * D");
  if (a.qkv.S > QKV_SLICES_LARGE) {
    set_error("fused q|k|v attention reads at most %d K slices of the projection",
              QKV_SLICES_LARGE);
    return GRPO_EUNSUPPORTED;
  }
  if (!cos_table || !sin_table || !append_pos || !context_lens || !k_cache || !v_cache ||
      !block_tables)
    return einval("null pointer");
  if ((reinterpret_cast<uintptr_t>(k_cache) & 15u) || (reinterpret_cast<uintptr_t>(v_cache) & 15u))
    return einval("caches must be 16-byte aligned");
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.num_blocks = num_blocks;
  a.bt = block_tables;
  a.bts = bt_stride;
  a.cl = context_lens;
  a.B = a.qkv.M;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.D = D;
  a.BS = block_size;
  a.max_blocks = max_blocks;
  a.scale = scale;
  a.cos_t = static_cast<const uint16_t*>(cos_table);
  a.sin_t = static_cast<const uint16_t*>(sin_table);
  a.max_pos = max_pos;
  a.append_pos = append_pos;
  if (out) {
    if (plan.S != 1) return einval("direct output needs one context split (grpo_paged_attn_splits)");
    if ((reinterpret_cast<uintptr_t>(out) & 7u) != 0) return einval("out must be 8-byte aligned");
    a.direct_out = static_cast<uint16_t*>(out);
    a.bps = plan.bps;
    a.S = plan.S;
  } else if (int rc = use_workspace(a, plan, workspace, workspace_bytes)) {
    return rc;
  }
  if (mg.cnt) {
    if (!mg.out || !mg.err) return einval("null pointer");
    if ((reinterpret_cast<uintptr_t>(mg.out) & 7u) != 0) return einval("out must be 8-byte aligned");
    if (mg.lora_r < 0 || mg.lora_r > 16) return einval("LoRA rank must be in [0, 16]");
    if (mg.lora_r > 0 && (!mg.lora_a || !mg.lora_t || !aligned8(mg.lora_a)))
      return einval("LoRA rank > 0 needs lora_a (8-byte aligned) and lora_t");
    a.mcnt = mg.cnt;
    a.xcd_err = mg.err;
    a.mout = mg.out;
    a.lora_a = mg.lora_a;
    a.lora_r = mg.lora_r;
    a.lora_t = mg.lora_t;
  }
  return launch_split_gq<true>(a, as_stream(stream));
}

}  // namespace

extern "C" int grpo_paged_attn_decode_qkv(const grpo_linear_parts_t* qkv, int Hq, int Hkv, int D,
                                          const void* cos_table, const void* sin_table,
                                          int max_pos, const int32_t* append_pos,
                                          const int32_t* context_lens, void* k_cache,
                                          void* v_cache, int64_t num_blocks,
                                          const int32_t* block_tables, int64_t bt_stride,
                                          int block_size, int max_blocks, float scale,
                                          void* workspace, size_t workspace_bytes, void* out,
                                          grpo_stream_t stream) {
  return run_attn_qkv(qkv, Hq, Hkv, D, cos_table, sin_table, max_pos, append_pos, context_lens,
                      k_cache, v_cache, num_blocks, block_tables, bt_stride, block_size,
                      max_blocks, scale, workspace, workspace_bytes, out, MergeTarget{}, stream);
}

extern "C" size_t grpo_paged_attn_merge_counter_bytes(int B, int Hkv) {
  return B > 0 && Hkv > 0 ? (size_t)B * Hkv * MERGE_CNT_STRIDE * sizeof(int) : 0;
}

extern "C" int grpo_paged_attn_decode_qkv_merged(
    const grpo_linear_parts_t* qkv, int Hq, int Hkv, int D, const void* cos_table,
    const void* sin_table, int max_pos, const int32_t* append_pos, const int32_t* context_lens,
    void* k_cache, void* v_cache, int64_t num_blocks, const int32_t* block_tables,
    int64_t bt_stride, int block_size, int max_blocks, float scale, void* workspace,
    size_t workspace_bytes, int* counters, int* xcd_err, void* out, const void* o_lora_a,
    int o_lora_r, float* o_lora_t, grpo_stream_t stream) {
  if (!counters) return einval("null counters");
  MergeTarget mg;
  mg.cnt = counters;
  mg.err = xcd_err;
  mg.out = static_cast<uint16_t*>(out);
  mg.lora_a = static_cast<const uint16_t*>(o_lora_a);
  mg.lora_r = o_lora_r;
  mg.lora_t = o_lora_t;
  return run_attn_qkv(qkv, Hq, Hkv, D, cos_table, sin_table, max_pos, append_pos, context_lens,
                      k_cache, v_cache, num_blocks, block_tables, bt_stride, block_size,
                      max_blocks, scale, workspace, workspace_bytes, nullptr, mg, stream);
}

extern "C" int grpo_paged_attn_qkv_max_slices(void) { return QKV_SLICES_LARGE; }

extern "C" int grpo_paged_attn_splits(int B, int Hq, int Hkv, int D, int block_size,
                                      int max_blocks) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || max_blocks <= 0) return 0;
  const AttnPlan plan = plan_attn(B, Hq, Hkv, D, block_size, max_blocks);
  return plan.fast ? plan.S : 0;
}

// ------------------------------------------------- allocation-free entry --
//
// grpo_paged_attn_decode_noalloc runs grpo_paged_attn_decode with its split
// partials in `scratch`, a file-scope device array, instead of a caller
// workspace.  In host code `scratch` names a host-side stand-in, never the
// device copy: the device address comes from hipGetSymbolAddress, taken once per
// device (with that device current) on the entry's first call there and kept in
// g_scratch_dev[device].  Every call on one GPU shares that GPU's array.
namespace {

constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(8) << 20;
constexpr int NOALLOC_MAX_DEVICES = 64;
__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
void* g_scratch_dev[NOALLOC_MAX_DEVICES] = {};

int scratch_address(void** out) {
  int dev = 0;
  if (int rc = hip_check(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return einval("device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    if (int rc = hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress"))
      return rc;
    if (!p) return hip_check(hipErrorInvalidSymbol, "hipGetSymbolAddress");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return GRPO_OK;
}

}  // namespace

extern "C" size_t grpo_paged_attn_noalloc_max_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int grpo_paged_attn_decode_noalloc(const void* q, int64_t q_stride_b,
                                              int64_t q_stride_h, const void* k_cache,
                                              const void* v_cache, int64_t num_blocks,
                                              const int32_t* block_tables, int64_t bt_stride,
                                              const int32_t* context_lens, void* out,
                                              int out_bf16, int B, int Hq, int Hkv, int D,
                                              int block_size, int max_blocks, float scale,
                                              grpo_stream_t stream) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || D <= 0 || block_size <= 0 || max_blocks < 0)
    return einval("bad attention dimensions");
  const size_t need =
      B > 0 && max_blocks > 0 ? plan_attn(B, Hq, Hkv, D, block_size, max_blocks).bytes : 0;
  if (need > NOALLOC_SCRATCH_BYTES) {
    set_error("invalid argument: this shape needs %zu bytes of split partials; the "
              "allocation-free entry holds at most %zu (use grpo_paged_attn_decode with a "
              "workspace)",
              need, NOALLOC_SCRATCH_BYTES);
    return GRPO_EWORKSPACE;
  }
  void* ws = nullptr;
  if (need > 0)
    if (int rc = scratch_address(&ws)) return rc;
  return grpo_paged_attn_decode(q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks,
                                block_tables, bt_stride, context_lens, out, out_bf16, B, Hq, Hkv,
                                D, block_size, max_blocks, scale, ws,
                                need > 0 ? NOALLOC_SCRATCH_BYTES : 0, stream);
}

extern "C" int grpo_paged_attn_merge(const void* attn_workspace, const int32_t* context_lens,
                                     int B, int Hq, int Hkv, int D, int block_size,
                                     int max_blocks, void* out, int out_bf16,
                                     grpo_stream_t stream) {
  if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || max_blocks <= 0)
    return einval("bad attention dimensions");
  if (B == 0) return GRPO_OK;
  const AttnPlan plan = plan_attn(B, Hq, Hkv, D, block_size, max_blocks);
  if (!plan.fast) {
    set_error("the split partials exist only on the fast path (head_dim 128, block size 16, "
              "Hq/Hkv <= 8)");
    return GRPO_EUNSUPPORTED;
  }
  if (!attn_workspace || !context_lens || !out) return einval("null pointer");
  if ((reinterpret_cast<uintptr_t>(attn_workspace) & 15u) != 0)
    return einval("attention workspace must be 16-byte aligned");
  AttnArgs a{};
  a.cl = context_lens;
  a.out = out;
  a.out_bf16 = out_bf16;
  a.B = B;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.D = D;
  a.BS = block_size;
  a.max_blocks = max_blocks;
  a.bps = plan.bps;
  a.S = plan.S;
  a.ws_o = static_cast<float*>(const_cast<void*>(attn_workspace));
  a.ws_ml = a.ws_o + (size_t)B * Hq * plan.S * D;
  paged_attn_merge<<<dim3(Hq, B), 128, 0, as_stream(stream)>>>(a);
  return launch_check("paged_attn_merge");
}

namespace grpo {

int attn_plan_geometry(int B, int Hq, int Hkv, int D, int block_size, int max_blocks, int* bps,
                       int* splits) {
  const AttnPlan plan = plan_attn(B, Hq, Hkv, D, block_size, max_blocks);
  if (!plan.fast || max_blocks <= 0) return GRPO_EUNSUPPORTED;
  *bps = plan.bps;
  *splits = plan.S;
  return GRPO_OK;
}

}  // namespace grpo
