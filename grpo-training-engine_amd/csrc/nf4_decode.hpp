// NF4 nibble decode shared by the NF4 kernels (gfx950).
//
// Weight format (bitsandbytes Params4bit, read by the reference in
// src/triton_kernels/lora_forward.py:171-206): W[N,K] flattened row-major,
// element e = n*K + k, byte e/2, even e = high nibble; one float32 absmax per
// `blocksize` flat elements; value = bf16_rne(code[q] * absmax) (float16_rne
// for float16 adapters).
#pragma once

#include "common.hpp"

namespace grpo {

constexpr int KSTEP = 256;  // k elements per step of an MFMA tile: 4 lane groups x 64

// NF4 weight bytes are read once per step.  Decode batches (M <= 16) load
// them with the non-temporal hint: with the weight, K/V and lm_head streams
// all marked so, a config-3 decode step keeps its small per-step data (split-K
// partials, activations, norms, LoRA, absmax) in L2 across kernels and runs in
// 1291 us against 1342 (each hint alone changes nothing).  Wide batches load
// them plainly (the hint cost 3 % at config 5).
template <bool NT>
__device__ __forceinline__ uint4 load_w(const uint4* p) {
  return NT ? load_stream(p) : *p;
}


__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) {
  return (m & a) | (~m & b);
}

// 16-entry bf16 codebook of one absmax block, split into high bytes (hb) and
// low bytes (lb): hb[i] byte j = high byte of bf16(code[4i+j] * a).
struct Lut {
  uint32_t hb[4], lb[4];
};

// F16: the table holds float16(code[j] * a) instead (the reference's cast to a
// float16 LoRA dtype, lora_forward.py:206); decode8 moves bytes only.
template <bool F16 = false>
__device__ __forceinline__ Lut make_lut(const float (&code)[16], float a) {
  Lut t;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t p01 = pack_e2<F16>(code[4 * i] * a, code[4 * i + 1] * a);
    const uint32_t p23 = pack_e2<F16>(code[4 * i + 2] * a, code[4 * i + 3] * a);
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

}  // namespace grpo
