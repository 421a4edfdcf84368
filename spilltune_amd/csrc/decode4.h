// Register-table 4-bit decode shared by the fused GEMMs (q4gemm.hip) and the
// standalone dequant (dequant.hip).  Per (row, 128-group) a 16-entry table
// of bf16_rne(codebook[c] * scale) is built -- the exact product of
// codecs.py:168-170 -- and split into a low-byte and a high-byte plane, so
// v_perm_b32 looks four codes up at once; no LDS is involved.
#pragma once
#include "common.h"

namespace st {

// Per-(row, group) decode table: entry c = bf16_rne(codebook[c] * scale), the
// exact product the reference computes, split into a low-byte plane and a
// high-byte plane of 16 bytes each so v_perm_b32 can index it by code.
struct Tbl {
  uint32_t lo[4], hi[4];
};
__device__ __forceinline__ Tbl make_tbl(const Lut16& lut, float s) {
  uint32_t t[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) t[j] = st::pack_bf16x2(lut.v[2 * j] * s, lut.v[2 * j + 1] * s);
  Tbl T;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    T.lo[q] = __builtin_amdgcn_perm(t[2 * q + 1], t[2 * q], 0x06040200u);
    T.hi[q] = __builtin_amdgcn_perm(t[2 * q + 1], t[2 * q], 0x07050301u);
  }
  return T;
}
// byte i of the result = plane[code_i] for the four codes in the bytes of n
__device__ __forceinline__ uint32_t sel4(const uint32_t (&pl)[4], uint32_t n7, uint32_t hsel) {
  uint32_t a = __builtin_amdgcn_perm(pl[1], pl[0], n7);
  uint32_t b = __builtin_amdgcn_perm(pl[3], pl[2], n7);
  return __builtin_amdgcn_perm(b, a, hsel);
}
// 8 codes of one packed word -> 4 bf16x2 words in element order.  sh_e / sh_o
// = 0 / 4 when the low nibble of a byte holds the even element, 4 / 0 when
// the high nibble does.
__device__ __forceinline__ void deq8(uint32_t w, const Tbl& T, uint32_t sh_e, uint32_t sh_o,
                                     uint32_t (&o)[4]) {
  // ne = codes of elements 0,2,4,6; no = codes of elements 1,3,5,7
  const uint32_t ne = (w >> sh_e) & 0x0F0F0F0Fu;
  const uint32_t no = (w >> sh_o) & 0x0F0F0F0Fu;
  const uint32_t se = 0x03020100u | ((ne >> 1) & 0x04040404u);
  const uint32_t so = 0x03020100u | ((no >> 1) & 0x04040404u);
  const uint32_t ne7 = ne & 0x07070707u, no7 = no & 0x07070707u;
  const uint32_t el = sel4(T.lo, ne7, se), eh = sel4(T.hi, ne7, se);
  const uint32_t ol = sel4(T.lo, no7, so), oh = sel4(T.hi, no7, so);
  const uint32_t e02 = __builtin_amdgcn_perm(eh, el, 0x05010400u);  // (e0, e2)
  const uint32_t e46 = __builtin_amdgcn_perm(eh, el, 0x07030602u);  // (e4, e6)
  const uint32_t o13 = __builtin_amdgcn_perm(oh, ol, 0x05010400u);  // (e1, e3)
  const uint32_t o57 = __builtin_amdgcn_perm(oh, ol, 0x07030602u);  // (e5, e7)
  o[0] = __builtin_amdgcn_perm(o13, e02, 0x05040100u);
  o[1] = __builtin_amdgcn_perm(o13, e02, 0x07060302u);
  o[2] = __builtin_amdgcn_perm(o57, e46, 0x05040100u);
  o[3] = __builtin_amdgcn_perm(o57, e46, 0x07060302u);
}

// deq8 with the nibble order fixed at compile time: the codes are first put
// in element order (e0..e3 | e4..e7), so each output word is one v_perm of a
// low-byte and a high-byte lookup (29 VALU per 8 weights instead of 32).
// Same table entries, so the same bf16 values as deq8.
template <bool HI>
__device__ __forceinline__ void deq8o(uint32_t w, const Tbl& T, uint32_t (&o)[4]) {
  const uint32_t ne = (HI ? w >> 4 : w) & 0x0F0F0F0Fu;   // codes of elements 0,2,4,6
  const uint32_t no = (HI ? w : w >> 4) & 0x0F0F0F0Fu;   // codes of elements 1,3,5,7
  const uint32_t ca = __builtin_amdgcn_perm(no, ne, 0x05010400u);  // e0 e1 e2 e3
  const uint32_t cb = __builtin_amdgcn_perm(no, ne, 0x07030602u);  // e4 e5 e6 e7
  const uint32_t sa = 0x03020100u | ((ca >> 1) & 0x04040404u);
  const uint32_t sb = 0x03020100u | ((cb >> 1) & 0x04040404u);
  const uint32_t a7 = ca & 0x07070707u, b7 = cb & 0x07070707u;
  const uint32_t la = sel4(T.lo, a7, sa), ha = sel4(T.hi, a7, sa);
  const uint32_t lb = sel4(T.lo, b7, sb), hb = sel4(T.hi, b7, sb);
  o[0] = __builtin_amdgcn_perm(ha, la, 0x05010400u);
  o[1] = __builtin_amdgcn_perm(ha, la, 0x07030602u);
  o[2] = __builtin_amdgcn_perm(hb, lb, 0x05010400u);
  o[3] = __builtin_amdgcn_perm(hb, lb, 0x07030602u);
}

}  // namespace st
