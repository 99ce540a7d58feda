// Device helpers shared by the gfx950 kernels of the quantized weight path.
//
// Block formats (skyla-gguf/src/lib.rs:33-43, quant.rs:5-89) as the planner splits
// them into 16-byte regions (skyla-engine/src/planner.rs:8-15):
//   Q4_K 144 B / 256 values: region 0 = qs (128 B, 8 uint4), region 1 = header
//        (16 B: d f16 | dmin f16 | 12 packed 6-bit scale/min bytes).
//   Q6_K 210 B / 256 values: ql (128 B), qh (64 B), sc (16 x i8), d (f16 array).
//   Q8_0 34 B / 32 values: q (32 x i8 = 2 uint4), d (f16 array).
// Offsets arriving in push words are in units of the binding they index.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define SK_DEV static __device__ __forceinline__

SK_DEV float f16_bits_to_f32(uint32_t bits16) {
  return (float)__builtin_bit_cast(f16, (uint16_t)bits16);
}

// Loads of weights that a step reads once: non-temporal, so the lines are not kept in the
// caches at the expense of what is re-read (activations, headers shared by a workgroup).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
SK_DEV uint4 load_nt(const uint4 *p) {
  const u32x4_t t = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(t.x, t.y, t.z, t.w);
}
SK_DEV uint2 load_nt(const uint2 *p) {
  const u32x2_t t = __builtin_nontemporal_load((const u32x2_t *)p);
  return make_uint2(t.x, t.y);
}
SK_DEV uint16_t load_nt(const uint16_t *p) { return __builtin_nontemporal_load(p); }

SK_DEV f16x2 as_f16x2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
SK_DEV uint32_t as_u32(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// Round-to-nearest-even pack of two floats (v_cvt_pk_f16_f32 on gfx950).
SK_DEV f16x2 pack_f16x2(float a, float b) {
  f16x2 r = {(f16)a, (f16)b};
  return r;
}

// acc + a.x*b.x + a.y*b.y with f32 accumulation (v_dot2_f32_f16).
SK_DEV float dot2(f16x2 a, f16x2 b, float acc) {
  return __builtin_amdgcn_fdot2(a, b, acc, false);
}

// Sum over groups of LPR consecutive lanes of a wave64 (LPR in {16, 32, 64}); every lane
// of a group receives the group total.
template <int LPR>
SK_DEV float group_sum(float v) {
#pragma unroll
  for (int d = LPR / 2; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

template <int CTRL>
SK_DEV float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// Sum over groups of LPR consecutive lanes (16, 32 or 64) through DPP row operations (and
// one or two cross-row shuffles); every lane gets its group's total.
template <int LPR>
SK_DEV float lane_sum(float v) {
  v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);  // row_half_mirror: the two quads of each 8
  v += dpp_f<0x140>(v);  // row_mirror: the two halves of each 16
  if (LPR >= 32) v += __shfl_xor(v, 16, 64);
  if (LPR >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

SK_DEV uint32_t ctl_word(const uint32_t *ctl, uint32_t i) { return ctl[i]; }

// rmsnorm's row (rmsnorm.comp; ops.rs:1-16) of n <= 4096 values at 16-byte aligned x and w,
// 256 threads: thread t reads values 4 (t + 256 k), k < 4, of x and w as float4 (all loads in
// flight together) and gets y = x * r * w there (zeros past n), r = 1 / sqrt(mean(x^2) + eps),
// the sums of squares per wave added in wave order.  One workgroup barrier.
SK_DEV void norm_row4(const float *xr, const float *wr, uint32_t n, float eps, float4 (&y)[4]) {
#pragma clang fp contract(off)
  __shared__ float part[4];
  const uint32_t t = threadIdx.x, n4 = n >> 2;
  float4 xv[4], wv[4];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t i = t + 256 * k;
    xv[k] = wv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i < n4) {
      xv[k] = ((const float4 *)xr)[i];
      wv[k] = ((const float4 *)wr)[i];
    }
  }
#pragma unroll
  for (int k = 0; k < 4; k++) ss += ((xv[k].x * xv[k].x + xv[k].y * xv[k].y) + xv[k].z * xv[k].z) + xv[k].w * xv[k].w;
  ss = group_sum<64>(ss);
  if ((t & 63) == 0) part[t >> 6] = ss;
  __syncthreads();
  const float total = ((part[0] + part[1]) + part[2]) + part[3];
  const float r = 1.0f / sqrtf(total / (float)n + eps);
#pragma unroll
  for (int k = 0; k < 4; k++)
    y[k] = make_float4(xv[k].x * r * wv[k].x, xv[k].y * r * wv[k].y, xv[k].z * r * wv[k].z, xv[k].w * r * wv[k].w);
}

// ---------------------------------------------------------------------------------------
// f32 products of exact integer quants (the decode matvecs, matvec.hip).
// ---------------------------------------------------------------------------------------
// s + sum over the four bytes b of word v of f32(b) * x[b], in byte order: four
// v_cvt_f32_ubyte0..3 (exact for 0..255) and four FMAs.
SK_DEV float fma_bytes(uint32_t v, float4 x, float s) {
  s = __builtin_fmaf((float)(v & 255u), x.x, s);
  s = __builtin_fmaf((float)((v >> 8) & 255u), x.y, s);
  s = __builtin_fmaf((float)((v >> 16) & 255u), x.z, s);
  s = __builtin_fmaf((float)(v >> 24), x.w, s);
  return s;
}

// A mask constant the compiler cannot see through, held in an SGPR.  With a visible
// constant such as 0x0f0f0f0f the compiler knows which bits of the masked word are zero
// and extracts each byte with its own v_bfe_u32 before a v_cvt_f32_ubyte0 (two VALU per
// quant), instead of one v_and_b32 per word and v_cvt_f32_ubyte0..3 (one per quant).
SK_DEV uint32_t opaque_mask(uint32_t c) {
  uint32_t r;
  asm volatile("s_mov_b32 %0, %1" : "=s"(r) : "i"(c));
  return r;
}

// sum of the 16 products of the masked bytes of q (word k holds values 4k..4k+3) with x,
// starting from s
SK_DEV float fma_bytes16(uint4 q, uint32_t mask, const float4 (&x)[4], float s) {
  s = fma_bytes(q.x & mask, x[0], s);
  s = fma_bytes(q.y & mask, x[1], s);
  s = fma_bytes(q.z & mask, x[2], s);
  s = fma_bytes(q.w & mask, x[3], s);
  return s;
}

SK_DEV float sum4(float4 v) { return (v.x + v.y) + (v.z + v.w); }

// Buffer resource over [base, base + bytes) for raw buffer loads: a load whose offset is
// past the end returns zero instead of touching memory (range checked per dword).  The
// offset of a load is voffset (per lane) + soffset (wave-uniform), so a constant step of a
// uniform loop goes in the scalar operand and costs no vector instruction.  Word 3 is the
// gfx9 descriptor format (32-bit data, no swizzle).
typedef __amdgpu_buffer_rsrc_t BufRes;
SK_DEV BufRes buf_res(const void *base, uint64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                           (int)(uint32_t)(bytes < 0xffffffffull ? bytes : 0xffffffffull),
                                           0x00020000);
}
SK_DEV uint4 buf_load(BufRes r, uint32_t voffset, uint32_t soffset) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 0));
}
// the same, non-temporal (cache policy bit 1, nt)
SK_DEV uint4 buf_load_nt(BufRes r, uint32_t voffset, uint32_t soffset) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voffset, soffset, 2));
}

// ---------------------------------------------------------------------------------------
// Segmented launch.  Dispatches of one pipeline that the engine records with no barrier
// between them are independent (a barrier is how it orders them), so the runtime fuses up
// to MAXSEG of them into one launch: grid.x is the sum of their grid.x, and block b runs
// segment s = number of start[1..] <= b with its own push words, at block b - start[s].
// A single dispatch is the one-segment case.  Unused starts are 0xffffffff.
// ---------------------------------------------------------------------------------------
constexpr int MAXSEG = 4;

template <typename P>
struct Segments {
  uint32_t n;
  uint32_t start[MAXSEG];
  P p[MAXSEG];
};

template <typename P>
SK_DEV uint32_t segment_of(const Segments<P> &m, uint32_t b) {
  return (uint32_t)(b >= m.start[1]) + (uint32_t)(b >= m.start[2]) + (uint32_t)(b >= m.start[3]);
}

// push words of segment s (wave-uniform), selected without indexing the argument array
template <typename P>
SK_DEV P segment_push(const Segments<P> &m, uint32_t s) {
  P r = m.p[0];
  if (s == 1) r = m.p[1];
  if (s == 2) r = m.p[2];
  if (s == 3) r = m.p[3];
  return r;
}

// ---------------------------------------------------------------------------------------
// Bit-exact dequantisation of one 32-value group, in the reference's operation order.
// FP contraction is switched off inside these bodies: Rust never fuses a*b-c.
// ---------------------------------------------------------------------------------------

// q4k_scale_min (quant.rs:40-49) over the 12 scale bytes held in words y, z, w of the
// 16-byte header.
SK_DEV void q4k_scale_min(uint32_t j, uint32_t sy, uint32_t sz, uint32_t sw, uint32_t &sc,
                          uint32_t &m) {
  auto byte = [&](uint32_t k) -> uint32_t {
    uint32_t word = k < 4 ? sy : (k < 8 ? sz : sw);
    return (word >> (8 * (k & 3))) & 255u;
  };
  if (j < 4) {
    sc = byte(j) & 63u;
    m = byte(j + 4) & 63u;
  } else {
    sc = (byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4);
    m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
  }
}

// Q4_K sub-block `sub` (0..7) of one super-block: 32 values
//   o[i] = (d * sc) * q - (dmin * m)               (quant.rs:60-65)
// `qa`, `qb` are the two uint4 of qs holding chunk sub/2 (32 bytes); low nibbles for even
// sub, high nibbles for odd.
SK_DEV void dequant_q4k_sub(uint4 hdr, uint4 qa, uint4 qb, uint32_t sub, float o[32]) {
#pragma clang fp contract(off)
  float d = f16_bits_to_f32(hdr.x & 0xffffu);
  float dmin = f16_bits_to_f32(hdr.x >> 16);
  uint32_t sc, m;
  q4k_scale_min(sub, hdr.y, hdr.z, hdr.w, sc, m);
  float d0 = d * (float)sc;
  float min0 = dmin * (float)m;
  uint32_t shift = (sub & 1) * 4;
  uint32_t wds[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
  for (int i = 0; i < 32; i++) {
    uint32_t q = (wds[i >> 2] >> (8 * (i & 3) + shift)) & 15u;
    o[i] = d0 * (float)q - min0;
  }
}

// Q6_K: 32 values of group g (0..3) in half `hf` (0..1) of one super-block
//   o[l + 32 g] = (d * sc[is + 2g]) * q_g(l)       (quant.rs:70-89), is = l / 16
// ql: the 4 uint4 of ql for this half (64 B), qh: the 2 uint4 of qh (32 B), sc: 16 x i8.
SK_DEV void dequant_q6k_group(const uint4 ql[4], const uint4 qh[2], uint4 scw, float d,
                              uint32_t hf, uint32_t g, float o[32]) {
#pragma clang fp contract(off)
  uint32_t lw[16] = {ql[0].x, ql[0].y, ql[0].z, ql[0].w, ql[1].x, ql[1].y, ql[1].z, ql[1].w,
                     ql[2].x, ql[2].y, ql[2].z, ql[2].w, ql[3].x, ql[3].y, ql[3].z, ql[3].w};
  uint32_t hw[8] = {qh[0].x, qh[0].y, qh[0].z, qh[0].w, qh[1].x, qh[1].y, qh[1].z, qh[1].w};
  uint32_t sw[4] = {scw.x, scw.y, scw.z, scw.w};
  // q1: ql[l] lo, qh bits 0-1; q2: ql[l+32] lo, bits 2-3; q3: ql[l] hi, bits 4-5;
  // q4: ql[l+32] hi, bits 6-7.
  uint32_t lbase = (g & 1) ? 32 : 0;
  uint32_t nshift = (g >> 1) * 4;
  uint32_t hshift = 2 * g;
#pragma unroll
  for (int l = 0; l < 32; l++) {
    uint32_t li = lbase + l;
    uint32_t lb = (lw[li >> 2] >> (8 * (li & 3) + nshift)) & 15u;
    uint32_t hb = (hw[l >> 2] >> (8 * (l & 3) + hshift)) & 3u;
    int q = (int)(lb | (hb << 4)) - 32;
    uint32_t k = hf * 8 + (uint32_t)(l / 16) + 2 * g;
    int s = (int)(int8_t)((sw[k >> 2] >> (8 * (k & 3))) & 255u);
    o[l] = d * (float)s * (float)q;
  }
  (void)hf;
}

// Q8_0 block: o[i] = d * q[i]   (quant.rs:17-24)
SK_DEV void dequant_q8_0_block(uint4 qa, uint4 qb, float d, float o[32]) {
#pragma clang fp contract(off)
  uint32_t wds[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
  for (int i = 0; i < 32; i++) {
    int q = (int)(int8_t)((wds[i >> 2] >> (8 * (i & 3))) & 255u);
    o[i] = d * (float)q;
  }
}
