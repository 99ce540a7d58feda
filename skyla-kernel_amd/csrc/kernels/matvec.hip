// Decode matvec (M = 1) over raw Q4_K / Q6_K / Q8_0 blocks for gfx950.
//
// Contract (what skyla-engine dispatches, graph.rs:23-34 and graph/moe.rs:8-24):
//   pipeline spec [WAVES, ACCUM, ROWS, MOE, LPR] (kernels.rs:92-97), workgroup = WAVES
//   wave64s, each lane group of LPR lanes owns ROWS consecutive output rows, so one
//   workgroup covers WAVES * ROWS * 64 / LPR rows and grid.x = ceil(n_out / that).
//   MOE: grid.y = slot; the expert is ids[ids_off + slot] and rows are offset by
//   expert * n_out (matvec_q4k.comp:68-71).  x and y move by x_stride / y_stride per slot.
//   ACCUM adds into y (residual add for O and down).
//
// Inner loop (MI355X-specific):
//   * one 16-byte coalesced load per row per lane per step (64 lanes read 1 KiB of a row
//     contiguously), the loads of every row of the step issued before any math, and the
//     next step's loads issued before the current step's math;
//   * activations are read once per step and shared by the ROWS rows: converted to f16
//     pairs (RNE) in the order the packed weights need them;
//   * weights are never converted to float one by one: a quant is OR-ed into the
//     mantissa of the f16 constant 1024.0 (0x6400), giving 1024+q exactly, and
//     v_dot2_f32_f16 multiplies two of them by two activations with f32 accumulation.
//     The accumulator starts at -1024 * sum(x) (the f16 activations' own sum), which
//     cancels the offset.  High nibbles are taken in place as 1024+16q (no shift) and
//     the group total is scaled by 1/16 afterwards.
//   * the sub-block scales are applied once per 16 (Q4_K, Q6_K) or 16 (Q8_0) values
//     per row, in f32;
//   * one shuffle reduction per row at the end; lane 0 of each lane group writes.
// Numerics: f16 activations (relative error 2^-11 per element) and f32 accumulation; the
// result differs from the reference's f32 dot only by rounding, far inside the 1e-2
// relative-L2 bar.
#include "common.h"

#define MAGIC 0x64006400u  // f16x2 {1024.0, 1024.0}

struct MatvecPush2 {  // Q4_K and Q8_0 (9 words, graph.rs:30 / graph/moe.rs:251-255)
  uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride;
};

struct MatvecPush4 {  // Q6_K (11 words, graph.rs:29 / graph/moe.rs:252)
  uint32_t o0, o1, o2, o3, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride;
};

SK_DEV float4 ld_x4(const float *p) { return *(const float4 *)p; }

// Converts 16 consecutive activations v[0..15] into the pair order of the packed quants:
// for dword k of a 16-byte weight unit, pair02 = (v[4k], v[4k+2]), pair13 = (v[4k+1],
// v[4k+3]).  Returns the sum of the f16 values (f32 accumulation).
SK_DEV float x16_pairs(const float4 v[4], f16x2 p02[4], f16x2 p13[4]) {
  const f16x2 one = {(f16)1.0f, (f16)1.0f};
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; k++) {
    p02[k] = pack_f16x2(v[k].x, v[k].z);
    p13[k] = pack_f16x2(v[k].y, v[k].w);
    s = dot2(p02[k], one, s);
    s = dot2(p13[k], one, s);
  }
  return s;
}

// Writes the reduced row results.  Lane 0 of each LPR group stores ROWS values.
template <int ACCUM, int ROWS, int LPR>
SK_DEV void store_rows(float *y, uint32_t y_off, uint32_t first, uint32_t n_out, uint32_t lane,
                       float acc[ROWS]) {
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    float total = group_sum<LPR>(acc[r]);
    uint32_t row = first + r;
    if (lane == 0 && row < n_out) {
      if (ACCUM)
        y[y_off + row] += total;
      else
        y[y_off + row] = total;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Q4_K: lane step = one 16-byte unit of qs (32 quants) per row.
// Unit u of a row: super-block u/8, chunk c = (u%8)/2, half h = u%2.  Its low nibbles are
// values 64c + 16h + [0,16) of sub-block 2c, its high nibbles values 64c + 32 + 16h +
// [0,16) of sub-block 2c+1 (quant.rs:56-66).
// ---------------------------------------------------------------------------------------
template <int WAVES, int ACCUM, int ROWS, int MOE, int LPR>
SK_DEV void matvec_q4k_body(const uint4 *__restrict__ w, const float *x, float *y,
                            const uint32_t *ids, const MatvecPush2 &p) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = (tid & 63) % LPR;
  const uint32_t sub = (tid & 63) / LPR;
  const uint32_t wave = blockIdx.x * WAVES + (tid >> 6);
  const uint32_t first = (wave * (64 / LPR) + sub) * ROWS;
  if (LPR == 64 && first >= p.n_out) return;
  const uint32_t slot = blockIdx.y;
  const uint32_t base = MOE ? ids[p.ids_off + slot] * p.n_out : 0;
  const float *xs = x + p.x_off + slot * p.x_stride;
  const uint32_t y_off = p.y_off + slot * p.y_stride;
  const uint32_t units = p.n_in >> 5;
  const uint32_t supers = p.n_in >> 8;

  const uint4 *qs[ROWS];
  const uint4 *hd[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    uint32_t row = base + min(first + r, p.n_out - 1);
    qs[r] = w + p.o0 + row * units;
    hd[r] = w + p.o1 + row * supers;
  }

  // Per-lane constants of the scale unpack (u % 8 == lane % 8 for every step).
  const uint32_t c = (lane >> 1) & 3;
  const uint32_t xlane = c * 64 + (lane & 1) * 16;
  const uint32_t sh = (c & 1) * 16;
  const bool hi = c >= 2;
  const uint32_t mW = hi ? 0x0f0fu : 0u;
  const uint32_t s2 = hi ? 2u : 0u;
  const uint32_t mY = hi ? 0x3030u : 0x3f3fu;

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;

  uint32_t u = lane;
  uint4 q[ROWS], h[ROWS];
  float4 xa[4], xb[4];
  if (u < units) {
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      q[r] = qs[r][u];
      h[r] = hd[r][u >> 3];
    }
    const float *xp = xs + (u >> 3) * 256 + xlane;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      xa[k] = ld_x4(xp + 4 * k);
      xb[k] = ld_x4(xp + 32 + 4 * k);
    }
  }
  for (; u < units; u += LPR) {
    const uint32_t un = u + LPR;
    uint4 qn[ROWS], hn[ROWS];
    float4 xan[4], xbn[4];
    if (un < units) {
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        qn[r] = qs[r][un];
        hn[r] = hd[r][un >> 3];
      }
      const float *xp = xs + (un >> 3) * 256 + xlane;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        xan[k] = ld_x4(xp + 4 * k);
        xbn[k] = ld_x4(xp + 32 + 4 * k);
      }
    }

    f16x2 a02[4], a13[4], b02[4], b13[4];
    const float sum_a = x16_pairs(xa, a02, a13);
    const float sum_b = x16_pairs(xb, b02, b13);
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      float sa = -1024.0f * sum_a;
      float sb = -1024.0f * sum_b;
      const uint32_t wd[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t w0 = wd[k];
        const uint32_t w8 = w0 >> 8;
        sa = dot2(as_f16x2((w0 & 0x000f000fu) | MAGIC), a02[k], sa);
        sa = dot2(as_f16x2((w8 & 0x000f000fu) | MAGIC), a13[k], sa);
        sb = dot2(as_f16x2((w0 & 0x00f000f0u) | MAGIC), b02[k], sb);
        sb = dot2(as_f16x2((w8 & 0x00f000f0u) | MAGIC), b13[k], sb);
      }
      // scales/mins j = 2c, 2c+1 (quant.rs:40-49), two bytes at a time
      const uint32_t ys = h[r].y >> sh, zs = h[r].z >> sh, ws = h[r].w >> sh;
      const uint32_t scv = (ws & mW) | ((ys >> s2) & mY);
      const uint32_t mv = ((ws >> 4) & mW) | ((zs >> s2) & mY);
      const float sc0 = (float)(scv & 0xffu), sc1 = (float)((scv >> 8) & 0xffu);
      const float m0 = (float)(mv & 0xffu), m1 = (float)((mv >> 8) & 0xffu);
      const float d = f16_bits_to_f32(h[r].x & 0xffffu);
      const float dmin = f16_bits_to_f32(h[r].x >> 16);
      const float t = sc0 * sa + (sc1 * 0.0625f) * sb;
      const float mt = m0 * sum_a + m1 * sum_b;
      acc[r] += d * t - dmin * mt;
    }
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      q[r] = qn[r];
      h[r] = hn[r];
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      xa[k] = xan[k];
      xb[k] = xbn[k];
    }
  }
  store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc);
}

// ---------------------------------------------------------------------------------------
// Q6_K: lane step = 64 values of one super-block: u -> super-block u/4, half (u%4)/2,
// li = u%2.  It reads 16 B of ql at l = 16 li (a), 16 B at l + 32 (b), 16 B of qh (h),
// the 16 scale bytes and d.  Groups g = 0..3 are values 128 half + 32 g + 16 li + [0,16)
// with scale sc[8 half + li + 2g] (quant.rs:72-87).
// ---------------------------------------------------------------------------------------
template <int WAVES, int ACCUM, int ROWS, int MOE, int LPR>
SK_DEV void matvec_q6k_body(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd,
                            const float *x, float *y, const uint32_t *ids,
                            const MatvecPush4 &p) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = (tid & 63) % LPR;
  const uint32_t sub = (tid & 63) / LPR;
  const uint32_t wave = blockIdx.x * WAVES + (tid >> 6);
  const uint32_t first = (wave * (64 / LPR) + sub) * ROWS;
  if (LPR == 64 && first >= p.n_out) return;
  const uint32_t slot = blockIdx.y;
  const uint32_t base = MOE ? ids[p.ids_off + slot] * p.n_out : 0;
  const float *xs = x + p.x_off + slot * p.x_stride;
  const uint32_t y_off = p.y_off + slot * p.y_stride;
  const uint32_t units = p.n_in >> 6;
  const uint32_t supers = p.n_in >> 8;

  uint32_t rowbase[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) rowbase[r] = (base + min(first + r, p.n_out - 1)) * supers;

  const uint32_t li = lane & 1;
  const uint32_t hf = (lane >> 1) & 1;
  const uint32_t inner = hf * 4 + li;           // uint4 index of `a` inside the block's ql
  const uint32_t xlane = hf * 128 + li * 16;    // first value of group 0
  const uint32_t bsh = li * 8;                  // byte of sc inside the selected word

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;

  for (uint32_t u = lane; u < units; u += LPR) {
    const uint32_t sb = u >> 2;
    uint4 qa[ROWS], qb[ROWS], qh[ROWS], sc[ROWS];
    uint32_t dd[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      const uint32_t rs = rowbase[r] + sb;
      qa[r] = w[p.o0 + rs * 8 + inner];
      qb[r] = w[p.o0 + rs * 8 + inner + 2];
      qh[r] = w[p.o1 + rs * 4 + hf * 2 + li];
      sc[r] = w[p.o2 + rs];
      dd[r] = wd[p.o3 + rs];
    }
    const float *xp = xs + sb * 256 + xlane;
    float4 xv[4][4];
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
      for (int k = 0; k < 4; k++) xv[g][k] = ld_x4(xp + 32 * g + 4 * k);
    f16x2 p02[4][4], p13[4][4];
    float xsum[4];
#pragma unroll
    for (int g = 0; g < 4; g++) xsum[g] = x16_pairs(xv[g], p02[g], p13[g]);

#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      // groups 0,1 hold 1024+q, groups 2,3 hold 1024+16q; q is the stored 6-bit value
      // and the quant is q-32: the starting values cancel both offsets.
      float s0 = -1056.0f * xsum[0], s1 = -1056.0f * xsum[1];
      float s2 = -1536.0f * xsum[2], s3 = -1536.0f * xsum[3];
      const uint32_t av[4] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w};
      const uint32_t bv[4] = {qb[r].x, qb[r].y, qb[r].z, qb[r].w};
      const uint32_t hv[4] = {qh[r].x, qh[r].y, qh[r].z, qh[r].w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t a0 = av[k], b0 = bv[k], h0 = hv[k];
        const uint32_t a8 = a0 >> 8, b8 = b0 >> 8, h8 = h0 >> 8;
        const uint32_t h4 = h0 << 4, h2 = h0 << 2, h84 = h8 << 4, h82 = h8 << 2;
        s0 = dot2(as_f16x2((a0 & 0x000f000fu) | MAGIC | (h4 & 0x00300030u)), p02[0][k], s0);
        s0 = dot2(as_f16x2((a8 & 0x000f000fu) | MAGIC | (h84 & 0x00300030u)), p13[0][k], s0);
        s1 = dot2(as_f16x2((b0 & 0x000f000fu) | MAGIC | (h2 & 0x00300030u)), p02[1][k], s1);
        s1 = dot2(as_f16x2((b8 & 0x000f000fu) | MAGIC | (h82 & 0x00300030u)), p13[1][k], s1);
        s2 = dot2(as_f16x2((a0 & 0x00f000f0u) | MAGIC | (h4 & 0x03000300u)), p02[2][k], s2);
        s2 = dot2(as_f16x2((a8 & 0x00f000f0u) | MAGIC | (h84 & 0x03000300u)), p13[2][k], s2);
        s3 = dot2(as_f16x2((b0 & 0x00f000f0u) | MAGIC | (h2 & 0x03000300u)), p02[3][k], s3);
        s3 = dot2(as_f16x2((b8 & 0x00f000f0u) | MAGIC | (h82 & 0x03000300u)), p13[3][k], s3);
      }
      const uint32_t w0 = hf ? sc[r].z : sc[r].x;
      const uint32_t w1 = hf ? sc[r].w : sc[r].y;
      const float c0 = (float)(int32_t)__builtin_amdgcn_sbfe(w0, bsh, 8);
      const float c1 = (float)(int32_t)__builtin_amdgcn_sbfe(w0, bsh + 16, 8);
      const float c2 = (float)(int32_t)__builtin_amdgcn_sbfe(w1, bsh, 8);
      const float c3 = (float)(int32_t)__builtin_amdgcn_sbfe(w1, bsh + 16, 8);
      const float t = c0 * s0 + c1 * s1 + 0.0625f * (c2 * s2 + c3 * s3);
      acc[r] += f16_bits_to_f32(dd[r]) * t;
    }
  }
  store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc);
}

// ---------------------------------------------------------------------------------------
// Q8_0: lane step = 16 quants (half a block) per row; d is block u/2's f16 scale.
// q as f16: (q ^ 0x80) is 0..255, so MAGIC | that = 1152 + q exactly.
// ---------------------------------------------------------------------------------------
template <int WAVES, int ACCUM, int ROWS, int MOE, int LPR>
SK_DEV void matvec_q8_0_body(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd,
                             const float *x, float *y, const uint32_t *ids,
                             const MatvecPush2 &p) {
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = (tid & 63) % LPR;
  const uint32_t sub = (tid & 63) / LPR;
  const uint32_t wave = blockIdx.x * WAVES + (tid >> 6);
  const uint32_t first = (wave * (64 / LPR) + sub) * ROWS;
  if (LPR == 64 && first >= p.n_out) return;
  const uint32_t slot = blockIdx.y;
  const uint32_t base = MOE ? ids[p.ids_off + slot] * p.n_out : 0;
  const float *xs = x + p.x_off + slot * p.x_stride;
  const uint32_t y_off = p.y_off + slot * p.y_stride;
  const uint32_t chunks = p.n_in >> 4;
  const uint32_t blocks = p.n_in >> 5;

  uint32_t rq[ROWS], rd[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    const uint32_t row = base + min(first + r, p.n_out - 1);
    rq[r] = p.o0 + row * chunks;
    rd[r] = p.o1 + row * blocks;
  }
  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;

  for (uint32_t c = lane; c < chunks; c += LPR) {
    uint4 q[ROWS];
    uint32_t dd[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      q[r] = w[rq[r] + c];
      dd[r] = wd[rd[r] + (c >> 1)];
    }
    float4 xv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) xv[k] = ld_x4(xs + c * 16 + 4 * k);
    f16x2 p02[4], p13[4];
    const float xsum = x16_pairs(xv, p02, p13);
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      float s = -1152.0f * xsum;
      const uint32_t wv[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t b = wv[k] ^ 0x80808080u;
        s = dot2(as_f16x2((b & 0x00ff00ffu) | MAGIC), p02[k], s);
        s = dot2(as_f16x2(((b >> 8) & 0x00ff00ffu) | MAGIC), p13[k], s);
      }
      acc[r] += f16_bits_to_f32(dd[r]) * s;
    }
  }
  store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc);
}

// ---------------------------------------------------------------------------------------
// Exported instantiations: symbol = <shader name>__<spec words joined by '_'>.
// ---------------------------------------------------------------------------------------
#define MV_Q4K(W, A, R, M, L)                                                                \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q4k__##W##_##A##_##R##_##M##_##L( \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, MatvecPush2 p) {        \
    matvec_q4k_body<W, A, R, M, L>(w, x, y, ids, p);                                         \
  }
#define MV_Q6K(W, A, R, M, L)                                                                \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q6k__##W##_##A##_##R##_##M##_##L( \
      const uint4 *w, const uint16_t *wd, const float *x, float *y, const uint32_t *ids,     \
      MatvecPush4 p) {                                                                       \
    matvec_q6k_body<W, A, R, M, L>(w, wd, x, y, ids, p);                                     \
  }
#define MV_Q8_0(W, A, R, M, L)                                                                \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q8_0__##W##_##A##_##R##_##M##_##L( \
      const uint4 *w, const uint16_t *wd, const float *x, float *y, const uint32_t *ids,      \
      MatvecPush2 p) {                                                                        \
    matvec_q8_0_body<W, A, R, M, L>(w, wd, x, y, ids, p);                                     \
  }

// dense (MOE = 0, LPR = 64) and expert (ACCUM = 0, MOE = 1, LPR in {64, 32, 16})
// instantiations for each (WAVES, ROWS) tactic
#define MV_TACTIC(F, W, R) \
  F(W, 0, R, 0, 64)        \
  F(W, 1, R, 0, 64)        \
  F(W, 0, R, 1, 64)        \
  F(W, 0, R, 1, 32)        \
  F(W, 0, R, 1, 16)

#define MV_ALL_TACTICS(F) \
  MV_TACTIC(F, 1, 1)      \
  MV_TACTIC(F, 1, 2)      \
  MV_TACTIC(F, 1, 4)      \
  MV_TACTIC(F, 2, 1)      \
  MV_TACTIC(F, 2, 2)      \
  MV_TACTIC(F, 2, 4)      \
  MV_TACTIC(F, 4, 1)      \
  MV_TACTIC(F, 4, 2)      \
  MV_TACTIC(F, 4, 4)      \
  MV_TACTIC(F, 8, 1)      \
  MV_TACTIC(F, 8, 2)

MV_ALL_TACTICS(MV_Q4K)
MV_ALL_TACTICS(MV_Q6K)
MV_ALL_TACTICS(MV_Q8_0)
