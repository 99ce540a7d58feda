// Decode matvec (M = 1) over raw Q4_K / Q6_K / Q8_0 blocks for gfx950.
//
// Contract (what skyla-engine dispatches, graph.rs:23-34 and graph/moe.rs:8-24):
//   pipeline spec [WAVES, ACCUM, ROWS, MOE, LPR] (kernels.rs:92-97): a workgroup is WAVES
//   wave64s; each group of LPR lanes owns ROWS consecutive output rows, so a workgroup covers
//   RWG = WAVES * (64 / LPR) * ROWS rows and grid.x = ceil(n_out / RWG).  MOE: grid.y = slot,
//   the expert is ids[ids_off + slot] and its rows start at expert * n_out
//   (matvec_q4k.comp:68-71); x and y move by x_stride / y_stride per slot.  ACCUM adds into y.
//
// Budget that shapes the kernel: at 8 TB/s each of the 256 CUs must consume ~13 B/clk of
// weights (~23 Q4_K values/clk) while it has 64 VALU lane-ops/clk and ~64 B/clk of L1.
//   * Activations are staged once per workgroup in LDS as f16 pairs in the order the packed
//     quants need them, with their per-16 sums, instead of every wave re-reading f32 x
//     through L1 (4x the weight bytes at two rows per wave).
//   * Each (row, super-block) header is decoded once per workgroup into f32 products
//     d*sc and dmin*m (the reference's d0 / min0, quant.rs:60-61), so a lane's per-row work
//     is the quant extraction, v_dot2 and four FMAs.
//   * A quant is OR-ed into the mantissa of the f16 constant 1024.0 (0x6400), giving 1024+q
//     exactly; v_dot2_f32_f16 multiplies two of them by two activations with f32
//     accumulation, and the accumulator starts at -1024 * sum(x) to cancel the offset.  High
//     nibbles are taken in place as 1024+16q (no shift) and their scale carries the 1/16.
//   * Weight loads are 16 B per lane, 1 KiB contiguous per wave instruction, and the first
//     step's loads are issued before the staging so they overlap it.
// Numerics: f16 activations (relative rounding 2^-11) with f32 accumulation -- within 1e-4
// relative L2 of the reference's f32 dot in practice, far inside the 1e-2 bar.
#include "common.h"

#define MAGIC 0x64006400u  // f16x2 {1024.0, 1024.0}

namespace {

struct MatvecPush2 {  // Q4_K and Q8_0 (9 words, graph.rs:30 / graph/moe.rs:251-255)
  uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride;
};

struct MatvecPush4 {  // Q6_K (11 words, graph.rs:29 / graph/moe.rs:252)
  uint32_t o0, o1, o2, o3, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride;
};

// The fused forms (matvec_*_silu, matvec_*_norm) append two words: the offset of the
// second activation vector (the up rows, or the RMSNorm weights) and the norm's eps.
struct MatvecPush2F {
  uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride, aux_off;
  float eps;
};
// matvec_q4k_glu: the gate matrix's regions, then the up matrix's (11 words)
struct MatvecPushGlu {
  uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride, u0, u1;
};
// matvec_q4k_glun: matvec_q4k_glu's words, then the norm weights and eps (13 words)
struct MatvecPushGluN {
  uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride, u0, u1, aux_off;
  float eps;
};
struct MatvecPush4F {
  uint32_t o0, o1, o2, o3, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride, aux_off;
  float eps;
};

// (a & m) | o as one v_and_or_b32 with register operands (the compiler otherwise splits it
// in two, because gfx9 VOP3 encodings take no literal).
SK_DEV uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
  return r;
}

template <int ACCUM, int ROWS, int LPR>
SK_DEV void store_rows(float *y, uint32_t y_off, uint32_t first, uint32_t n_out, uint32_t lane,
                       const float (&acc)[ROWS]) {
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    const float total = lane_sum<LPR>(acc[r]);
    const uint32_t row = first + r;
    if (lane == 0 && row < n_out) {
      if (ACCUM)
        y[y_off + row] += total;
      else
        y[y_off + row] = total;
    }
  }
}

SK_DEV uint32_t pk(float a, float b) { return as_u32(pack_f16x2(a, b)); }

// Range guard of the f16 activation staging.  A pass's activations are staged as f16, whose
// range ends at 65504, while the reference multiplies f32 activations (matvec_q4k.comp,
// matvec_q6k.comp, matvec_q8_0.comp) and inputs such as silu(g) * u reach 1e5-1e6.  Each
// wave notes in its LDS word the largest |x| >= 2^15 it staged (as float bits, which order
// like the values for x >= 0; a NaN counts as inf); lane 0 clears the word first, and one
// wave's LDS operations complete in issue order, so only lanes holding such a value pay for
// an LDS atomic.  A pass holding |x| >= 2^15 (or a NaN / inf, which no scaling helps) is staged
// again as x * 2^-e, e = exponent(max) - 14, and the rows' accumulators are scaled by 2^-e
// before that pass's steps and by 2^e after: exact powers of two, so the result is the
// unscaled sum up to the f16 rounding of the scaled values.  Passes without large values
// (all of them in practice) take the unscaled staging as is.
SK_DEV float abs_max4(float4 v) { return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))); }

SK_DEV void guard_note(uint32_t *wmax, float m) {
  uint32_t *slot = wmax + (threadIdx.x >> 6);
  if ((threadIdx.x & 63) == 0) *slot = 0u;
  if (!(m < 32768.0f)) atomicMax(slot, m == m ? __builtin_bit_cast(uint32_t, m) : 0x7f800000u);
}

// after the barrier that ends the staging: the pass's exponent (0: no scaling)
template <int WAVES>
SK_DEV int guard_exp(const uint32_t *wmax) {
  uint32_t m = 0u;
#pragma unroll
  for (int w = 0; w < WAVES; w++) m = max(m, wmax[w]);
  const int e = m == 0u || m >= 0x7f800000u ? 0 : (int)(m >> 23) - 127 - 14;
  return __builtin_amdgcn_readfirstlane(e);  // the same in every lane: keep it scalar
}

template <int ROWS>
SK_DEV void scale_rows(float (&acc)[ROWS], int e) {
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = __builtin_ldexpf(acc[r], e);
}

// Fused activation forms.  MODE 1 (SiLU; silu_mul.comp:15-23) stages x / (1 + e^-x) * aux:
// the down projection reads the gate and up rows itself.  MODE 2 (RMSNorm; rmsnorm.comp,
// ops.rs:1-16) stages x * aux (the norm weights) and adds x^2 to ss; the row's
// r = 1 / sqrt(sum / n_in + eps) multiplies the sums before they are stored, since every
// output is linear in the staged vector.  Every workgroup reads the whole x anyway, so each
// computes the same sum of squares itself (in the same order) and no separate launch runs.
template <int MODE>
SK_DEV float4 fuse4(float4 v, float4 aux, float &ss) {
#pragma clang fp contract(off)
  if constexpr (MODE == 1) {
    v.x = v.x / (1.0f + expf(-v.x)) * aux.x;
    v.y = v.y / (1.0f + expf(-v.y)) * aux.y;
    v.z = v.z / (1.0f + expf(-v.z)) * aux.z;
    v.w = v.w / (1.0f + expf(-v.w)) * aux.w;
  } else if constexpr (MODE == 2 || MODE == 4) {
    ss += ((v.x * v.x + v.y * v.y) + v.z * v.z) + v.w * v.w;
    v = make_float4(v.x * aux.x, v.y * aux.y, v.z * aux.z, v.w * aux.w);
  }
  return v;
}

// MODE 2: the pass's sums of squares, one per 16 lanes, into wss before the staging
// barrier; after it every thread adds all of them in the same order.
template <int MODE, int WAVES>
SK_DEV void norm_note(float *wss, float ssp) {
  if constexpr (MODE == 2 || MODE == 4) {
    const float v = lane_sum<16>(ssp);
    if ((threadIdx.x & 15) == 0) wss[threadIdx.x >> 4] = v;
  }
}
template <int MODE, int WAVES>
SK_DEV void norm_take(const float *wss, float &ss) {
  if constexpr (MODE == 2 || MODE == 4) {
#pragma unroll
    for (int i = 0; i < 4 * WAVES; i++) ss += wss[i];
  }
}
template <int MODE, int ROWS, typename P>
SK_DEV void norm_apply(float (&acc)[ROWS], float ss, const P &p) {
  if constexpr (MODE == 2 || MODE == 4) {
    const float r = 1.0f / sqrtf(ss / (float)p.n_in + p.eps);
#pragma unroll
    for (int i = 0; i < ROWS; i++) acc[i] *= r;
  }
}

// Geometry shared by the three formats.
template <int WAVES, int ROWS, int LPR>
struct Geo {
  static constexpr int SUBS = 64 / LPR;            // row groups per wave
  static constexpr int RWG = WAVES * SUBS * ROWS;  // rows per workgroup
  static constexpr int NT = 64 * WAVES;            // threads per workgroup
  // super-blocks of activations staged per pass: keeps the decoded scales <= 32 KiB
  static constexpr int CH_SUP = (512 / RWG) < 1 ? 1 : ((512 / RWG) > 32 ? 32 : (512 / RWG));
  static constexpr int CH = CH_SUP * 256;          // values per pass
};

// ---------------------------------------------------------------------------------------
// Q4_K.  Lane step = one 16 B unit of qs: unit u of a row is super-block u/8, chunk
// c = (u/2)%4, bytes 16(u%2) + [0,16) of that chunk's 32 -- low nibbles are values
// 64c + 16(u%2) + [0,16) of sub-block 2c, high nibbles the same positions of sub-block 2c+1
// (quant.rs:56-66).  LDS per pass: xq[0..3][unit] = the unit's 32 activations as f16 pairs in
// the (0,2),(1,3) order of the packed quants (low-nibble half, then high), xs[unit] = their
// two 16-value sums, and per (row, super-block, chunk) four products of the header
// (quant.rs:40-49, 60-61): d*sc_lo, d*sc_hi/16, and the terms that multiply the two sums,
// 1024*d*sc_lo + dmin*m_lo and 64*d*sc_hi + dmin*m_hi (the 1024 cancels the f16 offset of
// the packed quants, so a lane's dot products start from zero).
//
// Every lane of a workgroup runs the same number of steps S = ceil(units / LPR): units past
// the pass hold zero activations and zero products, so they add exactly zero, and the loop
// carries no per-lane guard.  Weights and headers are read through buffer resources that
// end at the matrix (rows past n_out are clamped, reads past the end return zero), so the
// ring's loads take their step offset in the scalar operand and need no address math.
// Activations are staged by all threads, a quarter unit (8 floats) each, so no thread
// holds more than 64 B of them in flight.
// ---------------------------------------------------------------------------------------
template <int WAVES, int ROWS, int LPR>
struct GeoQ4 {
  static constexpr int SUBS = 64 / LPR;
  static constexpr int RWG = WAVES * SUBS * ROWS;
  static constexpr int NT = 64 * WAVES;
  static constexpr int CH_A = (512 / RWG) < 1 ? 1 : ((512 / RWG) > 32 ? 32 : (512 / RWG));
  static constexpr int CH_B = CH_A > NT / 16 ? NT / 16 : CH_A;      // <= 64 B of x per thread
  static constexpr int CH_SUP = CH_B < LPR / 8 ? LPR / 8 : CH_B;     // super-blocks per pass
  static constexpr int CHU = CH_SUP * 8;                           // units per pass
  // weight steps in flight: 16 VGPRs of ring, and no more steps than a 4096-value row has
  static constexpr int PF = (ROWS >= 4 ? 1 : 4 / ROWS) > 128 / LPR ? 128 / LPR : (ROWS >= 4 ? 1 : 4 / ROWS);
  static_assert(CHU % LPR == 0, "a full pass gives every lane the same number of steps");
};

template <int WAVES, int ACCUM, int ROWS, int MOE, int LPR, int MODE = 0, typename P = MatvecPush2>
SK_DEV void matvec_q4k_body(const uint4 *__restrict__ w, const float *x, float *y,
                            const uint32_t *ids, const P &p, uint32_t bx) {
  using G = GeoQ4<WAVES, ROWS, LPR>;
  constexpr int CHU = G::CHU, PF = G::PF;
  __shared__ uint4 xq[4][CHU];  // component-major: lanes read consecutive 16 B
  __shared__ float2 xs[CHU];
  __shared__ float4 sc[G::RWG][G::CH_SUP][4];
  __shared__ uint32_t wmax[WAVES];
  __shared__ float wss[MODE == 2 || MODE == 4 ? 4 * WAVES : 1];
  // MODE 3 (gate and up in one launch): the first half of the waves computes gate rows,
  // the second half the up rows of the same outputs, and the store writes silu(g) * u.
  // MODE 4: MODE 3 with the FFN RMSNorm folded in as MODE 2 folds it (x * w staged, r
  // applied to the gate and up sums before the SiLU)
  constexpr bool PAIR = MODE == 3 || MODE == 4, AUX = MODE == 1 || MODE == 2 || MODE == 4;
  constexpr int OUT = PAIR ? G::RWG / 2 : G::RWG;  // outputs per workgroup
  __shared__ float ush[PAIR ? OUT : 1];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = (tid & 63) % LPR;
  const uint32_t sub = (tid & 63) / LPR;
  const uint32_t row0 = bx * OUT;
  const uint32_t wv = tid >> 6;
  const bool second = PAIR && wv >= (uint32_t)WAVES / 2;
  const uint32_t lrow0 = ((PAIR ? wv % (WAVES / 2) : wv) * G::SUBS + sub) * ROWS;  // first row of this group
  const uint32_t hrow0 = (second ? OUT : 0) + lrow0;  // its header rows in LDS
  const uint32_t first = row0 + lrow0;
  const uint32_t slot = blockIdx.y;
  const uint32_t base = MOE ? ids[p.ids_off + slot] * p.n_out : 0;
  const float *xv = x + p.x_off + slot * p.x_stride;
  const float *av = x;  // MODE 1, 2: the second vector, indexed as xv
  if constexpr (AUX) av = x + p.aux_off + (MODE == 1 ? slot * p.x_stride : 0);
  float ss = 0.0f;      // MODE 2: sum of x^2 over the passes so far
  const uint32_t y_off = p.y_off + slot * p.y_stride;
  const uint32_t units = p.n_in >> 5, supers = p.n_in >> 8;
  const uint32_t c = (lane >> 1) & 3;  // chunk of this lane's units (u % 8 == lane % 8)
  const uint32_t MW = MAGIC, LO = 0x000f000fu, HI = 0x00f000f0u;

  uint32_t mo0 = p.o0, mo1 = p.o1;  // this wave's matrix
  if constexpr (PAIR) {
    mo0 = __builtin_amdgcn_readfirstlane(second ? p.u0 : p.o0);
    mo1 = __builtin_amdgcn_readfirstlane(second ? p.u1 : p.o1);
  }
  const BufRes wq = buf_res(w + mo0, (uint64_t)(base + p.n_out) * units * 16);
  const BufRes wh = buf_res(w + p.o1, (uint64_t)(base + p.n_out) * supers * 16);
  uint32_t voff[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) voff[r] = ((base + min(first + r, p.n_out - 1)) * units + lane) * 16;

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;

  for (uint32_t k0 = 0; k0 < p.n_in; k0 += CHU * 32) {
    const uint32_t nk = min(p.n_in - k0, (uint32_t)CHU * 32);
    const uint32_t u0 = k0 >> 5, nu = nk >> 5, s0 = k0 >> 8, ns = nk >> 8;
    if (k0 != 0) __syncthreads();  // the previous pass is done with the LDS
    // Load order matters (a wave's loads complete in issue order): activations, then
    // headers, then the first PF weight steps, so staging waits only for its own data.
    constexpr int XI = (4 * CHU + G::NT - 1) / G::NT;  // activation quarters per thread
    float4 xa[XI][2], xu[AUX ? XI : 1][2];
    auto load_x = [&]() {
#pragma unroll
      for (int j = 0; j < XI; j++) {
        const uint32_t t = tid + j * G::NT, u = u0 + (t >> 2), qq = t & 3;
        xa[j][0] = xa[j][1] = make_float4(0.f, 0.f, 0.f, 0.f);  // every path defines them
        if constexpr (AUX) xu[j][0] = xu[j][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < 4 * nu) {
          const uint32_t at = (u >> 3) * 256 + ((u >> 1) & 3) * 64 + (u & 1) * 16 + (qq >> 1) * 32 + (qq & 1) * 8;
          xa[j][0] = *(const float4 *)(xv + at);
          xa[j][1] = *(const float4 *)(xv + at + 4);
          if constexpr (AUX) {
            xu[j][0] = *(const float4 *)(av + at);
            xu[j][1] = *(const float4 *)(av + at + 4);
          }
        }
      }
    };
    load_x();
    constexpr int NH = G::RWG * G::CH_SUP, HI_T = (NH + G::NT - 1) / G::NT;  // header items
    uint4 hd[HI_T];
#pragma unroll
    for (int j = 0; j < HI_T; j++) {
      const uint32_t i = tid + j * G::NT, lr = i / G::CH_SUP, s = i % G::CH_SUP;
      if constexpr (PAIR) {  // rows [0, OUT) of the gate, then the same rows of up
        if (i < NH && s < ns)
          hd[j] = w[(lr >= (uint32_t)OUT ? p.u1 : p.o1) + min(row0 + lr % OUT, p.n_out - 1) * supers + s0 + s];
      } else {
        if (i < NH && s < ns) hd[j] = buf_load(wh, ((base + min(row0 + lr, p.n_out - 1)) * supers + s) * 16, s0 * 16);
      }
    }
    uint4 q[PF][ROWS];
#pragma unroll
    for (int j = 0; j < PF; j++)
#pragma unroll
      for (int r = 0; r < ROWS; r++) q[j][r] = buf_load(wq, voff[r], (u0 + j * LPR) * 16);

    // stage: item t = quarter t%4 of unit t/4 (values 0-7, 8-15 of the low-nibble half,
    // then of the high half); the pair sums of quarters make the unit's two 16-value sums
    float ssp = 0.0f;  // MODE 2: this pass's sum of x^2 (first staging only)
    auto stage_x = [&](float scale) -> float {
      float big = 0.0f;  // largest |x| staged
#pragma unroll
      for (int j = 0; j < XI; j++) {
        const uint32_t t = tid + j * G::NT, u = t >> 2, qq = t & 3;
        float4 a = xa[j][0], b = xa[j][1];
        if constexpr (AUX) {
          float sq = 0.0f;
          a = fuse4<MODE>(a, xu[j][0], sq);
          b = fuse4<MODE>(b, xu[j][1], sq);
          if (scale == 1.0f) ssp += sq;
        }
        big = fmaxf(big, fmaxf(abs_max4(a), abs_max4(b)));
        if (scale != 1.0f) {
          a = make_float4(a.x * scale, a.y * scale, a.z * scale, a.w * scale);
          b = make_float4(b.x * scale, b.y * scale, b.z * scale, b.w * scale);
        }
        const uint32_t h0 = pk(a.x, a.z), h1 = pk(a.y, a.w), h2 = pk(b.x, b.z), h3 = pk(b.y, b.w);
        const f16x2 one = {(f16)1.0f, (f16)1.0f};
        float sum = dot2(as_f16x2(h0), one, 0.0f);
        sum = dot2(as_f16x2(h1), one, sum);
        sum = dot2(as_f16x2(h2), one, sum);
        sum = dot2(as_f16x2(h3), one, sum);
        sum += dpp_f<0xb1>(sum);  // + the other quarter of the same half
        if (t < 4 * CHU) {
          xq[qq][u] = make_uint4(h0, h1, h2, h3);
          if ((qq & 1) == 0) ((float *)&xs[u])[qq >> 1] = sum;
        }
      }
      return big;
    };
    guard_note(wmax, stage_x(1.0f));
    norm_note<MODE, WAVES>(wss, ssp);
    // decode: the 8 six-bit scales and mins as bytes of four words (quant.rs:40-49)
#pragma unroll
    for (int j = 0; j < HI_T; j++) {
      const uint32_t i = tid + j * G::NT, lr = i / G::CH_SUP, s = i % G::CH_SUP;
      if (i < NH && s >= ns) {
#pragma unroll
        for (int cc = 0; cc < 4; cc++) sc[lr][s][cc] = make_float4(0.f, 0.f, 0.f, 0.f);
      } else if (i < NH) {
        const uint4 h = hd[j];
        const float d = f16_bits_to_f32(h.x & 0xffffu), dmin = f16_bits_to_f32(h.x >> 16);
        const float d16 = d * 0.0625f, d1024 = d * 1024.0f, d64 = d * 64.0f;
        const uint32_t sw[2] = {h.y & 0x3f3f3f3fu, (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u)};
        const uint32_t mw[2] = {h.z & 0x3f3f3f3fu, ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u)};
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
          const uint32_t sv = sw[cc >> 1] >> (16 * (cc & 1)), mv = mw[cc >> 1] >> (16 * (cc & 1));
          const float s_lo = (float)(sv & 255u), s_hi = (float)((sv >> 8) & 255u);
          const float m_lo = (float)(mv & 255u), m_hi = (float)((mv >> 8) & 255u);
          sc[lr][s][cc] = make_float4(d * s_lo, d16 * s_hi, __builtin_fmaf(d1024, s_lo, dmin * m_lo),
                                      __builtin_fmaf(d64, s_hi, dmin * m_hi));
        }
      }
    }
    __syncthreads();
    norm_take<MODE, WAVES>(wss, ss);
    const int e = guard_exp<WAVES>(wmax);
    if (e) {  // rare: the pass again at x * 2^-e
      load_x();
      stage_x(__builtin_ldexpf(1.0f, -e));
      __syncthreads();
      scale_rows(acc, -e);
    }

    const uint32_t S = (nu + LPR - 1) / LPR;
    auto step = [&](uint32_t st, const uint4 (&qj)[ROWS]) {
      const uint32_t i = lane + st * LPR;
      const uint4 xa0 = xq[0][i], xa1 = xq[1][i], xb0 = xq[2][i], xb1 = xq[3][i];
      const float2 xsum = xs[i];
      const uint32_t pa[8] = {xa0.x, xa0.y, xa0.z, xa0.w, xa1.x, xa1.y, xa1.z, xa1.w};
      const uint32_t pb[8] = {xb0.x, xb0.y, xb0.z, xb0.w, xb1.x, xb1.y, xb1.z, xb1.w};
      const uint32_t s = (lane >> 3) + st * (LPR / 8);
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        float sa = 0.0f, sb = 0.0f;
        const uint32_t wd[4] = {qj[r].x, qj[r].y, qj[r].z, qj[r].w};
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const uint32_t w0 = wd[k], w8 = w0 >> 8;
          sa = dot2(as_f16x2(and_or(w0, LO, MW)), as_f16x2(pa[2 * k]), sa);
          sa = dot2(as_f16x2(and_or(w8, LO, MW)), as_f16x2(pa[2 * k + 1]), sa);
          sb = dot2(as_f16x2(and_or(w0, HI, MW)), as_f16x2(pb[2 * k]), sb);
          sb = dot2(as_f16x2(and_or(w8, HI, MW)), as_f16x2(pb[2 * k + 1]), sb);
        }
        const float4 f = sc[hrow0 + r][s][c];
        acc[r] = __builtin_fmaf(f.x, sa, acc[r]);
        acc[r] = __builtin_fmaf(f.y, sb, acc[r]);
        acc[r] = __builtin_fmaf(-f.z, xsum.x, acc[r]);
        acc[r] = __builtin_fmaf(-f.w, xsum.y, acc[r]);
      }
    };
    uint32_t j0 = 0;
    for (; j0 + PF < S; j0 += PF) {
#pragma unroll
      for (int j = 0; j < PF; j++) {
        step(j0 + j, q[j]);
#pragma unroll
        for (int r = 0; r < ROWS; r++) q[j][r] = buf_load(wq, voff[r], (u0 + (j0 + j + PF) * LPR) * 16);
        __builtin_amdgcn_sched_barrier(0);  // each refill right behind the step it replaces
      }
    }
#pragma unroll
    for (int j = 0; j < PF; j++)
      if (j0 + j < S) step(j0 + j, q[j]);
    if (e) scale_rows(acc, e);
  }
  norm_apply<MODE>(acc, ss, p);
  if constexpr (PAIR) {
    float tot[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; r++) {
      tot[r] = lane_sum<LPR>(acc[r]);
      if (second && lane == 0) ush[lrow0 + r] = tot[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < ROWS; r++)
      if (!second && lane == 0 && first + r < p.n_out) {
#pragma clang fp contract(off)
        const float g = tot[r];
        y[y_off + first + r] = g / (1.0f + expf(-g)) * ush[lrow0 + r];  // silu_mul.comp:15-23
      }
  } else {
    store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc);
  }
}

// ---------------------------------------------------------------------------------------
// Q6_K.  Lane step = 64 values of one super-block: u -> super-block u/4, half hf = (u%4)/2,
// li = u%2.  It reads 16 B of ql at l = 16 li (a), 16 B at l + 32 (b) and 16 B of qh.
// Group g = 0..3 is values 128 hf + 32 g + 16 li + [0,16) with scale sc[8 hf + li + 2g]
// (quant.rs:72-87).  Groups 0,1 are built as 1024+q, groups 2,3 as 1024+16q (q the stored
// 6-bit value, quant = q - 32).
// LDS per pass: xq[unit] = 32 f16 pairs (4 groups x 8), xs[unit] = the 4 group sums, and per
// (row, super-block) and (hf, li): d*sc for the lane's 4 groups (1/16 folded into g = 2, 3).
// ---------------------------------------------------------------------------------------
template <int WAVES, int ACCUM, int ROWS, int MOE, int LPR, int MODE = 0, typename P = MatvecPush4>
SK_DEV void matvec_q6k_body(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd,
                            const float *x, float *y, const uint32_t *ids, const P &p,
                            uint32_t bx) {
  using G = Geo<WAVES, ROWS, LPR>;
  __shared__ uint4 xq[8][G::CH / 64];  // component-major
  __shared__ float4 xs[G::CH / 64];
  __shared__ float4 sc[G::RWG][G::CH_SUP][4];
  __shared__ uint32_t wmax[WAVES];
  __shared__ float wss[MODE == 2 ? 4 * WAVES : 1];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = (tid & 63) % LPR;
  const uint32_t sub = (tid & 63) / LPR;
  const uint32_t row0 = bx * G::RWG;
  const uint32_t lrow0 = ((tid >> 6) * G::SUBS + sub) * ROWS;
  const uint32_t first = row0 + lrow0;
  const uint32_t slot = blockIdx.y;
  const uint32_t base = MOE ? ids[p.ids_off + slot] * p.n_out : 0;
  const float *xv = x + p.x_off + slot * p.x_stride;
  const float *av = x;  // MODE != 0: the second vector, indexed as xv
  if constexpr (MODE != 0) av = x + p.aux_off + (MODE == 1 ? slot * p.x_stride : 0);
  float ss = 0.0f;
  const uint32_t y_off = p.y_off + slot * p.y_stride;
  const uint32_t supers = p.n_in >> 8;
  const uint32_t li = lane & 1, hf = (lane >> 1) & 1;
  const uint32_t MW = MAGIC, L4 = 0x000f000fu, H4 = 0x00f000f0u, LH = 0x00300030u, HH = 0x03000300u;

  uint32_t rb[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) rb[r] = (base + min(first + r, p.n_out - 1)) * supers;

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;

  for (uint32_t k0 = 0; k0 < p.n_in; k0 += G::CH) {
    const uint32_t nk = min(p.n_in - k0, (uint32_t)G::CH);
    const uint32_t u0 = k0 >> 6, nu = nk >> 6, s0 = k0 >> 8, ns = nk >> 8;
    constexpr int PF = 2;
    uint4 qa[PF][ROWS], qb[PF][ROWS], qh[PF][ROWS];
    auto load = [&](uint32_t i, uint4 (&a)[ROWS], uint4 (&b)[ROWS], uint4 (&h)[ROWS]) {
      const uint32_t u = u0 + i;
      const uint32_t s = u >> 2;
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        const uint32_t rs = rb[r] + s;
        a[r] = w[p.o0 + rs * 8 + hf * 4 + li];
        b[r] = w[p.o0 + rs * 8 + hf * 4 + 2 + li];
        h[r] = w[p.o1 + rs * 4 + hf * 2 + li];
      }
    };
    // activation item t = group t%4 of unit t/4: 16 values (4 x 16 B) that become 8 f16
    // pairs and one 16-value sum (16 VGPRs in flight per item, not a whole unit's 64)
    const uint32_t n_xi = 4 * nu;
    float4 xu4[MODE ? 4 : 1];
    auto x_item = [&](uint32_t t, float4 (&v)[4]) {
      const uint32_t u = u0 + (t >> 2), g = t & 3;
      const uint32_t at = (u >> 2) * 256 + ((u >> 1) & 1) * 128 + (u & 1) * 16 + 32 * g;
#pragma unroll
      for (int k = 0; k < 4; k++) v[k] = *(const float4 *)(xv + at + 4 * k);
      if constexpr (MODE != 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) xu4[k] = *(const float4 *)(av + at + 4 * k);
      }
    };
    float big = 0.0f;  // largest |x| this thread staged
    float ssp = 0.0f;  // MODE 2: this pass's sum of x^2 (first staging only)
    auto x_store = [&](uint32_t t, const float4 (&v)[4], float scale) {
      const uint32_t i = t >> 2, g = t & 3;
      const f16x2 one = {(f16)1.0f, (f16)1.0f};
      uint32_t pp[8];
      float s = 0.0f, sq = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        float4 f = v[k];
        if constexpr (MODE != 0) f = fuse4<MODE>(f, xu4[k], sq);
        big = fmaxf(big, abs_max4(f));
        const float4 e = scale != 1.0f ? make_float4(f.x * scale, f.y * scale, f.z * scale, f.w * scale) : f;
        pp[2 * k] = pk(e.x, e.z);
        pp[2 * k + 1] = pk(e.y, e.w);
        s = dot2(as_f16x2(pp[2 * k]), one, s);
        s = dot2(as_f16x2(pp[2 * k + 1]), one, s);
      }
      xq[2 * g][i] = make_uint4(pp[0], pp[1], pp[2], pp[3]);
      xq[2 * g + 1][i] = make_uint4(pp[4], pp[5], pp[6], pp[7]);
      ((float *)&xs[i])[g] = s;
      if (scale == 1.0f) ssp += sq;
    };
    const uint32_t n_items = (uint32_t)G::RWG * ns;
    auto h_load = [&](uint32_t i, uint4 &sv, uint32_t &dv) {
      const uint32_t lr = i / ns, s = i % ns;
      const uint32_t rs = (base + min(row0 + lr, p.n_out - 1)) * supers + s0 + s;
      sv = w[p.o2 + rs];
      dv = wd[p.o3 + rs];
    };
    auto h_store = [&](uint32_t i, const uint4 sv, uint32_t dv) {
      const uint32_t lr = i / ns, s = i % ns;
      const float d = f16_bits_to_f32(dv);
      const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
      for (int lp = 0; lp < 4; lp++) {  // (hf, li) = (lp / 2, lp % 2)
        float o[4];
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const uint32_t k = 8 * (lp >> 1) + (lp & 1) + 2 * g;
          const int s8 = (int)(int8_t)((sw[k >> 2] >> (8 * (k & 3))) & 255u);
          o[g] = d * (float)s8 * (g >= 2 ? 0.0625f : 1.0f);
        }
        sc[lr][s][lp] = make_float4(o[0], o[1], o[2], o[3]);
      }
    };
    if (k0 != 0) __syncthreads();
    float4 xv4[4];
    uint4 sv0 = make_uint4(0, 0, 0, 0);
    uint32_t dv0 = 0;
    if (tid < n_xi) x_item(tid, xv4);
    if (tid < n_items) h_load(tid, sv0, dv0);
#pragma unroll
    for (int j = 0; j < PF; j++) load(min(lane + j * LPR, nu - 1), qa[j], qb[j], qh[j]);
    if (tid < n_xi) x_store(tid, xv4, 1.0f);
    if (tid < n_items) h_store(tid, sv0, dv0);
    for (uint32_t t = tid + G::NT; t < n_xi; t += G::NT) {
      x_item(t, xv4);
      x_store(t, xv4, 1.0f);
    }
    for (uint32_t i = tid + G::NT; i < n_items; i += G::NT) {
      h_load(i, sv0, dv0);
      h_store(i, sv0, dv0);
    }
    guard_note(wmax, big);
    norm_note<MODE, WAVES>(wss, ssp);
    __syncthreads();
    norm_take<MODE, WAVES>(wss, ss);
    const int e = guard_exp<WAVES>(wmax);
    if (e) {  // rare: the pass again at x * 2^-e
      for (uint32_t t = tid; t < n_xi; t += G::NT) {
        x_item(t, xv4);
        x_store(t, xv4, __builtin_ldexpf(1.0f, -e));
      }
      __syncthreads();
      scale_rows(acc, -e);
    }

    for (uint32_t j0 = 0; lane + j0 * LPR < nu; j0 += PF) {
#pragma unroll
      for (int j = 0; j < PF; j++) {
        const uint32_t i = lane + (j0 + j) * LPR;
        if (i < nu) {
          const float4 xsum = xs[i];
          const float ib[4] = {-1056.0f * xsum.x, -1056.0f * xsum.y, -1536.0f * xsum.z, -1536.0f * xsum.w};
          const uint32_t s = i >> 2;
#pragma unroll
          for (int r = 0; r < ROWS; r++) {
            float t[4];
            // group g: quants from ql half a (g even) or b (g odd), low nibbles for g < 2 and
            // high for g >= 2; qh bits 2g, 2g+1 land on bits 4-5 (g < 2) or 8-9 of each lane.
            // One group's operands are live at a time (157 -> 108 VGPRs).
#pragma unroll
            for (int g = 0; g < 4; g++) {
              const uint4 x0 = xq[2 * g][i], x1 = xq[2 * g + 1][i];
              const uint32_t px[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
              const uint4 qv = (g & 1) ? qb[j][r] : qa[j][r];
              const uint32_t wv[4] = {qv.x, qv.y, qv.z, qv.w};
              const uint32_t hv[4] = {qh[j][r].x, qh[j][r].y, qh[j][r].z, qh[j][r].w};
              const uint32_t QM = g < 2 ? L4 : H4, HM = g < 2 ? LH : HH, SH = (g & 1) ? 2 : 4;
              float tg = ib[g];
#pragma unroll
              for (int k = 0; k < 4; k++) {
                const uint32_t w0 = wv[k], w8 = w0 >> 8, h0 = hv[k] << SH, h8 = (hv[k] >> 8) << SH;
                tg = dot2(as_f16x2(and_or(h0, HM, and_or(w0, QM, MW))), as_f16x2(px[2 * k]), tg);
                tg = dot2(as_f16x2(and_or(h8, HM, and_or(w8, QM, MW))), as_f16x2(px[2 * k + 1]), tg);
              }
              t[g] = tg;
              __builtin_amdgcn_sched_barrier(0);
            }
            const float4 f = sc[lrow0 + r][s][hf * 2 + li];
            acc[r] = __builtin_fmaf(f.x, t[0], acc[r]);
            acc[r] = __builtin_fmaf(f.y, t[1], acc[r]);
            acc[r] = __builtin_fmaf(f.z, t[2], acc[r]);
            acc[r] = __builtin_fmaf(f.w, t[3], acc[r]);
          }
        }
        load(min(i + PF * LPR, nu - 1), qa[j], qb[j], qh[j]);  // unconditional, as in Q4_K
        __builtin_amdgcn_sched_barrier(0);  // each refill right behind the step it replaces
      }
    }
    if (e) scale_rows(acc, e);
  }
  norm_apply<MODE>(acc, ss, p);
  store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc);
}

// ---------------------------------------------------------------------------------------
// Q8_0.  Lane step = 16 quants (half a block) of one row; the block scale d is staged per
// (row, block) as f32.  q as f16: (q ^ 0x80) is 0..255, so MAGIC | that = 1152 + q.
// LDS per pass: xq[unit] = 8 f16 pairs, xs[unit] = their sum, dd[row][block] = d.
// ---------------------------------------------------------------------------------------
template <int WAVES, int ACCUM, int ROWS, int MOE, int LPR, int MODE = 0, typename P = MatvecPush2>
SK_DEV void matvec_q8_0_body(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd,
                             const float *x, float *y, const uint32_t *ids, const P &p,
                             uint32_t bx) {
  using G = Geo<WAVES, ROWS, LPR>;
  constexpr int NBLK = G::CH / 32;
  __shared__ uint4 xq[2][G::CH / 16];  // component-major
  __shared__ float xs[G::CH / 16];
  __shared__ float dd[G::RWG][NBLK];
  __shared__ uint32_t wmax[WAVES];
  __shared__ float wss[MODE == 2 ? 4 * WAVES : 1];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = (tid & 63) % LPR;
  const uint32_t sub = (tid & 63) / LPR;
  const uint32_t row0 = bx * G::RWG;
  const uint32_t lrow0 = ((tid >> 6) * G::SUBS + sub) * ROWS;
  const uint32_t first = row0 + lrow0;
  const uint32_t slot = blockIdx.y;
  const uint32_t base = MOE ? ids[p.ids_off + slot] * p.n_out : 0;
  const float *xv = x + p.x_off + slot * p.x_stride;
  const float *av = x;  // MODE != 0: the second vector, indexed as xv
  if constexpr (MODE != 0) av = x + p.aux_off + (MODE == 1 ? slot * p.x_stride : 0);
  float ss = 0.0f;
  const uint32_t y_off = p.y_off + slot * p.y_stride;
  const uint32_t chunks = p.n_in >> 4, blocks = p.n_in >> 5;
  const uint32_t MW = MAGIC, M8 = 0x00ff00ffu;

  const uint4 *qr[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) qr[r] = w + p.o0 + (base + min(first + r, p.n_out - 1)) * chunks;

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;

  for (uint32_t k0 = 0; k0 < p.n_in; k0 += G::CH) {
    const uint32_t nk = min(p.n_in - k0, (uint32_t)G::CH);
    const uint32_t u0 = k0 >> 4, nu = nk >> 4, b0 = k0 >> 5, nb = nk >> 5;
    float4 xu4[MODE ? 4 : 1];
    auto x_unit = [&](uint32_t i, float4 (&v)[4]) {
      const uint32_t at = (u0 + i) * 16;
#pragma unroll
      for (int k = 0; k < 4; k++) v[k] = *(const float4 *)(xv + at + 4 * k);
      if constexpr (MODE != 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) xu4[k] = *(const float4 *)(av + at + 4 * k);
      }
    };
    float big = 0.0f;  // largest |x| this thread staged
    float ssp = 0.0f;  // MODE 2: this pass's sum of x^2 (first staging only)
    auto x_store = [&](uint32_t i, const float4 (&v)[4], float scale) {
      uint32_t pp[8];
      const f16x2 one = {(f16)1.0f, (f16)1.0f};
      float s = 0.0f, sq = 0.0f;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        float4 f = v[k];
        if constexpr (MODE != 0) f = fuse4<MODE>(f, xu4[k], sq);
        big = fmaxf(big, abs_max4(f));
        const float4 e = scale != 1.0f ? make_float4(f.x * scale, f.y * scale, f.z * scale, f.w * scale) : f;
        pp[2 * k] = pk(e.x, e.z);
        pp[2 * k + 1] = pk(e.y, e.w);
        s = dot2(as_f16x2(pp[2 * k]), one, s);
        s = dot2(as_f16x2(pp[2 * k + 1]), one, s);
      }
      xq[0][i] = make_uint4(pp[0], pp[1], pp[2], pp[3]);
      xq[1][i] = make_uint4(pp[4], pp[5], pp[6], pp[7]);
      xs[i] = s;
      if (scale == 1.0f) ssp += sq;
    };
    const uint32_t n_items = (uint32_t)G::RWG * nb;
    auto d_load = [&](uint32_t i) -> uint32_t {
      const uint32_t lr = i / nb, bl = i % nb;
      const uint32_t row = base + min(row0 + lr, p.n_out - 1);
      return wd[p.o1 + row * blocks + b0 + bl];
    };
    if (k0 != 0) __syncthreads();
    float4 xv4[4];
    uint32_t dv0 = 0;
    if (tid < nu) x_unit(tid, xv4);
    if (tid < n_items) dv0 = d_load(tid);
    constexpr int PF = 4;  // unconditional loads, as in Q4_K
    uint4 q[PF][ROWS];
#pragma unroll
    for (int j = 0; j < PF; j++) {
      const uint32_t i = min(lane + j * LPR, nu - 1);
#pragma unroll
      for (int r = 0; r < ROWS; r++) q[j][r] = qr[r][u0 + i];
    }
    if (tid < nu) x_store(tid, xv4, 1.0f);
    if (tid < n_items) dd[tid / nb][tid % nb] = f16_bits_to_f32(dv0);
    for (uint32_t i = tid + G::NT; i < nu; i += G::NT) {
      x_unit(i, xv4);
      x_store(i, xv4, 1.0f);
    }
    for (uint32_t i = tid + G::NT; i < n_items; i += G::NT) dd[i / nb][i % nb] = f16_bits_to_f32(d_load(i));
    guard_note(wmax, big);
    norm_note<MODE, WAVES>(wss, ssp);
    __syncthreads();
    norm_take<MODE, WAVES>(wss, ss);
    const int e = guard_exp<WAVES>(wmax);
    if (e) {  // rare: the pass again at x * 2^-e
      for (uint32_t i = tid; i < nu; i += G::NT) {
        x_unit(i, xv4);
        x_store(i, xv4, __builtin_ldexpf(1.0f, -e));
      }
      __syncthreads();
      scale_rows(acc, -e);
    }

    for (uint32_t j0 = 0; lane + j0 * LPR < nu; j0 += PF) {
#pragma unroll
      for (int j = 0; j < PF; j++) {
        const uint32_t i = lane + (j0 + j) * LPR;
        if (i < nu) {
          const uint4 x0 = xq[0][i], x1 = xq[1][i];
          const uint32_t px[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
          const float bias = -1152.0f * xs[i];
#pragma unroll
          for (int r = 0; r < ROWS; r++) {
            float s = bias;
            const uint32_t wv[4] = {q[j][r].x, q[j][r].y, q[j][r].z, q[j][r].w};
#pragma unroll
            for (int k = 0; k < 4; k++) {
              const uint32_t b = wv[k] ^ 0x80808080u;
              s = dot2(as_f16x2(and_or(b, M8, MW)), as_f16x2(px[2 * k]), s);
              s = dot2(as_f16x2(and_or(b >> 8, M8, MW)), as_f16x2(px[2 * k + 1]), s);
            }
            acc[r] = __builtin_fmaf(dd[lrow0 + r][i >> 1], s, acc[r]);
          }
        }
        const uint32_t inext = min(i + PF * LPR, nu - 1);
#pragma unroll
        for (int r = 0; r < ROWS; r++) q[j][r] = qr[r][u0 + inext];
      }
    }
    if (e) scale_rows(acc, e);
  }
  norm_apply<MODE>(acc, ss, p);
  store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc);
}

}  // namespace

// ---------------------------------------------------------------------------------------
// Exported instantiations: symbol = <shader name>__<spec words joined by '_'>.  Each takes
// the push words as a segment table (Segments, common.h), which the runtime builds.
// ---------------------------------------------------------------------------------------
// Waves per SIMD the Q4_K kernels are register-budgeted for: eight-wave workgroups keep
// three per CU (the LDS allows three), which caps them at 80 VGPRs.
#define MV_Q4K_WPE(W, R) ((W) >= 8 && (R) == 1 ? 6 : 1)
#define MV_Q4K(W, A, R, M, L)                                                                \
  extern "C" __global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(MV_Q4K_WPE(W, R)))) \
  void matvec_q4k__##W##_##A##_##R##_##M##_##L(                                                \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPush2> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    matvec_q4k_body<W, A, R, M, L>(w, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
#define MV_Q6K(W, A, R, M, L)                                                                \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q6k__##W##_##A##_##R##_##M##_##L( \
      const uint4 *w, const uint16_t *wd, const float *x, float *y, const uint32_t *ids,     \
      Segments<MatvecPush4> m) {                                                             \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    matvec_q6k_body<W, A, R, M, L>(w, wd, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
#define MV_Q8_0(W, A, R, M, L)                                                                \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q8_0__##W##_##A##_##R##_##M##_##L( \
      const uint4 *w, const uint16_t *wd, const float *x, float *y, const uint32_t *ids,      \
      Segments<MatvecPush2> m) {                                                              \
    const uint32_t s = segment_of(m, blockIdx.x);                                             \
    matvec_q8_0_body<W, A, R, M, L>(w, wd, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]); \
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

// Fused forms (MODE 1 = SiLU of the gate rows times the up rows, the down projection;
// MODE 2 = RMSNorm, the projections that read a normed residual), dense rows only.
#define MV_Q4K_F(SUF, MODE, W, A, R, L)                                                       \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q4k_##SUF##__##W##_##A##_##R##_0_##L(                                            \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPush2F> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    matvec_q4k_body<W, A, R, 0, L, MODE>(w, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
#define MV_Q6K_F(SUF, MODE, W, A, R, L)                                                       \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q6k_##SUF##__##W##_##A##_##R##_0_##L( \
      const uint4 *w, const uint16_t *wd, const float *x, float *y, const uint32_t *ids,     \
      Segments<MatvecPush4F> m) {                                                            \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    matvec_q6k_body<W, A, R, 0, L, MODE>(w, wd, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
#define MV_Q8_0_F(SUF, MODE, W, A, R, L)                                                      \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q8_0_##SUF##__##W##_##A##_##R##_0_##L( \
      const uint4 *w, const uint16_t *wd, const float *x, float *y, const uint32_t *ids,     \
      Segments<MatvecPush2F> m) {                                                            \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    matvec_q8_0_body<W, A, R, 0, L, MODE>(w, wd, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
// the engine's default tactic (4 waves, 2 rows, 64 lanes) and the runtime's size variants;
// the norm forms write (ACCUM 0: q, k, v, gate, up, the head), the SiLU forms accumulate
// (the down projection adds into the residual)
MV_Q4K_F(norm, 2, 4, 0, 2, 64)
MV_Q4K_F(norm, 2, 8, 0, 1, 16)
MV_Q4K_F(norm, 2, 8, 0, 1, 64)
MV_Q4K_F(silu, 1, 4, 1, 2, 64)
MV_Q4K_F(silu, 1, 8, 1, 1, 16)
MV_Q4K_F(silu, 1, 8, 1, 1, 64)
MV_Q6K_F(norm, 2, 4, 0, 2, 64)
MV_Q6K_F(norm, 2, 4, 0, 1, 16)
MV_Q6K_F(norm, 2, 8, 0, 1, 32)
MV_Q6K_F(silu, 1, 4, 1, 2, 64)
MV_Q6K_F(silu, 1, 4, 1, 1, 16)
MV_Q6K_F(silu, 1, 8, 1, 1, 32)
MV_Q8_0_F(norm, 2, 4, 0, 2, 64)
MV_Q8_0_F(silu, 1, 4, 1, 2, 64)
// gate and up of a decode token in one launch, writing silu(gate) * up (MODE 3): half the
// waves take gate rows, half the same rows of up, so a workgroup outputs RWG / 2 values
#define MV_Q4K_GLU(W, R, L)                                                                    \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q4k_glu__##W##_0_##R##_0_##L(      \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPushGlu> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    matvec_q4k_body<W, 0, R, 0, L, 3>(w, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
MV_Q4K_GLU(8, 1, 16)
MV_Q4K_GLU(8, 1, 64)
// the same with the FFN RMSNorm folded in (MODE 4): x is the raw residual
#define MV_Q4K_GLUN(W, R, L)                                                                   \
  extern "C" __global__ __launch_bounds__(64 * W) void matvec_q4k_glun__##W##_0_##R##_0_##L(     \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPushGluN> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    matvec_q4k_body<W, 0, R, 0, L, 4>(w, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
MV_Q4K_GLUN(8, 1, 16)

// Dense variants with fewer lanes per row (more pipelined steps per lane) that the runtime
// picks for large launches (skyla_hip.cpp, choose_variant).
MV_Q4K(8, 0, 1, 0, 16)
MV_Q4K(8, 1, 1, 0, 16)
MV_Q6K(4, 0, 1, 0, 32)
MV_Q6K(4, 1, 1, 0, 32)
MV_Q6K(8, 0, 1, 0, 32)
MV_Q6K(8, 1, 1, 0, 32)
MV_Q6K(4, 0, 1, 0, 16)
MV_Q6K(4, 1, 1, 0, 16)
