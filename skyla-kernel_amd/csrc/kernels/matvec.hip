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
//   * Activations are staged once per workgroup in LDS as f32, in the order the packed
//     quants need them, with their per-16 sums, instead of every wave re-reading x
//     through L1.
//   * Each (row, super-block) header is decoded once per workgroup into f32 products
//     d*sc and dmin*m (the reference's d0 / min0, quant.rs:60-61), so a lane's per-row work
//     is the quant extraction, one FMA per value and four FMAs per unit.
//   * Arithmetic is the reference's: f32 activations times exact integer quants in f32
//     (matvec_q4k.comp:84-100).  Four quants sit in the bytes of a masked word and
//     v_cvt_f32_ubyte0..3 turns each into an exact f32; high nibbles are taken in place as
//     16q (no shift) and their scale carries the 1/16.  Each lane sums value * quant in
//     f32 FMAs, so the result differs from the reference's f32 dot only in summation order.
//   * Weight loads are 16 B per lane, 1 KiB contiguous per wave instruction, and the first
//     step's loads are issued before the staging so they overlap it.
#include "common.h"
#include "route.h"

namespace {

struct MatvecPush2 {  // Q4_K and Q8_0 (9 words, graph.rs:30 / graph/moe.rs:8-24)
  uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride;
};

struct MatvecPush4 {  // Q6_K (11 words, graph.rs:29 / graph/moe.rs:8-24)
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
// matvec_q4k_glur: matvec_q4k_glu's words, then moe_route's (16 words)
struct MatvecPushGluR {
  MatvecPushGlu g;
  RoutePush r;
};
// matvec_q4k_glun: matvec_q4k_glu's words, then the norm weights and eps (13 words)
struct MatvecPushGluN {
  uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride, u0, u1, aux_off;
  float eps;
};
// matvec_q4k_ecomb: an expert matvec's words, then moe_combine's residual offset, routing
// weights offset and experts per token (12 words)
struct MatvecPushComb {
  uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride, res_off, w_off, n_used;
};
struct MatvecPush4F {
  uint32_t o0, o1, o2, o3, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride, aux_off;
  float eps;
};

// The old outputs of an accumulating launch (lane 0 of each row group, the lane that stores
// them), read at entry next to the first loads: the store at the end then adds without
// waiting for a load (the same y + total).
template <int ACCUM, int ROWS>
SK_DEV void load_old(const float *y, uint32_t y_off, uint32_t first, uint32_t n_out, uint32_t lane,
                     float (&old)[ROWS]) {
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    old[r] = 0.0f;
    if (ACCUM && lane == 0 && first + r < n_out) old[r] = y[y_off + first + r];
  }
}

template <int ACCUM, int ROWS, int LPR>
SK_DEV void store_rows(float *y, uint32_t y_off, uint32_t first, uint32_t n_out, uint32_t lane,
                       const float (&acc)[ROWS], const float (&old)[ROWS]) {
#pragma unroll
  for (int r = 0; r < ROWS; r++) {
    const float total = lane_sum<LPR>(acc[r]);
    const uint32_t row = first + r;
    if (lane == 0 && row < n_out) {
      if (ACCUM)
        y[y_off + row] = old[r] + total;
      else
        y[y_off + row] = total;
    }
  }
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

// ---------------------------------------------------------------------------------------
// Q4_K.  Lane step = one 16 B unit of qs: unit u of a row is super-block u/8, chunk
// c = (u/2)%4, bytes 16(u%2) + [0,16) of that chunk's 32 -- low nibbles are values
// 64c + 16(u%2) + [0,16) of sub-block 2c, high nibbles the same positions of sub-block 2c+1
// (quant.rs:56-66).  LDS per pass: xf[0..3][unit] = the 16 activations of the low-nibble
// values, xf[4..7][unit] those of the high nibbles (f32, 4 per component), xs[unit] = their
// two 16-value sums, and per (row, super-block, chunk) four products of the header
// (quant.rs:40-49, 60-61): d*sc_lo, d*sc_hi/16, dmin*m_lo and dmin*m_hi.  A unit adds
//   d*sc_lo * sum(q_lo x) + d*sc_hi/16 * sum(16 q_hi x) - dmin*m_lo * sum(x_lo) - dmin*m_hi * sum(x_hi)
// which is the reference's sum of ((d sc) q - dmin m) x regrouped.
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
  __shared__ float4 xf[8][CHU];  // component-major: lanes read consecutive 16 B
  __shared__ float2 xs[CHU];
  __shared__ float4 sc[G::RWG][G::CH_SUP][4];
  __shared__ float wss[MODE == 2 || MODE == 4 ? 4 * WAVES : 1];
  // MODE 3 (gate and up in one launch): the first half of the waves computes gate rows,
  // the second half the up rows of the same outputs, and the store writes silu(g) * u.
  // MODE 4: MODE 3 with the FFN RMSNorm folded in as MODE 2 folds it (x * w staged, r
  // applied to the gate and up sums before the SiLU).
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
  const uint32_t LO4 = opaque_mask(0x0f0f0f0fu), HI4 = opaque_mask(0xf0f0f0f0u);

  uint32_t mo0 = p.o0, mo1 = p.o1;  // this wave's matrix
  if constexpr (PAIR) {
    mo0 = __builtin_amdgcn_readfirstlane(second ? p.u0 : p.o0);
    mo1 = __builtin_amdgcn_readfirstlane(second ? p.u1 : p.o1);
  }
  (void)mo1;
  const BufRes wq = buf_res(w + mo0, (uint64_t)(base + p.n_out) * units * 16);
  const BufRes wh = buf_res(w + p.o1, (uint64_t)(base + p.n_out) * supers * 16);
  uint32_t voff[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) voff[r] = ((base + min(first + r, p.n_out - 1)) * units + lane) * 16;

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;
  float yold[ROWS];
  load_old<ACCUM, ROWS>(y, y_off, first, p.n_out, lane, yold);

  for (uint32_t k0 = 0; k0 < p.n_in; k0 += CHU * 32) {
    const uint32_t nk = min(p.n_in - k0, (uint32_t)CHU * 32);
    const uint32_t u0 = k0 >> 5, nu = nk >> 5, s0 = k0 >> 8, ns = nk >> 8;
    if (k0 != 0) __syncthreads();  // the previous pass is done with the LDS
    // Load order matters (a wave's loads complete in issue order): activations, then
    // headers, then the first PF weight steps, so staging waits only for its own data.
    constexpr int XI = (4 * CHU + G::NT - 1) / G::NT;  // activation quarters per thread
    float4 xa[XI][2], xu[AUX ? XI : 1][2];
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
    constexpr int NH = G::RWG * G::CH_SUP, HI_T = (NH + G::NT - 1) / G::NT;  // header items
    uint4 hd[HI_T];
#pragma unroll
    for (int j = 0; j < HI_T; j++) {
      const uint32_t i = tid + j * G::NT, lr = i / G::CH_SUP, s = i % G::CH_SUP;
      if constexpr (PAIR) {  // rows [0, OUT) of the gate, then the same rows of up
        if (i < NH && s < ns)
          hd[j] = load_nt(w + (lr >= (uint32_t)OUT ? p.u1 : p.o1) + (base + min(row0 + lr % OUT, p.n_out - 1)) * supers + s0 + s);
      } else {
        if (i < NH && s < ns) hd[j] = buf_load_nt(wh, ((base + min(row0 + lr, p.n_out - 1)) * supers + s) * 16, s0 * 16);
      }
    }
    uint4 q[PF][ROWS];
#pragma unroll
    for (int j = 0; j < PF; j++)
#pragma unroll
      for (int r = 0; r < ROWS; r++) q[j][r] = buf_load_nt(wq, voff[r], (u0 + j * LPR) * 16);

    // stage: item t = quarter t%4 of unit t/4 (values 0-7, 8-15 of the low-nibble half,
    // then of the high half); the pair sums of quarters make the unit's two 16-value sums
    float ssp = 0.0f;  // MODE 2: this pass's sum of x^2
#pragma unroll
    for (int j = 0; j < XI; j++) {
      const uint32_t t = tid + j * G::NT, u = t >> 2, qq = t & 3;
      float4 a = xa[j][0], b = xa[j][1];
      if constexpr (AUX) {
        a = fuse4<MODE>(a, xu[j][0], ssp);
        b = fuse4<MODE>(b, xu[j][1], ssp);
      }
      float sum = sum4(a) + sum4(b);
      sum += dpp_f<0xb1>(sum);  // + the other quarter of the same half
      if (t < 4 * CHU) {
        xf[(qq >> 1) * 4 + (qq & 1) * 2][u] = a;
        xf[(qq >> 1) * 4 + (qq & 1) * 2 + 1][u] = b;
        if ((qq & 1) == 0) ((float *)&xs[u])[qq >> 1] = sum;
      }
    }
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
        const float d16 = d * 0.0625f;
        const uint32_t sw[2] = {h.y & 0x3f3f3f3fu, (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u)};
        const uint32_t mw[2] = {h.z & 0x3f3f3f3fu, ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u)};
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
          const uint32_t sv = sw[cc >> 1] >> (16 * (cc & 1)), mv = mw[cc >> 1] >> (16 * (cc & 1));
          const float s_lo = (float)(sv & 255u), s_hi = (float)((sv >> 8) & 255u);
          const float m_lo = (float)(mv & 255u), m_hi = (float)((mv >> 8) & 255u);
          sc[lr][s][cc] = make_float4(d * s_lo, d16 * s_hi, dmin * m_lo, dmin * m_hi);
        }
      }
    }
    __syncthreads();
    norm_take<MODE, WAVES>(wss, ss);

    const uint32_t S = (nu + LPR - 1) / LPR;
    auto step = [&](uint32_t st, const uint4 (&qj)[ROWS]) {
      const uint32_t i = lane + st * LPR;
      const uint32_t s = (lane >> 3) + st * (LPR / 8);
      float sa[ROWS], sb[ROWS];
      {
        const float4 xl[4] = {xf[0][i], xf[1][i], xf[2][i], xf[3][i]};
#pragma unroll
        for (int r = 0; r < ROWS; r++) sa[r] = fma_bytes16(qj[r], LO4, xl, 0.0f);
      }
      {
        const float4 xh[4] = {xf[4][i], xf[5][i], xf[6][i], xf[7][i]};
#pragma unroll
        for (int r = 0; r < ROWS; r++) sb[r] = fma_bytes16(qj[r], HI4, xh, 0.0f);
      }
      const float2 xsum = xs[i];
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        const float4 f = sc[hrow0 + r][s][c];
        acc[r] = __builtin_fmaf(f.x, sa[r], acc[r]);
        acc[r] = __builtin_fmaf(f.y, sb[r], acc[r]);
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
        for (int r = 0; r < ROWS; r++) q[j][r] = buf_load_nt(wq, voff[r], (u0 + (j0 + j + PF) * LPR) * 16);
        __builtin_amdgcn_sched_barrier(0);  // each refill right behind the step it replaces
      }
    }
#pragma unroll
    for (int j = 0; j < PF; j++)
      if (j0 + j < S) step(j0 + j, q[j]);
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
    store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc, yold);
  }
}

// ---------------------------------------------------------------------------------------
// Q4_K, K-split form for n_in = 4096 KU (KU = 1: the Qwen3-8B q, k, v, o, gate and up rows;
// KU = 3: the 12288-wide down rows).  The workgroup's eight waves split every row it owns
// by super-blocks: wave w takes units 16w .. 16w+15 (super-blocks 2w, 2w+1) of each
// 4096-value part k < KU of the row, lane l the unit 16w + l%16 of the rows of its slot
// l/16.  A lane's 32 KU activations are therefore the same for every row it touches: they
// are loaded once, into registers, with their two 16-value sums per part, and no
// activation goes through LDS.  A row-group is 4 slots x RPL rows; its weights (KU 16 B
// units per lane and row) and headers (16 B per row and super-block) are loaded one group
// ahead of the arithmetic.  Each wave decodes its own headers into the products d*sc_lo,
// d*sc_hi/16, dmin*m_lo and dmin*m_hi (quant.rs:40-49, 60-61) in a region of LDS that only
// it touches, so no workgroup barrier is needed there; a lane's sum over its KU units is
// reduced over its 16 lanes with DPP, and the eight waves' partial rows meet in LDS once,
// at the end, added in wave order.
// MODE 2 (RMSNorm folded in: x * w in the registers, the totals scaled by r) and MODE 3
// (gate and up of the same outputs in one launch: slots 0, 1 take gate rows, 2, 3 the same
// rows of up, and the store writes silu(gate) * up) as in the forms above (KU = 1).
// ---------------------------------------------------------------------------------------
template <int ACCUM, int RPL, int NG, int MODE = 0, typename P = MatvecPush2, int KU = 1>
SK_DEV void matvec_q4k_ks_body(const uint4 *__restrict__ w, const float *x, float *y, const P &p,
                               uint32_t bx) {
  constexpr bool PAIR = MODE == 3 || MODE == 4, NORM = MODE == 2 || MODE == 4;
  constexpr int RG = 4 * RPL;             // rows per row-group
  constexpr int OG = PAIR ? RG / 2 : RG;  // outputs per row-group
  constexpr int OUT = OG * NG;            // outputs per workgroup
  constexpr int CPL = RG / 8;             // header chunks each lane decodes per row-group and part
  constexpr uint32_t SUP = 16 * KU, UNITS = 128 * KU;  // super-blocks and 16 B units per row
  static_assert(RG % 8 == 0 && CPL >= 1 && CPL <= 4, "two headers per row, 64 lanes");
  static_assert(KU == 1 || MODE == 0, "the fused forms are compiled for n_in 4096");
  __shared__ float4 hp[8][RG][2 * KU][4];  // per wave: row, (part, super-block), chunk
  __shared__ float part[8][RG * NG];
  __shared__ float wss[NORM ? 8 : 1];

  const uint32_t tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
  const uint32_t ul = l & 15, slot = l >> 4;
  const uint32_t unit = wv * 16 + ul;  // of each part's 128
  const uint32_t sbl = ul >> 3;        // the unit's super-block is 2 wv + sbl (of its part)
  const uint32_t c = (unit >> 1) & 3;  // its chunk
  const uint32_t LO4 = opaque_mask(0x0f0f0f0fu), HI4 = opaque_mask(0xf0f0f0f0u);
  const uint32_t out0 = bx * OUT;

  // row (clamped) and matrix regions of (group g, slot s, row r of the slot)
  auto row_of = [&](uint32_t g, uint32_t s, uint32_t r) -> uint32_t {
    const uint32_t o = out0 + g * OG + (PAIR ? (s & 1) : s) * RPL + r;
    return min(o, p.n_out - 1);
  };
  auto regions = [&](uint32_t s, uint32_t &q_off, uint32_t &h_off) {
    q_off = p.o0;
    h_off = p.o1;
    if constexpr (PAIR) {
      if (s >= 2) {
        q_off = p.u0;
        h_off = p.u1;
      }
    }
  };
  uint32_t qo, ho;
  regions(slot, qo, ho);
  // the header this lane decodes: h = (l * CPL) / 4, chunks (l * CPL) % 4 + [0, CPL)
  const uint32_t hh = (l * CPL) >> 2, hc0 = (l * CPL) & 3;
  const uint32_t h_rl = hh >> 1, h_sb = hh & 1;  // its row of the group and super-block
  uint32_t hqo, hho;
  regions(h_rl / RPL, hqo, hho);
  (void)hqo;

  auto load_group = [&](uint32_t g, uint4 (&q)[RPL][KU], uint4 (&h)[KU]) {
    const size_t hrow = (size_t)row_of(g, h_rl / RPL, h_rl % RPL) * SUP + 2 * wv + h_sb;
#pragma unroll
    for (int k = 0; k < KU; k++) h[k] = load_nt(w + hho + hrow + 16 * k);
#pragma unroll
    for (int r = 0; r < RPL; r++) {
      const size_t qrow = (size_t)row_of(g, slot, r) * UNITS + unit;
#pragma unroll
      for (int k = 0; k < KU; k++) q[r][k] = load_nt(w + qo + qrow + 128 * k);
    }
  };

  // activations first: they are what every row waits on
  const uint32_t at = (unit >> 3) * 256 + c * 64 + (unit & 1) * 16;
  const float *xv = x + p.x_off;
  float4 xl[KU][4], xh[KU][4];
#pragma unroll
  for (int k = 0; k < KU; k++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      xl[k][j] = *(const float4 *)(xv + at + 4096 * k + 4 * j);
      xh[k][j] = *(const float4 *)(xv + at + 4096 * k + 32 + 4 * j);
    }
  uint4 qc[RPL][KU], hc[KU];
  load_group(0, qc, hc);
  // an accumulating launch reads its old outputs now, so the store at the end waits for none
  float yold = 0.0f;
  if constexpr (ACCUM && !PAIR)
    if (tid < (uint32_t)OUT && out0 + tid < p.n_out) yold = y[p.y_off + out0 + tid];
  if constexpr (NORM) {  // x * w (the norm weights sit at aux_off), and sum(x^2)
    const float *wn = x + p.aux_off;
    float sq = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float4 a = *(const float4 *)(wn + at + 4 * j), b = *(const float4 *)(wn + at + 32 + 4 * j);
      xl[0][j] = fuse4<2>(xl[0][j], a, sq);
      xh[0][j] = fuse4<2>(xh[0][j], b, sq);
    }
    sq = lane_sum<16>(slot == 0 ? sq : 0.0f);  // each value once: slot 0's lanes
    if (l == 0) wss[wv] = sq;
  }
  float sl[KU], sh[KU];
#pragma unroll
  for (int k = 0; k < KU; k++) {
    sl[k] = (sum4(xl[k][0]) + sum4(xl[k][1])) + (sum4(xl[k][2]) + sum4(xl[k][3]));
    sh[k] = (sum4(xh[k][0]) + sum4(xh[k][1])) + (sum4(xh[k][2]) + sum4(xh[k][3]));
  }

#pragma unroll
  for (int g = 0; g < NG; g++) {
    uint4 qn[RPL][KU], hn[KU];
    if (g + 1 < NG) load_group(g + 1, qn, hn);
    // decode this group's headers into the wave's products
#pragma unroll
    for (int k = 0; k < KU; k++) {
      const uint4 hk = hc[k];
      const float d = f16_bits_to_f32(hk.x & 0xffffu), dmin = f16_bits_to_f32(hk.x >> 16);
      const float d16 = d * 0.0625f;
      const uint32_t sw[2] = {hk.y & 0x3f3f3f3fu, (hk.w & 0x0f0f0f0fu) | ((hk.y >> 2) & 0x30303030u)};
      const uint32_t mw[2] = {hk.z & 0x3f3f3f3fu, ((hk.w >> 4) & 0x0f0f0f0fu) | ((hk.z >> 2) & 0x30303030u)};
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        const uint32_t cc = hc0 + i;
        const uint32_t sv = (cc < 2 ? sw[0] : sw[1]) >> (16 * (cc & 1));
        const uint32_t mv = (cc < 2 ? mw[0] : mw[1]) >> (16 * (cc & 1));
        hp[wv][h_rl][2 * k + h_sb][cc] = make_float4(d * (float)(sv & 255u), d16 * (float)((sv >> 8) & 255u),
                                                     dmin * (float)(mv & 255u), dmin * (float)((mv >> 8) & 255u));
      }
    }
#pragma unroll
    for (int r = 0; r < RPL; r++) {
      float v = 0.0f;
#pragma unroll
      for (int k = 0; k < KU; k++) {
        const float sa = fma_bytes16(qc[r][k], LO4, xl[k], 0.0f);
        const float sb = fma_bytes16(qc[r][k], HI4, xh[k], 0.0f);
        const float4 f = hp[wv][slot * RPL + r][2 * k + sbl][c];
        v = k == 0 ? f.x * sa : __builtin_fmaf(f.x, sa, v);
        v = __builtin_fmaf(f.y, sb, v);
        v = __builtin_fmaf(-f.z, sl[k], v);
        v = __builtin_fmaf(-f.w, sh[k], v);
      }
      v = lane_sum<16>(v);
      if (ul == 0) part[wv][g * RG + slot * RPL + r] = v;
    }
    if (g + 1 < NG) {
#pragma unroll
      for (int r = 0; r < RPL; r++)
#pragma unroll
        for (int k = 0; k < KU; k++) qc[r][k] = qn[r][k];
#pragma unroll
      for (int k = 0; k < KU; k++) hc[k] = hn[k];
    }
  }
  __syncthreads();
  if (tid < (uint32_t)OUT && out0 + tid < p.n_out) {
    const uint32_t g = tid / OG, o = tid % OG;
    float t = 0.0f, u = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      t += part[i][g * RG + o];
      if constexpr (PAIR) u += part[i][g * RG + 2 * RPL + o];
    }
    if constexpr (NORM) {  // the pair scales its gate and up sums alike, before the SiLU
      float s2 = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; i++) s2 += wss[i];
      const float r = 1.0f / sqrtf(s2 / (float)p.n_in + p.eps);
      t *= r;
      if constexpr (PAIR) u *= r;
    }
    const uint32_t yo = p.y_off + out0 + tid;
    if constexpr (PAIR) {
#pragma clang fp contract(off)
      y[yo] = t / (1.0f + expf(-t)) * u;  // silu_mul.comp:15-23
    } else if (ACCUM) {
      y[yo] = yold + t;
    } else {
      y[yo] = t;
    }
  }
}

// ---------------------------------------------------------------------------------------
// A decode token's expert down projections and moe_combine in one launch
// (matvec_q4k_dcomb__8): graph/moe.rs:42-80 runs the down projections as the expert matvec
// over grid.y = n_used slots (four waves, one row, 16 lanes per row -- the runtime's
// variant for expert rows) and then moe_combine.  Here a workgroup owns DR rows for every
// slot, so no workgroup waits for another:
//   * each slot's activations are staged and each (slot, row) header decoded in LDS exactly
//     as matvec_q4k_body stages them (zero past n_in, zero products past the last
//     super-block), and every (slot, row) is summed by 16 lanes in that kernel's step
//     order and reduced with the same DPP pattern, so each slot's row is bit-identical to
//     the expert matvec's;
//   * the rows' weighted sum is added to the residual in moe_combine's order
//     (moe_combine.comp:16-27), so the residual is bit-identical to the two launches;
//   * all the workgroup's weights are in flight at once: 16 groups of 16 lanes, group g
//     taking slot g % 8 and rows g / 8, g / 8 + 2, ...  (n_used <= 8, n_in <= 1024), and
//     with them every header (one per thread), the routing weights and the residual rows:
//     one dependent round trip after the ids.
// The per-slot down rows are not written (nothing after moe_combine reads them).
// ---------------------------------------------------------------------------------------
template <int DR>
SK_DEV void matvec_q4k_dcomb_body(const uint4 *__restrict__ w, float *a, const uint32_t *ids,
                                  const MatvecPushComb &p, uint32_t bx) {
  constexpr int SLOTS = 8, CHU = 32, CH_SUP = CHU / 8, LPR = 16, S = CHU / LPR;
  static_assert(DR % 2 == 0, "two row sets per slot");
  static_assert(SLOTS * DR * CH_SUP == 256, "one (slot, row, super-block) header per thread");
  __shared__ float4 xf[SLOTS][8][CHU];
  __shared__ float2 xs[SLOTS][CHU];
  __shared__ float4 sc[SLOTS][DR][CH_SUP][4];
  __shared__ float tot[SLOTS][DR];
  __shared__ float rw[SLOTS];
  const uint32_t tid = threadIdx.x;
  const uint32_t units = p.n_in >> 5, supers = p.n_in >> 8;
  const uint32_t row0 = bx * DR;
  const uint32_t LO4 = opaque_mask(0x0f0f0f0fu), HI4 = opaque_mask(0xf0f0f0f0u);

  // Everything is loaded before anything is used, so the launch waits for one round trip
  // after the ids: the slots' activations (which need no ids), then this lane's weights, its
  // header and the combine's routing weights and residual row.
  constexpr int XJ = SLOTS * 4 * CHU / 256;  // activation items per thread: slot, unit, quarter
  float4 va[XJ], vb[XJ];
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const uint32_t t = tid + 256 * j, sl = t / (4 * CHU), tt = t % (4 * CHU), u = tt >> 2, qq = tt & 3;
    va[j] = vb[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (sl < p.n_used && u < units) {
      const float *xv = a + p.x_off + sl * p.x_stride;
      const uint32_t at = (u >> 3) * 256 + ((u >> 1) & 3) * 64 + (u & 1) * 16 + (qq >> 1) * 32 + (qq & 1) * 8;
      va[j] = *(const float4 *)(xv + at);
      vb[j] = *(const float4 *)(xv + at + 4);
    }
  }
  // this lane's weights: group gi (slot gs, rows gr, gr + 2, ..), lane L of its 16
  const uint32_t gi = tid >> 4, L = tid & 15, gs = gi % SLOTS, gr = gi / SLOTS;
  const bool live = gs < p.n_used;
  const uint32_t gbase = live ? ids[p.ids_off + gs] * p.n_out : 0;
  uint4 q[DR / 2][S];
#pragma unroll
  for (int k = 0; k < DR / 2; k++) {
    const uint32_t row = min(row0 + gr + 2 * k, p.n_out - 1);
#pragma unroll
    for (int st = 0; st < S; st++) {
      const uint32_t i = L + st * LPR;
      q[k][st] = make_uint4(0, 0, 0, 0);  // past n_in: multiplied by zero activations
      if (live && i < units) q[k][st] = load_nt(w + p.o0 + (size_t)(gbase + row) * units + i);
    }
  }
  // this thread's header: slot hs, row hr, super-block hb
  const uint32_t hs = tid / (DR * CH_SUP), hr = (tid / CH_SUP) % DR, hb = tid % CH_SUP;
  const bool hlive = hs < p.n_used && hb < supers;
  uint4 h = make_uint4(0, 0, 0, 0);
  if (hlive)
    h = load_nt(w + p.o1 + (size_t)(ids[p.ids_off + hs] * p.n_out + min(row0 + hr, p.n_out - 1)) * supers + hb);
  const bool owner = tid < (uint32_t)DR && row0 + tid < p.n_out;  // combines row row0 + tid
  const float res = owner ? a[p.res_off + row0 + tid] : 0.0f;
  if (tid < SLOTS) rw[tid] = tid < p.n_used ? a[p.w_off + tid] : 0.0f;

  // stage every slot's activations and decode the headers (zero products past the last
  // super-block and for absent slots)
#pragma unroll
  for (int j = 0; j < XJ; j++) {
    const uint32_t t = tid + 256 * j, sl = t / (4 * CHU), tt = t % (4 * CHU), u = tt >> 2, qq = tt & 3;
    float sum = sum4(va[j]) + sum4(vb[j]);
    sum += dpp_f<0xb1>(sum);  // + the other quarter of the same half
    xf[sl][(qq >> 1) * 4 + (qq & 1) * 2][u] = va[j];
    xf[sl][(qq >> 1) * 4 + (qq & 1) * 2 + 1][u] = vb[j];
    if ((qq & 1) == 0) ((float *)&xs[sl][u])[qq >> 1] = sum;
  }
  if (!hlive) {
#pragma unroll
    for (int cc = 0; cc < 4; cc++) sc[hs][hr][hb][cc] = make_float4(0.f, 0.f, 0.f, 0.f);
  } else {
    const float d = f16_bits_to_f32(h.x & 0xffffu), dmin = f16_bits_to_f32(h.x >> 16);
    const float d16 = d * 0.0625f;
    const uint32_t sw[2] = {h.y & 0x3f3f3f3fu, (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u)};
    const uint32_t mw[2] = {h.z & 0x3f3f3f3fu, ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u)};
#pragma unroll
    for (int cc = 0; cc < 4; cc++) {
      const uint32_t sv = sw[cc >> 1] >> (16 * (cc & 1)), mv = mw[cc >> 1] >> (16 * (cc & 1));
      const float s_lo = (float)(sv & 255u), s_hi = (float)((sv >> 8) & 255u);
      const float m_lo = (float)(mv & 255u), m_hi = (float)((mv >> 8) & 255u);
      sc[hs][hr][hb][cc] = make_float4(d * s_lo, d16 * s_hi, dmin * m_lo, dmin * m_hi);
    }
  }
  __syncthreads();
  // the expert matvec's steps: unit i = L + 16 st, super-block i / 8, chunk (L / 2) % 4
  const uint32_t c = (L >> 1) & 3;
#pragma unroll
  for (int k = 0; k < DR / 2; k++) {
    const uint32_t lr = gr + 2 * k;
    float acc = 0.0f;
#pragma unroll
    for (int st = 0; st < S; st++) {
      const uint32_t i = L + st * LPR, sb = (L >> 3) + st * (LPR / 8);
      const float4 xl[4] = {xf[gs][0][i], xf[gs][1][i], xf[gs][2][i], xf[gs][3][i]};
      const float sa = fma_bytes16(q[k][st], LO4, xl, 0.0f);
      const float4 xh[4] = {xf[gs][4][i], xf[gs][5][i], xf[gs][6][i], xf[gs][7][i]};
      const float sb2 = fma_bytes16(q[k][st], HI4, xh, 0.0f);
      const float2 xsum = xs[gs][i];
      const float4 f = sc[gs][lr][sb][c];
      acc = __builtin_fmaf(f.x, sa, acc);
      acc = __builtin_fmaf(f.y, sb2, acc);
      acc = __builtin_fmaf(-f.z, xsum.x, acc);
      acc = __builtin_fmaf(-f.w, xsum.y, acc);
    }
    const float total = lane_sum<LPR>(acc);
    if (L == 0) tot[gs][lr] = total;
  }
  __syncthreads();
  if (owner) {
#pragma clang fp contract(off)
    float sum = 0.0f;
    for (uint32_t s = 0; s < p.n_used; s++) sum += rw[s] * tot[s][tid];
    a[p.res_off + row0 + tid] = res + sum;
  }
}

// ---------------------------------------------------------------------------------------
// Q6_K.  Lane step = 64 values of one super-block: u -> super-block u/4, half hf = (u%4)/2,
// li = u%2.  It reads 16 B of ql at l = 16 li (a), 16 B at l + 32 (b) and 16 B of qh.
// Group g = 0..3 is values 128 hf + 32 g + 16 li + [0,16) with scale sc[8 hf + li + 2g]
// (quant.rs:72-87).  Each word of a group is rebuilt as four bytes q = nibble | 2 high bits
// << 4 (the stored 6-bit value; the quant is q - 32), converted exactly to f32 and
// multiplied with f32 activations; the group sum starts at -32 * sum(x).
// LDS per pass: xf[4g + k][unit] = activations 4k..4k+3 of group g (f32), xs[unit] = the 4
// group sums, and per (row, super-block) and (hf, li): d*sc for the lane's 4 groups.
// ---------------------------------------------------------------------------------------
template <int WAVES, int ROWS, int LPR>
struct GeoQ6 {
  static constexpr int RWG = WAVES * (64 / LPR) * ROWS;  // rows per workgroup
  static constexpr int NT = 64 * WAVES;
  // super-blocks of activations per pass: 16 KiB of f32 activations and <= 16 KiB of scales
  static constexpr int CH_SUP = (256 / RWG) < 1 ? 1 : ((256 / RWG) > 16 ? 16 : (256 / RWG));
  static constexpr int CH = CH_SUP * 256;          // values per pass
};

template <int WAVES, int ACCUM, int ROWS, int MOE, int LPR, int MODE = 0, typename P = MatvecPush4>
SK_DEV void matvec_q6k_body(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd,
                            const float *x, float *y, const uint32_t *ids, const P &p,
                            uint32_t bx) {
  using G = GeoQ6<WAVES, ROWS, LPR>;
  __shared__ float4 xf[16][G::CH / 64];  // component-major
  __shared__ float4 xs[G::CH / 64];
  __shared__ float4 sc[G::RWG][G::CH_SUP][4];
  __shared__ float wss[MODE == 2 ? 4 * WAVES : 1];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = (tid & 63) % LPR;
  const uint32_t sub = (tid & 63) / LPR;
  const uint32_t row0 = bx * G::RWG;
  const uint32_t lrow0 = ((tid >> 6) * (64 / LPR) + sub) * ROWS;
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
  const uint32_t LO4 = opaque_mask(0x0f0f0f0fu), H2 = opaque_mask(0x30303030u);

  uint32_t rb[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) rb[r] = (base + min(first + r, p.n_out - 1)) * supers;

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;
  float yold[ROWS];
  load_old<ACCUM, ROWS>(y, y_off, first, p.n_out, lane, yold);

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
        a[r] = load_nt(w + p.o0 + rs * 8 + hf * 4 + li);
        b[r] = load_nt(w + p.o0 + rs * 8 + hf * 4 + 2 + li);
        h[r] = load_nt(w + p.o1 + rs * 4 + hf * 2 + li);
      }
    };
    // activation item t = group t%4 of unit t/4: 16 values (4 x 16 B) and their sum
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
    float ssp = 0.0f;  // MODE 2: this pass's sum of x^2
    auto x_store = [&](uint32_t t, float4 (&v)[4]) {
      const uint32_t i = t >> 2, g = t & 3;
      if constexpr (MODE != 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = fuse4<MODE>(v[k], xu4[k], ssp);
      }
#pragma unroll
      for (int k = 0; k < 4; k++) xf[4 * g + k][i] = v[k];
      ((float *)&xs[i])[g] = (sum4(v[0]) + sum4(v[1])) + (sum4(v[2]) + sum4(v[3]));
    };
    const uint32_t n_items = (uint32_t)G::RWG * ns;
    auto h_load = [&](uint32_t i, uint4 &sv, uint32_t &dv) {
      const uint32_t lr = i / ns, s = i % ns;
      const uint32_t rs = (base + min(row0 + lr, p.n_out - 1)) * supers + s0 + s;
      sv = load_nt(w + p.o2 + rs);
      dv = load_nt(wd + p.o3 + rs);
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
          o[g] = d * (float)s8;
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
    if (tid < n_xi) x_store(tid, xv4);
    if (tid < n_items) h_store(tid, sv0, dv0);
    for (uint32_t t = tid + G::NT; t < n_xi; t += G::NT) {
      x_item(t, xv4);
      x_store(t, xv4);
    }
    for (uint32_t i = tid + G::NT; i < n_items; i += G::NT) {
      h_load(i, sv0, dv0);
      h_store(i, sv0, dv0);
    }
    norm_note<MODE, WAVES>(wss, ssp);
    __syncthreads();
    norm_take<MODE, WAVES>(wss, ss);

    for (uint32_t j0 = 0; lane + j0 * LPR < nu; j0 += PF) {
#pragma unroll
      for (int j = 0; j < PF; j++) {
        const uint32_t i = lane + (j0 + j) * LPR;
        if (i < nu) {
          const float4 xsum = xs[i];
          const float ib[4] = {-32.0f * xsum.x, -32.0f * xsum.y, -32.0f * xsum.z, -32.0f * xsum.w};
          const uint32_t s = i >> 2;
#pragma unroll
          for (int r = 0; r < ROWS; r++) {
            float t[4];
            // group g: quants from ql half a (g even) or b (g odd), low nibbles for g < 2 and
            // high for g >= 2; qh bits 2g, 2g+1 of each byte moved to bits 4-5.  One group's
            // operands are live at a time.
#pragma unroll
            for (int g = 0; g < 4; g++) {
              const float4 xg[4] = {xf[4 * g][i], xf[4 * g + 1][i], xf[4 * g + 2][i], xf[4 * g + 3][i]};
              const uint4 qv = (g & 1) ? qb[j][r] : qa[j][r];
              const uint32_t wv4[4] = {qv.x, qv.y, qv.z, qv.w};
              const uint32_t hv[4] = {qh[j][r].x, qh[j][r].y, qh[j][r].z, qh[j][r].w};
              float tg = ib[g];
#pragma unroll
              for (int k = 0; k < 4; k++) {
                const uint32_t lo = g < 2 ? wv4[k] : wv4[k] >> 4;
                const uint32_t hb = g == 0 ? hv[k] << 4 : g == 1 ? hv[k] << 2 : g == 2 ? hv[k] : hv[k] >> 2;
                tg = fma_bytes((lo & LO4) | (hb & H2), xg[k], tg);
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
  }
  norm_apply<MODE>(acc, ss, p);
  store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc, yold);
}

// ---------------------------------------------------------------------------------------
// Q6_K, K-split form for n_in = 12288 (the Qwen3-8B down projection).  Three waves split
// every row the workgroup owns into its 192 units of 64 values: lane l of wave w takes unit
// u = 64 w + l (super-block u/4, half hf = (u/2)%2, li = u%2, as in matvec_q6k_body) of
// each row.  A lane's 64 activations and their four 16-value sums are the same for every
// row it touches: they are loaded once, into registers, and no activation goes through
// LDS.  Per row the lane loads its unit's 48 quant bytes (16 B of ql at l = 16 li, 16 B at
// l + 32, 16 B of qh), the 8 scale bytes of its half and d, one row-group of RPL rows ahead
// of the arithmetic.  Each group sum is matvec_q6k_body's (from -32 sum(x), four words of
// rebuilt 6-bit quants); the four take d*sc (quant.rs:72-87) and are reduced over the wave
// with DPP, and the three waves' row partials meet in LDS once, at the end, in wave order.
// PD row-groups are loaded ahead of the arithmetic (at 4096 rows one row-group of one row
// ahead measured fastest: issuing more of a lane's rows at once was slower).
// ---------------------------------------------------------------------------------------
template <int ACCUM, int RPL, int NG, int PD = 1>
SK_DEV void matvec_q6k_ks_body(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd, const float *x,
                               float *y, const MatvecPush4 &p, uint32_t bx) {
  constexpr int OUT = RPL * NG;     // rows per workgroup
  constexpr uint32_t SUPERS = 48;   // super-blocks per row (n_in = 12288, checked by the host)
  __shared__ float part[3][OUT];

  const uint32_t tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
  const uint32_t u = wv * 64 + l;
  const uint32_t sb = u >> 2, hf = (u >> 1) & 1, li = u & 1;
  const uint32_t LO4 = opaque_mask(0x0f0f0f0fu), H2 = opaque_mask(0x30303030u);
  const uint32_t out0 = bx * OUT;

  struct RowQ {
    uint4 a, b, h;
    uint2 sc;
    uint32_t d;
  };
  auto load_group = [&](uint32_t g, RowQ (&q)[RPL]) {
#pragma unroll
    for (int r = 0; r < RPL; r++) {
      const uint32_t rs = min(out0 + g * RPL + r, p.n_out - 1) * SUPERS + sb;
      q[r].a = load_nt(w + p.o0 + rs * 8 + hf * 4 + li);
      q[r].b = load_nt(w + p.o0 + rs * 8 + hf * 4 + 2 + li);
      q[r].h = load_nt(w + p.o1 + rs * 4 + hf * 2 + li);
      q[r].sc = load_nt((const uint2 *)(w + p.o2 + rs) + hf);
      q[r].d = load_nt(wd + p.o3 + rs);
    }
  };

  // activations first: group g = values 128 hf + 32 g + 16 li + [0, 16) of super-block sb
  RowQ q[NG][RPL];  // row-group g's operands, loaded PD groups ahead of its arithmetic
  const float *xv = x + p.x_off + sb * 256 + hf * 128 + li * 16;
  float4 xg[4][4];
#pragma unroll
  for (int g = 0; g < 4; g++)
#pragma unroll
    for (int k = 0; k < 4; k++) xg[g][k] = *(const float4 *)(xv + 32 * g + 4 * k);
#pragma unroll
  for (int g = 0; g < PD && g < NG; g++) load_group(g, q[g]);
  // an accumulating launch reads its old outputs now, so the store at the end waits for none
  float yold = 0.0f;
  if constexpr (ACCUM)
    if (tid < (uint32_t)OUT && out0 + tid < p.n_out) yold = y[p.y_off + out0 + tid];
  float ib[4];
#pragma unroll
  for (int g = 0; g < 4; g++)
    ib[g] = -32.0f * ((sum4(xg[g][0]) + sum4(xg[g][1])) + (sum4(xg[g][2]) + sum4(xg[g][3])));

#pragma unroll
  for (int g = 0; g < NG; g++) {
    if (g + PD < NG) load_group(g + PD, q[g + PD]);
    const RowQ (&qc)[RPL] = q[g];
#pragma unroll
    for (int r = 0; r < RPL; r++) {
      const uint32_t hv[4] = {qc[r].h.x, qc[r].h.y, qc[r].h.z, qc[r].h.w};
      float t[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint4 qv = (j & 1) ? qc[r].b : qc[r].a;
        const uint32_t wv4[4] = {qv.x, qv.y, qv.z, qv.w};
        float tg = ib[j];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const uint32_t lo = j < 2 ? wv4[k] : wv4[k] >> 4;
          const uint32_t hb = j == 0 ? hv[k] << 4 : j == 1 ? hv[k] << 2 : j == 2 ? hv[k] : hv[k] >> 2;
          tg = fma_bytes((lo & LO4) | (hb & H2), xg[j][k], tg);
        }
        t[j] = tg;
      }
      // d * sc[8 hf + li + 2 j]: bytes li + 2 j of the half's 8 scale bytes
      const float d = f16_bits_to_f32(qc[r].d & 0xffffu);
      float f[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t word = j < 2 ? qc[r].sc.x : qc[r].sc.y;
        f[j] = d * (float)(int)(int8_t)((word >> (8 * (li + 2 * (j & 1)))) & 255u);
      }
      float v = f[0] * t[0];
      v = __builtin_fmaf(f[1], t[1], v);
      v = __builtin_fmaf(f[2], t[2], v);
      v = __builtin_fmaf(f[3], t[3], v);
      v = lane_sum<64>(v);
      if (l == 0) part[wv][g * RPL + r] = v;
    }
  }
  __syncthreads();
  if (tid < (uint32_t)OUT && out0 + tid < p.n_out) {
    const float t = (part[0][tid] + part[1][tid]) + part[2][tid];
    const uint32_t yo = p.y_off + out0 + tid;
    if (ACCUM)
      y[yo] = yold + t;
    else
      y[yo] = t;
  }
}

// ---------------------------------------------------------------------------------------
// Q8_0.  Lane step = 16 quants (half a block) of one row; the block scale d is staged per
// (row, block) as f32.  q ^ 0x80 is q + 128 as a byte (0..255), converted exactly to f32;
// the unit's sum starts at -128 * sum(x), then takes d.
// LDS per pass: xf[k][unit] = activations 4k..4k+3 (f32), xs[unit] = their sum,
// dd[row][block] = d.
// ---------------------------------------------------------------------------------------
template <int WAVES, int ROWS, int LPR>
struct GeoQ8 {
  static constexpr int RWG = WAVES * (64 / LPR) * ROWS;  // rows per workgroup
  static constexpr int NT = 64 * WAVES;
  // values per pass: 32 KiB of f32 activations and <= 32 KiB of block scales
  static constexpr int CH = (8192 * 8 / RWG) > 8192 ? 8192 : (8192 * 8 / RWG);
};

template <int WAVES, int ACCUM, int ROWS, int MOE, int LPR, int MODE = 0, typename P = MatvecPush2>
SK_DEV void matvec_q8_0_body(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd,
                             const float *x, float *y, const uint32_t *ids, const P &p,
                             uint32_t bx) {
  using G = GeoQ8<WAVES, ROWS, LPR>;
  constexpr int NBLK = G::CH / 32;
  __shared__ float4 xf[4][G::CH / 16];  // component-major
  __shared__ float xs[G::CH / 16];
  __shared__ float dd[G::RWG][NBLK];
  __shared__ float wss[MODE == 2 ? 4 * WAVES : 1];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = (tid & 63) % LPR;
  const uint32_t sub = (tid & 63) / LPR;
  const uint32_t row0 = bx * G::RWG;
  const uint32_t lrow0 = ((tid >> 6) * (64 / LPR) + sub) * ROWS;
  const uint32_t first = row0 + lrow0;
  const uint32_t slot = blockIdx.y;
  const uint32_t base = MOE ? ids[p.ids_off + slot] * p.n_out : 0;
  const float *xv = x + p.x_off + slot * p.x_stride;
  const float *av = x;  // MODE != 0: the second vector, indexed as xv
  if constexpr (MODE != 0) av = x + p.aux_off + (MODE == 1 ? slot * p.x_stride : 0);
  float ss = 0.0f;
  const uint32_t y_off = p.y_off + slot * p.y_stride;
  const uint32_t chunks = p.n_in >> 4, blocks = p.n_in >> 5;
  const uint32_t SG = opaque_mask(0x80808080u);

  const uint4 *qr[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) qr[r] = w + p.o0 + (base + min(first + r, p.n_out - 1)) * chunks;

  float acc[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; r++) acc[r] = 0.0f;
  float yold[ROWS];
  load_old<ACCUM, ROWS>(y, y_off, first, p.n_out, lane, yold);

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
    float ssp = 0.0f;  // MODE 2: this pass's sum of x^2
    auto x_store = [&](uint32_t i, float4 (&v)[4]) {
      if constexpr (MODE != 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = fuse4<MODE>(v[k], xu4[k], ssp);
      }
#pragma unroll
      for (int k = 0; k < 4; k++) xf[k][i] = v[k];
      xs[i] = (sum4(v[0]) + sum4(v[1])) + (sum4(v[2]) + sum4(v[3]));
    };
    const uint32_t n_items = (uint32_t)G::RWG * nb;
    auto d_load = [&](uint32_t i) -> uint32_t {
      const uint32_t lr = i / nb, bl = i % nb;
      const uint32_t row = base + min(row0 + lr, p.n_out - 1);
      return load_nt(wd + p.o1 + row * blocks + b0 + bl);
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
      for (int r = 0; r < ROWS; r++) q[j][r] = load_nt(qr[r] + u0 + i);
    }
    if (tid < nu) x_store(tid, xv4);
    if (tid < n_items) dd[tid / nb][tid % nb] = f16_bits_to_f32(dv0);
    for (uint32_t i = tid + G::NT; i < nu; i += G::NT) {
      x_unit(i, xv4);
      x_store(i, xv4);
    }
    for (uint32_t i = tid + G::NT; i < n_items; i += G::NT) dd[i / nb][i % nb] = f16_bits_to_f32(d_load(i));
    norm_note<MODE, WAVES>(wss, ssp);
    __syncthreads();
    norm_take<MODE, WAVES>(wss, ss);

    for (uint32_t j0 = 0; lane + j0 * LPR < nu; j0 += PF) {
#pragma unroll
      for (int j = 0; j < PF; j++) {
        const uint32_t i = lane + (j0 + j) * LPR;
        if (i < nu) {
          const float4 xk[4] = {xf[0][i], xf[1][i], xf[2][i], xf[3][i]};
          const float bias = -128.0f * xs[i];
#pragma unroll
          for (int r = 0; r < ROWS; r++) {
            float s = bias;
            s = fma_bytes(q[j][r].x ^ SG, xk[0], s);
            s = fma_bytes(q[j][r].y ^ SG, xk[1], s);
            s = fma_bytes(q[j][r].z ^ SG, xk[2], s);
            s = fma_bytes(q[j][r].w ^ SG, xk[3], s);
            acc[r] = __builtin_fmaf(dd[lrow0 + r][i >> 1], s, acc[r]);
          }
        }
        const uint32_t inext = min(i + PF * LPR, nu - 1);
#pragma unroll
        for (int r = 0; r < ROWS; r++) q[j][r] = load_nt(qr[r] + u0 + inext);
      }
    }
  }
  norm_apply<MODE>(acc, ss, p);
  store_rows<ACCUM, ROWS, LPR>(y, y_off, first, p.n_out, lane, acc, yold);
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
MV_Q8_0_F(silu, 1, 4, 1, 1, 64)  // dense Q8_0 launches below 2048 rows
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
// the Q8_0 output head (65536 rows or more, no accumulation): 16 lanes per row, 16 rows a workgroup
MV_Q8_0(4, 0, 1, 0, 16)

// K-split Q4_K form for n_in = 4096 (matvec_q4k_ks_body): RPL rows per slot, NG row-groups
// per workgroup; the runtime picks it for dense Q4_K launches whose rows all have n_in 4096.
#define MV_Q4K_KS(A, R, G)                                                                   \
  extern "C" __global__ __launch_bounds__(512) void matvec_q4k_ks__##A##_##R##_##G(           \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPush2> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    (void)ids;                                                                               \
    matvec_q4k_ks_body<A, R, G>(w, x, y, segment_push(m, s), blockIdx.x - m.start[s]);       \
  }
#define MV_Q4K_KS_NORM(R, G)                                                                 \
  extern "C" __global__ __launch_bounds__(512) void matvec_q4k_ks_norm__0_##R##_##G(          \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPush2F> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    (void)ids;                                                                               \
    matvec_q4k_ks_body<0, R, G, 2>(w, x, y, segment_push(m, s), blockIdx.x - m.start[s]);    \
  }
#define MV_Q4K_KS_GLU(R, G)                                                                  \
  extern "C" __global__ __launch_bounds__(512) void matvec_q4k_ks_glu__0_##R##_##G(           \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPushGlu> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    (void)ids;                                                                               \
    matvec_q4k_ks_body<0, R, G, 3>(w, x, y, segment_push(m, s), blockIdx.x - m.start[s]);    \
  }
#define MV_Q4K_KS_GLUN(R, G)                                                                 \
  extern "C" __global__ __launch_bounds__(512) void matvec_q4k_ks_glun__0_##R##_##G(          \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPushGluN> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    (void)ids;                                                                               \
    matvec_q4k_ks_body<0, R, G, 4>(w, x, y, segment_push(m, s), blockIdx.x - m.start[s]);    \
  }
#define MV_Q4K_KS_ALL(R, G) MV_Q4K_KS(0, R, G) MV_Q4K_KS(1, R, G) MV_Q4K_KS_NORM(R, G) MV_Q4K_KS_GLU(R, G) \
  MV_Q4K_KS_GLUN(R, G)
MV_Q4K_KS_ALL(2, 1)
MV_Q4K_KS_ALL(2, 2)
MV_Q4K_KS_ALL(4, 1)
MV_Q4K_KS_ALL(4, 2)
MV_Q4K_KS_ALL(4, 3)
MV_Q4K_KS_ALL(4, 6)
MV_Q4K_KS_ALL(8, 1)
MV_Q4K_KS_ALL(8, 3)
// K-split Q4_K form for n_in = 12288 (KU = 3): the Qwen3-8B Q4_K down projection
#define MV_Q4K_KS3(A, R, G)                                                                  \
  extern "C" __global__ __launch_bounds__(512) void matvec_q4k_ks3__##A##_##R##_##G(          \
      const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPush2> m) { \
    const uint32_t s = segment_of(m, blockIdx.x);                                            \
    (void)ids;                                                                               \
    matvec_q4k_ks_body<A, R, G, 0, MatvecPush2, 3>(w, x, y, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
MV_Q4K_KS3(0, 2, 1)
MV_Q4K_KS3(1, 2, 1)
MV_Q4K_KS3(0, 2, 2)
MV_Q4K_KS3(1, 2, 2)
MV_Q4K_KS3(0, 4, 1)
MV_Q4K_KS3(1, 4, 1)

// K-split Q6_K form for n_in = 12288 (matvec_q6k_ks_body): RPL rows per row-group, NG
// row-groups per workgroup of three waves, loaded D row-groups ahead
#define MV_Q6K_KS(A, R, G, D)                                                                \
  extern "C" __global__ __launch_bounds__(192) void matvec_q6k_ks__##A##_##R##_##G##_##D(     \
      const uint4 *w, const uint16_t *wd, const float *x, float *y, const uint32_t *ids,      \
      Segments<MatvecPush4> m) {                                                              \
    const uint32_t s = segment_of(m, blockIdx.x);                                             \
    (void)ids;                                                                                \
    matvec_q6k_ks_body<A, R, G, D>(w, wd, x, y, segment_push(m, s), blockIdx.x - m.start[s]); \
  }
#define MV_Q6K_KS_ALL(R, G, D) MV_Q6K_KS(0, R, G, D) MV_Q6K_KS(1, R, G, D)
MV_Q6K_KS_ALL(1, 8, 1)
MV_Q6K_KS_ALL(1, 8, 2)
MV_Q6K_KS_ALL(1, 8, 7)
MV_Q6K_KS_ALL(1, 16, 2)
MV_Q6K_KS_ALL(2, 4, 2)
MV_Q6K_KS_ALL(8, 1, 1)

// MoE decode forms the runtime substitutes for engine dispatch runs (skyla_hip.cpp,
// fuse_moe): an expert's gate and up with silu_mul after them (MODE 3 over the slot grid),
// the same with moe_route's selection in front, and an expert down projection with
// moe_combine after it.
extern "C" __global__ __launch_bounds__(256) void matvec_q4k_glu__4_0_1_1_16(
    const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPushGlu> m) {
  const uint32_t s = segment_of(m, blockIdx.x);
  matvec_q4k_body<4, 0, 1, 1, 16, 3>(w, x, y, ids, segment_push(m, s), blockIdx.x - m.start[s]);
}
// moe_route then the experts' gate + up + silu of one decode token in one launch: every
// workgroup ranks the logits itself (route_ranked, all four waves), so each knows its slot's
// expert without waiting for another; workgroup (0, 0) also stores the ids and routing
// weights for the launches after it.  Same ids, weights and outputs, bit for bit, as
// moe_route then matvec_q4k_glu__4_0_1_1_16.
extern "C" __global__ __launch_bounds__(256) void matvec_q4k_glur__4_0_1_1_16(
    const uint4 *w, const float *x, float *y, uint32_t *ids, Segments<MatvecPushGluR> m) {
  __shared__ uint32_t sid[16];
  __shared__ float sval[16];
  const MatvecPushGluR pp = m.p[0];
  route_ranked(y, pp.r, 0, threadIdx.x, sid, sval);
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 64) {
    const uint32_t n_used = min(pp.r.n_used, 16u), t = threadIdx.x;
    const float wt = route_weight(t < n_used ? sval[t] : 0.0f, n_used);
    if (t < n_used) {
      ids[pp.r.ids_off + t] = sid[t];
      y[pp.r.weights_off + t] = wt;
    }
  }
  MatvecPushGlu g = pp.g;
  g.ids_off = 0;
  matvec_q4k_body<4, 0, 1, 1, 16, 3>(w, x, y, sid, g, blockIdx.x);
}
// an expert down projection and moe_combine for one token, no handoff (matvec_q4k_dcomb_body)
extern "C" __global__ __launch_bounds__(256) void matvec_q4k_dcomb__8(
    const uint4 *w, const float *x, float *y, const uint32_t *ids, Segments<MatvecPushComb> m) {
  (void)x;  // the arena is bound as x, y and ids; y is its writable view
  matvec_q4k_dcomb_body<8>(w, y, ids, m.p[0], blockIdx.x);
}
