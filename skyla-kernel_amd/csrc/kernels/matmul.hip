// Prefill matmul over raw Q8_0 / Q4_K / Q6_K blocks on gfx950 MFMA.
//
// Contract (matmul.comp:113-184, graph.rs:23-34, graph/moe.rs:26-40):
//   spec [TYPE, ACCUM, MOE(, X_HALF)]: TYPE 0/1/2 = Q8_0/Q4_K/Q6_K.  Workgroup = 128 output
//   rows (MATMUL_TILE_ROWS) x TN tokens; grid = [ceil(n_out/128), 1 | n_expert, z] and tile z
//   covers tokens [z*TN, z*TN+TN).  Dense: token count = ctl[2], token i reads x row i and
//   writes y row i.  MOE: expert e = grid.y, (count, start) = table[e], token i of the
//   group is slot s = list[start + i]; it reads x row s / x_div and writes y row s; the
//   weight rows are offset by e * n_out.  Output is token-major: y[y_off + row_tok *
//   y_stride + out_row] (+= with ACCUM).  X is f32, or f16 when X_HALF (then x_off and
//   x_stride count f16 elements).
//
// MI355X design:
//   * v_mfma_f32_32x32x16_f16 with f32 accumulation.  D = X * W^T so each lane owns one
//     output row and stores are 128-byte coalesced runs along the row dimension.
//   * weights never touch LDS: each wave owns 32 rows and dequantises its fragments in
//     registers, 8 values per lane per MFMA step, into exactly the operand layout the MFMA
//     reads (lane l: row l%32, lane half l/32 selects which 8 k of the step).  Quants
//     become f16 through the 0x6400 mantissa trick, then one packed f16 add removes the
//     offset (exact) and one packed f16 fma/mul applies scale and min.
//   * the K order inside a 256-value super-block is permuted freely (a sum does not care),
//     so each lane half always reads from a single sub-block per step; activations are
//     staged in the same order: 8 consecutive k per lane, pairs stored as (0,2),(1,3),(4,6),
//     (5,7) to match the packed-quant extraction.
//   * activations go through LDS as f16, double buffered: the next super-block's global
//     loads are in flight while the current one runs on the matrix cores.
#include "common.h"

namespace {

constexpr int TM = 128;        // rows per workgroup
constexpr uint32_t TILE_MAP = 640;  // words of moe_sort's tile map before its table (moe.hip)
constexpr int KC = 256;        // k per LDS stage (one K-quant super-block)
constexpr int PITCH = KC + 8;  // f16 per staged token row (16 B pad: conflict-free b128)

struct MatmulPush {  // 13 words (graph.rs:27-32, graph/moe.rs:26-40)
  uint32_t o0, o1, o2, o3, x_off, y_off, n_in, n_out, x_stride, y_stride, table_off, list_off,
      x_div;
};

SK_DEV f16x2 splat(f16 v) {
  f16x2 r = {v, v};
  return r;
}

// k offset (inside the current 256-k stage) of the 8 values lane-half hh holds at step t
template <int TYPE>
SK_DEV uint32_t koff(int t, uint32_t hh) {
  if (TYPE == 1) return 64 * (t >> 2) + 32 * hh + 8 * (t & 3);                  // Q4_K
  if (TYPE == 2) return 128 * (t >> 3) + 32 * ((t >> 1) & 3) + 16 * (t & 1) + 8 * hh;  // Q6_K
  return 16 * t + 8 * hh;                                                            // Q8_0
}

// Raw weight bytes of one row for one 256-k stage, held by each lane.
template <int TYPE>
struct WStage;

template <>
struct WStage<1> {  // Q4_K: 128 B qs + 16 B header
  uint4 qs[8];
  uint4 hd;
};
template <>
struct WStage<2> {  // Q6_K: ql 128 B, qh 64 B, 16 scales, d
  uint4 ql[8];
  uint4 qh[4];
  uint4 sc;
  uint32_t d;
};
template <>
struct WStage<0> {  // Q8_0: 8 blocks of 32 quants + 8 scales
  uint4 q[16];
  uint32_t d[8];
};

template <int TYPE>
SK_DEV void load_stage(WStage<TYPE> &s, const uint4 *w, const uint16_t *wd, const MatmulPush &p,
                       uint32_t row, uint32_t kc, uint32_t nk) {
  if constexpr (TYPE == 1) {
    const uint32_t units = p.n_in >> 5, supers = p.n_in >> 8, sb = kc >> 8;
    const uint4 *q = w + p.o0 + row * units + sb * 8;
#pragma unroll
    for (int i = 0; i < 8; i++) s.qs[i] = q[i];
    s.hd = w[p.o1 + row * supers + sb];
  } else if constexpr (TYPE == 2) {
    const uint32_t rs = row * (p.n_in >> 8) + (kc >> 8);
#pragma unroll
    for (int i = 0; i < 8; i++) s.ql[i] = w[p.o0 + rs * 8 + i];
#pragma unroll
    for (int i = 0; i < 4; i++) s.qh[i] = w[p.o1 + rs * 4 + i];
    s.sc = w[p.o2 + rs];
    s.d = wd[p.o3 + rs];
  } else {
    const uint32_t chunks = p.n_in >> 4, blocks = p.n_in >> 5;
    const uint4 *q = w + p.o0 + row * chunks + (kc >> 4);
    const uint16_t *d = wd + p.o1 + row * blocks + (kc >> 5);
    const uint32_t nb = nk >> 5;  // whole blocks in this stage
#pragma unroll
    for (int b = 0; b < 8; b++) {
      if ((uint32_t)b < nb) {
        s.q[2 * b] = q[2 * b];
        s.q[2 * b + 1] = q[2 * b + 1];
        s.d[b] = d[b];
      } else {
        s.q[2 * b] = make_uint4(0, 0, 0, 0);
        s.q[2 * b + 1] = make_uint4(0, 0, 0, 0);
        s.d[b] = 0;
      }
    }
  }
}

// Dequantised f16 operand (8 values, pair-permuted) of lane half hh at step t.
template <int TYPE>
SK_DEV f16x8 weight_frag(const WStage<TYPE> &s, int t, uint32_t hh, f16x2 scale, f16x2 negmin) {
  const uint32_t M = 0x64006400u;
  uint32_t d0, d1, m0, m1;
  f16x2 off;
  if constexpr (TYPE == 1) {
    // chunk c = t/4 holds sub-blocks 2c (low nibbles, hh = 0) and 2c+1 (high, hh = 1)
    const int c = t >> 2, pc = t & 3;
    const uint4 v = s.qs[2 * c + (pc >> 1)];
    d0 = (pc & 1) ? v.z : v.x;
    d1 = (pc & 1) ? v.w : v.y;
    const uint32_t mask = hh ? 0x00f000f0u : 0x000f000fu;
    m0 = mask;
    m1 = mask;
    off = splat((f16)-1024.0f);
    const uint32_t a = (d0 & m0) | M, b = ((d0 >> 8) & m0) | M;
    const uint32_t e = (d1 & m1) | M, f = ((d1 >> 8) & m1) | M;
    f16x2 w0 = __builtin_elementwise_fma(as_f16x2(a) + off, scale, negmin);
    f16x2 w1 = __builtin_elementwise_fma(as_f16x2(b) + off, scale, negmin);
    f16x2 w2 = __builtin_elementwise_fma(as_f16x2(e) + off, scale, negmin);
    f16x2 w3 = __builtin_elementwise_fma(as_f16x2(f) + off, scale, negmin);
    f16x8 r = {w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
    return r;
  } else if constexpr (TYPE == 2) {
    // step t: half hf = t/8, group g = (t/2)%4, l0 = 16 (t%2) + 8 hh
    const int hf = t >> 3, g = (t >> 1) & 3;
    // byte offsets inside the 32-byte runs for lane half 0; half 1 reads 8 bytes further.
    // Both candidates use constant indices (t is unrolled) and the lane picks one, so the
    // staged arrays stay in registers.
    const uint32_t l0 = 16 * (t & 1);
    const uint32_t lbyte = hf * 64 + ((g & 1) ? 32 : 0) + l0;
    const uint32_t hbyte = hf * 32 + l0;
    auto word = [](const uint4 *v, uint32_t byte) -> uint32_t {
      const uint4 q = v[byte >> 4];
      const uint32_t k = (byte >> 2) & 3;
      return k == 0 ? q.x : (k == 1 ? q.y : (k == 2 ? q.z : q.w));
    };
    const uint32_t l_0 = hh ? word(s.ql, lbyte + 8) : word(s.ql, lbyte);
    const uint32_t l_1 = hh ? word(s.ql, lbyte + 12) : word(s.ql, lbyte + 4);
    const uint32_t h_0 = hh ? word(s.qh, hbyte + 8) : word(s.qh, hbyte);
    const uint32_t h_1 = hh ? word(s.qh, hbyte + 12) : word(s.qh, hbyte + 4);
    const uint32_t lmask = (g >= 2) ? 0x00f000f0u : 0x000f000fu;
    const uint32_t hmask = (g >= 2) ? 0x03000300u : 0x00300030u;
    const int hs = 4 - 2 * (g & 1);
    auto q6 = [&](uint32_t l, uint32_t h) -> uint32_t { return (l & lmask) | M | ((h << hs) & hmask); };
    off = splat((g >= 2) ? (f16)-1536.0f : (f16)-1056.0f);
    f16x2 w0 = (as_f16x2(q6(l_0, h_0)) + off) * scale;
    f16x2 w1 = (as_f16x2(q6(l_0 >> 8, h_0 >> 8)) + off) * scale;
    f16x2 w2 = (as_f16x2(q6(l_1, h_1)) + off) * scale;
    f16x2 w3 = (as_f16x2(q6(l_1 >> 8, h_1 >> 8)) + off) * scale;
    (void)negmin;
    (void)m0;
    (void)m1;
    f16x8 r = {w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
    return r;
  } else {
    const uint4 v = s.q[t];
    d0 = hh ? v.z : v.x;
    d1 = hh ? v.w : v.y;
    d0 ^= 0x80808080u;
    d1 ^= 0x80808080u;
    off = splat((f16)-1152.0f);
    f16x2 w0 = (as_f16x2((d0 & 0x00ff00ffu) | M) + off) * scale;
    f16x2 w1 = (as_f16x2(((d0 >> 8) & 0x00ff00ffu) | M) + off) * scale;
    f16x2 w2 = (as_f16x2((d1 & 0x00ff00ffu) | M) + off) * scale;
    f16x2 w3 = (as_f16x2(((d1 >> 8) & 0x00ff00ffu) | M) + off) * scale;
    (void)negmin;
    (void)m0;
    (void)m1;
    f16x8 r = {w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
    return r;
  }
}

// Scale (and negated min) of lane half hh at step t, as f16 pairs.  The f32 products
// d*sc and dmin*m are the reference's d0 / min0 (quant.rs:60-61), rounded once to f16.
template <int TYPE>
SK_DEV void step_scale(const WStage<TYPE> &s, int t, uint32_t hh, f16x2 &scale, f16x2 &negmin) {
  if constexpr (TYPE == 1) {
    const uint32_t j = 2 * (t >> 2) + hh;
    uint32_t sc, m;
    q4k_scale_min(j, s.hd.y, s.hd.z, s.hd.w, sc, m);
    const float d = f16_bits_to_f32(s.hd.x & 0xffffu);
    const float dmin = f16_bits_to_f32(s.hd.x >> 16);
    // high nibbles arrive as 16q: fold the 1/16 into the scale
    const float sc_f = d * (float)sc * (hh ? 0.0625f : 1.0f);
    scale = splat((f16)sc_f);
    negmin = splat((f16)(-(dmin * (float)m)));
  } else if constexpr (TYPE == 2) {
    const int hf = t >> 3, g = (t >> 1) & 3;
    const uint32_t k = 8 * hf + (t & 1) + 2 * g;
    const uint32_t wv = k < 4 ? s.sc.x : (k < 8 ? s.sc.y : (k < 12 ? s.sc.z : s.sc.w));
    const int sc = (int)(int8_t)((wv >> (8 * (k & 3))) & 255u);
    const float d = f16_bits_to_f32(s.d);
    scale = splat((f16)(d * (float)sc * (g >= 2 ? 0.0625f : 1.0f)));
    negmin = splat((f16)0.0f);
  } else {
    scale = splat(__builtin_bit_cast(f16, (uint16_t)s.d[t >> 1]));
    negmin = splat((f16)0.0f);
  }
}

// Activations of one stage: TN tokens x nk k, read by 256 threads as 8-k items (token
// n = item / 32, k group g = item % 32).  f32 inputs are kept as f32 until the store so
// the range guard below can rescale them; f16 inputs are staged as they are.
template <int TN, int XHALF>
struct XStage {
  static constexpr int ITEMS = TN * (KC / 8) / 256;
  float4 a[XHALF ? 1 : ITEMS], b[XHALF ? 1 : ITEMS];
  uint4 h[XHALF ? ITEMS : 1];
};

template <int TN, int XHALF>
SK_DEV void load_x(XStage<TN, XHALF> &xr, const void *xv, const uint32_t *xrow, uint32_t x_off,
                   uint32_t x_stride, uint32_t kc, uint32_t nk) {
  const uint32_t tid = threadIdx.x;
#pragma unroll
  for (int it = 0; it < XStage<TN, XHALF>::ITEMS; it++) {
    const uint32_t id = tid + 256 * it;
    const uint32_t n = id >> 5, g = id & 31;
    const bool live = 8 * g < nk;
    const size_t base = (size_t)x_off + (size_t)xrow[n] * x_stride + kc + 8 * g;
    if constexpr (XHALF) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (live) v = *(const uint4 *)((const f16 *)xv + base);
      xr.h[it] = v;
    } else {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
      if (live) {
        const float *xp = (const float *)xv + base;
        a = *(const float4 *)xp;
        b = *(const float4 *)(xp + 4);
      }
      xr.a[it] = a;
      xr.b[it] = b;
    }
  }
}

// f16 range guard.  f16 tops out at 65504; GEMM inputs such as silu(g)*u can exceed it.
// When any value of a token's 256-k stage reaches 2^15, that (token, stage) is staged as
// x * 2^-e (e = exponent(max) - 14, exact) and the stage's products are scaled back by 2^e.
// The per-wave ballot keeps the common case (no large value in the wave) on a fast path.
// exps[n] receives e for each token, flags[wave] whether the wave rescaled anything.
template <int TN, int XHALF>
SK_DEV void store_x(f16 *lds, const XStage<TN, XHALF> &xr, int *exps, uint32_t *flags) {
  const uint32_t tid = threadIdx.x;
  uint32_t any = 0;
#pragma unroll
  for (int it = 0; it < XStage<TN, XHALF>::ITEMS; it++) {
    const uint32_t id = tid + 256 * it;
    uint4 out;
    int e = 0;
    if constexpr (XHALF) {
      const uint4 v = xr.h[it];
      // (x0,x1),(x2,x3) -> (x0,x2),(x1,x3)
      out.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
      out.y = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
      out.z = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
      out.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
    } else {
      float4 a = xr.a[it], b = xr.b[it];
      const float m = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                            fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
      const bool big = !(m < 32768.0f);  // NaN counts as big: keeps the slow path honest
      if (__ballot(big) != 0) {
        float tm = m;
#pragma unroll
        for (int d = 16; d >= 1; d >>= 1) tm = fmaxf(tm, __shfl_xor(tm, d, 32));
        e = tm >= 32768.0f ? (int)((__builtin_bit_cast(uint32_t, tm) >> 23) & 255u) - 127 - 14 : 0;
        const float sc = __builtin_ldexpf(1.0f, -e);
        a = make_float4(a.x * sc, a.y * sc, a.z * sc, a.w * sc);
        b = make_float4(b.x * sc, b.y * sc, b.z * sc, b.w * sc);
        any = 1;
      }
      out.x = as_u32(pack_f16x2(a.x, a.z));
      out.y = as_u32(pack_f16x2(a.y, a.w));
      out.z = as_u32(pack_f16x2(b.x, b.z));
      out.w = as_u32(pack_f16x2(b.y, b.w));
    }
    *(uint4 *)(lds + (id >> 5) * PITCH + 8 * (id & 31)) = out;
    if ((id & 31) == 0) exps[id >> 5] = e;
  }
  if ((tid & 63) == 0) flags[tid >> 6] = any;
}

template <int TYPE, int ACCUM, int MOE, int XHALF>
SK_DEV void matmul_body(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd,
                        const void *x, float *y, const uint32_t *ctl, const MatmulPush &p) {
  constexpr int TN = MOE ? 32 : 64;  // MOE_TILE_COLS / MATMUL_TILE_COLS of this backend
  constexpr int NB = TN / 32;
  __shared__ __attribute__((aligned(16))) f16 xs[2][TN * PITCH];
  __shared__ uint32_t xrow[TN];
  __shared__ uint32_t yrow[TN];
  __shared__ int xexp[2][TN];
  __shared__ uint32_t xflag[2][4];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63, wave = tid >> 6;
  const uint32_t hh = lane >> 5;
  const uint32_t row0 = blockIdx.x * TM;
  const uint32_t e = blockIdx.y;
  const uint32_t n_all = MOE ? ctl[p.table_off + 2 * e] : ctl[2];
  const uint32_t col0 = blockIdx.z * TN;
  if (col0 >= n_all) return;
  const uint32_t n_tok = min(n_all - col0, (uint32_t)TN);
  const uint32_t list = p.list_off + col0 + (MOE ? ctl[p.table_off + 2 * e + 1] : 0);
  if (tid < TN) {
    const uint32_t i = min(tid, n_tok - 1);
    const uint32_t slot = MOE ? ctl[list + i] : col0 + i;
    xrow[tid] = MOE ? slot / p.x_div : slot;
    yrow[tid] = slot;
  }
  __syncthreads();

  const uint32_t my_row = row0 + wave * 32 + (lane & 31);
  const uint32_t wrow = (MOE ? e * p.n_out : 0) + min(my_row, p.n_out - 1);

  f32x16 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int i = 0; i < 16; i++) acc[j][i] = 0.0f;

  const uint32_t n_stage = (p.n_in + KC - 1) / KC;
  WStage<TYPE> ws;
  {
    XStage<TN, XHALF> x0;
    load_x<TN, XHALF>(x0, x, xrow, p.x_off, p.x_stride, 0, min(p.n_in, (uint32_t)KC));
    load_stage<TYPE>(ws, w, wd, p, wrow, 0, min(p.n_in, (uint32_t)KC));
    store_x<TN, XHALF>(xs[0], x0, xexp[0], xflag[0]);
  }
  __syncthreads();

  for (uint32_t st = 0; st < n_stage; st++) {
    const uint32_t kc = st * KC;
    const uint32_t nk = min(p.n_in - kc, (uint32_t)KC);
    const uint32_t buf = st & 1;
    const f16 *cur = xs[buf];
    WStage<TYPE> wn;
    XStage<TN, XHALF> xn;
    const bool more = st + 1 < n_stage;
    if (more) {
      const uint32_t kn = kc + KC;
      load_stage<TYPE>(wn, w, wd, p, wrow, kn, min(p.n_in - kn, (uint32_t)KC));
      load_x<TN, XHALF>(xn, x, xrow, p.x_off, p.x_stride, kn, min(p.n_in - kn, (uint32_t)KC));
    }
    const int steps = (int)(nk >> 4);
    // f16 rows never rescale (store_x leaves the flags 0): the check compiles away
    const bool rescaled = !XHALF && (xflag[buf][0] | xflag[buf][1] | xflag[buf][2] | xflag[buf][3]) != 0;
    auto run = [&](f32x16 *dst) {
#pragma unroll
      for (int t = 0; t < 16; t++) {
        if (t < steps) {
          f16x2 sc, nm;
          step_scale<TYPE>(ws, t, hh, sc, nm);
          const f16x8 wf = weight_frag<TYPE>(ws, t, hh, sc, nm);
          const uint32_t ko = koff<TYPE>(t, hh);
#pragma unroll
          for (int j = 0; j < NB; j++) {
            const f16x8 xf = *(const f16x8 *)(cur + (32 * j + (lane & 31)) * PITCH + ko);
            dst[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xf, wf, dst[j], 0, 0, 0);
          }
        }
      }
    };
    if (!rescaled) {
      run(acc);
    } else {
      f32x16 part[NB];
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < 16; i++) part[j][i] = 0.0f;
      run(part);
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const uint32_t tok = 32 * j + 8 * (i >> 2) + 4 * hh + (i & 3);
          acc[j][i] += __builtin_ldexpf(part[j][i], xexp[buf][tok]);
        }
    }
    if (more) {
      store_x<TN, XHALF>(xs[buf ^ 1], xn, xexp[buf ^ 1], xflag[buf ^ 1]);
      ws = wn;
    }
    __syncthreads();
  }

  // D[token][row]: lane l holds row l%32, tokens 8(i/4) + 4(l/32) + i%4 of block j
  if (my_row < p.n_out) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t tok = 32 * j + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (tok < n_tok) {
          float *o = y + p.y_off + (size_t)yrow[tok] * p.y_stride + my_row;
          *o = ACCUM ? *o + acc[j][i] : acc[j][i];
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// Dense prefill tile: 128 rows x 128 tokens (MATMUL_TILE_COLS = 128), eight waves of
// 32 rows x 64 tokens (two per SIMD, so one wave's dequantisation overlaps the other's MFMAs).
//   * Weights: a super-block (256 k) of raw blocks per lane, prefetched one super-block
//     ahead; scale/min products decoded once per super-block; fragments dequantised per
//     16-k step as in weight_frag.
//   * Activations: 128-k chunks (eight steps) staged in LDS as f16; the next chunk's loads
//     are in flight in registers while the current one runs on the matrix cores.
//   * Tile order is XCD-aware (see below).
//   * f16 range guard per (token, 128-k chunk): a chunk holding |x| >= 2^15 is staged as
//     x * 2^-e (exact), and the wave scales its accumulators by 2^-e before that chunk's
//     MFMAs and by 2^e after (exact for powers of two), so no extra registers are needed.
// ---------------------------------------------------------------------------------------
constexpr int TN2 = 128;            // tokens per tile
constexpr int NT2 = 512;            // threads per dense workgroup (8 waves, 2 per SIMD)
constexpr int KX_W = 256;           // k per activation chunk: K-quant tiles (one super-block)
constexpr int KX_Q8 = 128;          // k per activation chunk: Q8_0 tile (register weights)
constexpr int DL_KX = 64;           // k per activation chunk: direct-to-LDS tile

// 16 B unit slot swizzle of a direct-to-LDS row (128 B rows, 8 units): distinct banks for 16
// consecutive rows in a 256 B bank line and for 8 in a 128 B one
SK_DEV uint32_t dl_swz(uint32_t r) { return (r & 7u) ^ ((r >> 3) & 1u); }
typedef __attribute__((address_space(3))) void dl_lds;
// vmcnt(N), the other counters unconstrained (gfx9 s_waitcnt encoding)
template <int N>
SK_DEV void dl_wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}
template <int KX>
constexpr int pitch2() { return KX + 8; }  // f16 per staged token row (16 B pad)

// Per-lane scale/min of every step of a super-block, decoded once.
template <int TYPE>
struct StageScales;
template <>
struct StageScales<1> {
  f16x2 sc[4], nm[4];
  __device__ __forceinline__ void get(int t, f16x2 &s, f16x2 &m) const { s = sc[t >> 2]; m = nm[t >> 2]; }
};
template <>
struct StageScales<2> {
  f16x2 sc[16];
  __device__ __forceinline__ void get(int t, f16x2 &s, f16x2 &m) const { s = sc[t]; m = splat((f16)0.0f); }
};
template <>
struct StageScales<0> {
  f16x2 sc[8];
  __device__ __forceinline__ void get(int t, f16x2 &s, f16x2 &m) const { s = sc[t >> 1]; m = splat((f16)0.0f); }
};

template <int TYPE>
SK_DEV void stage_scales(const WStage<TYPE> &s, uint32_t hh, StageScales<TYPE> &o) {
  if constexpr (TYPE == 1) {
#pragma unroll
    for (int c = 0; c < 4; c++) step_scale<1>(s, 4 * c, hh, o.sc[c], o.nm[c]);
  } else if constexpr (TYPE == 2) {
#pragma unroll
    for (int t = 0; t < 16; t++) {
      f16x2 m;
      step_scale<2>(s, t, hh, o.sc[t], m);
    }
  } else {
#pragma unroll
    for (int b = 0; b < 8; b++) {
      f16x2 m;
      step_scale<0>(s, 2 * b, hh, o.sc[b], m);
    }
  }
}

// One KX-k activation chunk of the tile.  f32 inputs: item J = tid + 512 i is 4 values,
// token J / (KX/4), values 4 (J % (KX/4)) + [0, 4) of the chunk, so a load instruction
// reads whole token rows with 16 consecutive bytes per lane.  f16 inputs: item = 8 values
// (16 B), token J / (KX/8).  Either way the LDS row holds pairs (0,2),(1,3) of every four
// values, the order of the packed-quant extraction.
template <int KX, int XHALF, int NT, int TN = TN2>
struct XChunk {
  static constexpr int PER = XHALF ? 8 : 4;              // values per item
  static constexpr int IPT = TN * KX / PER / NT;         // items per thread
  static constexpr int IPR = KX / PER;                   // items per token row
  float4 v[XHALF ? 1 : IPT];
  uint4 h[XHALF ? IPT : 1];
};

// LIVE (expert groups): token rows past `live` (the group's last tile pads its 32 columns
// with copies of its last row) read zeros without touching memory; their columns are not
// stored.  f16 rows: a raw buffer load over the rows from x_off, whose offset for a padding
// row lies past the resource's end.  f32 rows: the padding rows are not loaded and keep the
// chunk's contents, which the caller zeroes once before its first load.  A branch around
// the load or zeros written here, in the loop, made every chunk wait for all loads in
// flight, the next stage's weights included, before issuing its own.
template <int KX, int XHALF, int NT, int TN, bool LIVE = false>
SK_DEV void load_chunk(XChunk<KX, XHALF, NT, TN> &c, const void *xv, const uint32_t *xrow, uint32_t x_off,
                       uint32_t x_stride, uint32_t k0, uint32_t n_in, uint32_t live = 0) {
  using C = XChunk<KX, XHALF, NT, TN>;
  constexpr int IPT = C::IPT, IPR = C::IPR, PER = C::PER;
#pragma unroll
  for (int i = 0; i < IPT; i++) {
    const uint32_t J = threadIdx.x + NT * i;
    const uint32_t kb = k0 + PER * (J % IPR);
    // load unconditionally from a clamped, in-bounds address; values past n_in are zeroed
    // when the chunk is stored (a select here would make the loads wait at once, and a
    // predicated load is split into per-dword branches)
    const size_t base = (size_t)x_off + (size_t)xrow[J / IPR] * x_stride + (kb < n_in ? kb : n_in - PER);
    if constexpr (LIVE && XHALF) {
      const BufRes xr = buf_res((const f16 *)xv + x_off, 0x7fffffffull);
      const uint32_t off = J / IPR < live && kb < n_in ? 2u * (uint32_t)(base - x_off) : 0x80000000u;
      c.h[i] = buf_load(xr, off, 0);
    } else if constexpr (XHALF) {
      c.h[i] = *(const uint4 *)((const f16 *)xv + base);
    } else if (!LIVE || J / IPR < live) {
      c.v[i] = *(const float4 *)((const float *)xv + base);
    }
  }
}

template <int KX, int XHALF, int NT, int TN>
SK_DEV void zero_chunk(XChunk<KX, XHALF, NT, TN> &c) {
  using C = XChunk<KX, XHALF, NT, TN>;
#pragma unroll
  for (int i = 0; i < (XHALF ? C::IPT : 1); i++) c.h[i] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
  for (int i = 0; i < (XHALF ? 1 : C::IPT); i++) c.v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

// Stores a chunk to LDS, pair-permuted as the weight fragments; returns whether this
// wave rescaled any token.
template <int KX, int XHALF, int NT, int TN>
SK_DEV bool store_chunk(f16 *lds, XChunk<KX, XHALF, NT, TN> &c, int *exps, uint32_t k0, uint32_t n_in) {
  using C = XChunk<KX, XHALF, NT, TN>;
  constexpr int IPT = C::IPT, IPR = C::IPR, PER = C::PER;
  constexpr int PITCH2 = pitch2<KX>();
  if (k0 + KX > n_in) {  // partial chunk (Q8_0 tail): zero the values past n_in
#pragma unroll
    for (int i = 0; i < IPT; i++) {
      const bool live = k0 + PER * ((threadIdx.x + NT * i) % IPR) < n_in;
      if constexpr (XHALF) {
        if (!live) c.h[i] = make_uint4(0, 0, 0, 0);
      } else if (!live) {
        c.v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  }
  bool any = false;
  if constexpr (!XHALF) {
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < IPT; i++)
      m = fmaxf(m, fmaxf(fmaxf(fabsf(c.v[i].x), fabsf(c.v[i].y)), fmaxf(fabsf(c.v[i].z), fabsf(c.v[i].w))));
    any = __ballot(!(m < 32768.0f)) != 0;  // NaN counts as big
  }
#pragma unroll
  for (int i = 0; i < IPT; i++) {
    const uint32_t J = threadIdx.x + NT * i;
    const uint32_t n = J / IPR, kq = J % IPR;
    if constexpr (XHALF == 2) {  // x_half_rows wrote the rows pair-permuted already
      *(uint4 *)(lds + n * PITCH2 + 8 * kq) = c.h[i];
      if (kq == 0) exps[n] = 0;
    } else if constexpr (XHALF) {
      const uint4 v = c.h[i];
      uint4 o;
      o.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
      o.y = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
      o.z = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
      o.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
      *(uint4 *)(lds + n * PITCH2 + 8 * kq) = o;
      if (kq == 0) exps[n] = 0;
    } else {
      float4 a = c.v[i];
      int e = 0;
      if (any) {  // wave-uniform slow path: the token's max over its IPR lanes
        float tm = fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w)));
#pragma unroll
        for (int d = IPR / 2; d >= 1; d >>= 1) tm = fmaxf(tm, __shfl_xor(tm, d, 64));
        e = tm >= 32768.0f ? (int)((__builtin_bit_cast(uint32_t, tm) >> 23) & 255u) - 127 - 14 : 0;
        const float sc = __builtin_ldexpf(1.0f, -e);
        a = make_float4(a.x * sc, a.y * sc, a.z * sc, a.w * sc);
      }
      // values k0..k3 = a.xyzw -> pairs (0,2),(1,3)
      *(uint2 *)(lds + n * PITCH2 + 4 * kq) =
          make_uint2(as_u32(pack_f16x2(a.x, a.z)), as_u32(pack_f16x2(a.y, a.w)));
      if (kq == 0) exps[n] = e;
    }
  }
  return any;
}

// K-quant weights of one 256-k stage, staged in LDS once per workgroup: the 128 rows'
// raw block bytes are loaded with whole-line 16 B loads (8 or 13 lanes per row) and every
// lane then reads the 8 bytes it dequantises per step from LDS.  Rows are PW bytes apart
// (PW/4 odd multiple of 2 dwords), so the 32 rows a wave reads hit distinct bank pairs.
// NT threads share the loads (NT >= 256).
template <int TYPE, int NT>
struct WLds;
template <int NT>
struct WLds<1, NT> {  // Q4_K row: qs 128 | header 16
  static constexpr uint32_t PW = 152;
  static constexpr int QI = TM * 8 / NT;  // qs units per thread
  uint4 q[QI], hd;
  SK_DEV void load(WLds &r, const uint4 *w, const MatmulPush &p, uint32_t row0, uint32_t sb, uint32_t tid,
                   uint32_t base = 0) {
    const uint32_t units = p.n_in >> 5, supers = p.n_in >> 8;
#pragma unroll
    for (int i = 0; i < QI; i++) {
      const uint32_t u = tid + NT * i, lr = u >> 3;
      r.q[i] = w[p.o0 + (base + min(row0 + lr, p.n_out - 1)) * units + sb * 8 + (u & 7)];
    }
    if (tid < TM) r.hd = w[p.o1 + (base + min(row0 + tid, p.n_out - 1)) * supers + sb];
  }
  SK_DEV void store(const WLds &r, uint32_t *lds, uint32_t tid) {
#pragma unroll
    for (int i = 0; i < QI; i++) {
      const uint32_t u = tid + NT * i, lr = u >> 3;
      uint2 *d = (uint2 *)(lds + (lr * PW + 16 * (u & 7)) / 4);
      d[0] = make_uint2(r.q[i].x, r.q[i].y);
      d[1] = make_uint2(r.q[i].z, r.q[i].w);
    }
    if (tid < TM) {
      uint2 *d = (uint2 *)(lds + (tid * PW + 128) / 4);
      d[0] = make_uint2(r.hd.x, r.hd.y);
      d[1] = make_uint2(r.hd.z, r.hd.w);
    }
  }
};
template <int NT>
struct WLds<2, NT> {  // Q6_K row: ql 128 | qh 64 | scales 16 | d 2
  static constexpr uint32_t PW = 216;
  static constexpr int LI = TM * 8 / NT, HI = TM * 4 / NT;  // ql / qh units per thread
  uint4 ql[LI], qh[HI], sc;
  uint32_t d;
  SK_DEV void load(WLds &r, const uint4 *w, const uint16_t *wd, const MatmulPush &p, uint32_t row0,
                   uint32_t sb, uint32_t tid, uint32_t base = 0) {
    const uint32_t supers = p.n_in >> 8;
#pragma unroll
    for (int i = 0; i < LI; i++) {
      const uint32_t u = tid + NT * i, lr = u >> 3;
      r.ql[i] = w[p.o0 + ((base + min(row0 + lr, p.n_out - 1)) * supers + sb) * 8 + (u & 7)];
    }
#pragma unroll
    for (int i = 0; i < HI; i++) {
      const uint32_t u = tid + NT * i, lr = u >> 2;
      r.qh[i] = w[p.o1 + ((base + min(row0 + lr, p.n_out - 1)) * supers + sb) * 4 + (u & 3)];
    }
    const uint32_t lr = tid & (TM - 1);
    const uint32_t rs = (base + min(row0 + lr, p.n_out - 1)) * supers + sb;
    if (tid < TM) r.sc = w[p.o2 + rs];
    else if (tid < 2 * TM) r.d = wd[p.o3 + rs];
  }
  SK_DEV void store(const WLds &r, uint32_t *lds, uint32_t tid) {
#pragma unroll
    for (int i = 0; i < LI; i++) {
      const uint32_t u = tid + NT * i, lr = u >> 3;
      uint2 *d = (uint2 *)(lds + (lr * PW + 16 * (u & 7)) / 4);
      d[0] = make_uint2(r.ql[i].x, r.ql[i].y);
      d[1] = make_uint2(r.ql[i].z, r.ql[i].w);
    }
#pragma unroll
    for (int i = 0; i < HI; i++) {
      const uint32_t u = tid + NT * i, lr = u >> 2;
      uint2 *d = (uint2 *)(lds + (lr * PW + 128 + 16 * (u & 3)) / 4);
      d[0] = make_uint2(r.qh[i].x, r.qh[i].y);
      d[1] = make_uint2(r.qh[i].z, r.qh[i].w);
    }
    const uint32_t lr = tid & (TM - 1);
    if (tid < TM) {
      uint2 *d = (uint2 *)(lds + (lr * PW + 192) / 4);
      d[0] = make_uint2(r.sc.x, r.sc.y);
      d[1] = make_uint2(r.sc.z, r.sc.w);
    } else if (tid < 2 * TM) {
      lds[(lr * PW + 208) / 4] = r.d;
    }
  }
};

// Expert groups: the same stage loads (WLds layout), read through buffer resources over
// this expert's slice of each tensor.  A thread's offsets are fixed and a stage adds a
// scalar offset; a stage past the last, and a wave that owns none of a load's rows, read
// through a resource of no bytes, which returns zeros without touching memory.  Every load
// is thus one unconditional instruction: with the loads inside branches, the compiler's
// in-order load counting merged the paths and waited for every load in flight (the next
// stage's included) at each use.
template <int TYPE, int NT>
struct WBuf;
template <int NT>
struct WBuf<1, NT> {
  using R = WLds<1, NT>;
  BufRes rq, rh, none;
  uint32_t vq[R::QI], vh;
  bool hwave;  // waves 0, 1: the header loads (rows tid < TM)
  __device__ __forceinline__ WBuf(const uint4 *w, const MatmulPush &p, uint32_t base, uint32_t row0, uint32_t tid) {
    const uint32_t units = p.n_in >> 5, supers = p.n_in >> 8;
    rq = buf_res(w + p.o0 + (size_t)base * units, (uint64_t)p.n_out * units * 16);
    rh = buf_res(w + p.o1 + (size_t)base * supers, (uint64_t)p.n_out * supers * 16);
    none = buf_res(nullptr, 0);
#pragma unroll
    for (int i = 0; i < R::QI; i++) {
      const uint32_t u = tid + NT * i;
      vq[i] = (min(row0 + (u >> 3), p.n_out - 1) * units + (u & 7)) * 16;
    }
    vh = min(row0 + (tid & (TM - 1)), p.n_out - 1) * supers * 16;
    hwave = __builtin_amdgcn_readfirstlane(tid >> 6) < (uint32_t)(TM / 64);
  }
  __device__ __forceinline__ void load(R &r, uint32_t sb, bool live) const {
    const BufRes q = live ? rq : none, h = live && hwave ? rh : none;
#pragma unroll
    for (int i = 0; i < R::QI; i++) r.q[i] = buf_load(q, vq[i], sb * 128);
    r.hd = buf_load(h, vh, sb * 16);
  }
};
template <int NT>
struct WBuf<2, NT> {
  using R = WLds<2, NT>;
  BufRes rl, rq, rs, rd, none;
  uint32_t vl[R::LI], vq[R::HI], vs, vd;
  bool swave, dwave;  // waves 0, 1: the scales (rows tid < TM); waves 2, 3: the d (tid - TM)
  __device__ __forceinline__ WBuf(const uint4 *w, const uint16_t *wd, const MatmulPush &p, uint32_t base, uint32_t row0,
              uint32_t tid) {
    const uint32_t supers = p.n_in >> 8;
    const uint64_t rows = (uint64_t)p.n_out * supers;  // (row, super-block) pairs of the expert
    rl = buf_res(w + p.o0 + (size_t)base * supers * 8, rows * 128);
    rq = buf_res(w + p.o1 + (size_t)base * supers * 4, rows * 64);
    rs = buf_res(w + p.o2 + (size_t)base * supers, rows * 16);
    rd = buf_res(wd + p.o3 + (size_t)base * supers, rows * 2);
    none = buf_res(nullptr, 0);
#pragma unroll
    for (int i = 0; i < R::LI; i++) {
      const uint32_t u = tid + NT * i;
      vl[i] = (min(row0 + (u >> 3), p.n_out - 1) * supers * 8 + (u & 7)) * 16;
    }
#pragma unroll
    for (int i = 0; i < R::HI; i++) {
      const uint32_t u = tid + NT * i;
      vq[i] = (min(row0 + (u >> 2), p.n_out - 1) * supers * 4 + (u & 3)) * 16;
    }
    const uint32_t rr = min(row0 + (tid & (TM - 1)), p.n_out - 1) * supers;
    vs = rr * 16;
    vd = rr * 2;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    swave = wv < (uint32_t)(TM / 64);
    dwave = !swave && wv < (uint32_t)(2 * TM / 64);
  }
  __device__ __forceinline__ void load(R &r, uint32_t sb, bool live) const {
    const BufRes l = live ? rl : none, q = live ? rq : none;
    const BufRes sc = live && swave ? rs : none, d = live && dwave ? rd : none;
#pragma unroll
    for (int i = 0; i < R::LI; i++) r.ql[i] = buf_load(l, vl[i], sb * 128);
#pragma unroll
    for (int i = 0; i < R::HI; i++) r.qh[i] = buf_load(q, vq[i], sb * 64);
    r.sc = buf_load(sc, vs, sb * 16);
    r.d = __builtin_amdgcn_raw_buffer_load_b16(d, vd, sb * 2, 0);
  }
};

template <int TYPE, int NT>
SK_DEV WBuf<TYPE, NT> make_wbuf(const uint4 *w, const uint16_t *wd, const MatmulPush &p, uint32_t base,
                                uint32_t row0, uint32_t tid) {
  if constexpr (TYPE == 1) {
    (void)wd;
    return WBuf<1, NT>(w, p, base, row0, tid);
  } else {
    return WBuf<2, NT>(w, wd, p, base, row0, tid);
  }
}

// Q4_K fragment of lane half hh from the 8 qs bytes of its step (same arithmetic as
// weight_frag): low nibbles for hh = 0, high nibbles (16q, the 1/16 is in the scale) for 1.
SK_DEV f16x8 q4k_frag(uint2 v, uint32_t hh, f16x2 scale, f16x2 negmin) {
  const uint32_t M = 0x64006400u;
  const uint32_t mask = hh ? 0x00f000f0u : 0x000f000fu;
  const f16x2 off = splat((f16)-1024.0f);
  const uint32_t a = (v.x & mask) | M, b = ((v.x >> 8) & mask) | M;
  const uint32_t e = (v.y & mask) | M, f = ((v.y >> 8) & mask) | M;
  f16x2 w0 = __builtin_elementwise_fma(as_f16x2(a) + off, scale, negmin);
  f16x2 w1 = __builtin_elementwise_fma(as_f16x2(b) + off, scale, negmin);
  f16x2 w2 = __builtin_elementwise_fma(as_f16x2(e) + off, scale, negmin);
  f16x2 w3 = __builtin_elementwise_fma(as_f16x2(f) + off, scale, negmin);
  f16x8 r = {w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
  return r;
}

// Q6_K fragment of step t from its 8 ql bytes l and 8 qh bytes h (same arithmetic as
// weight_frag): quant groups g >= 2 take the high nibbles (16q, the 1/16 is in the scale).
SK_DEV f16x8 q6k_frag(uint2 l, uint2 h, int t, f16x2 scale) {
  const uint32_t M = 0x64006400u;
  const int g = (t >> 1) & 3;
  const uint32_t lmask = (g >= 2) ? 0x00f000f0u : 0x000f000fu;
  const uint32_t hmask = (g >= 2) ? 0x03000300u : 0x00300030u;
  const int hs = 4 - 2 * (g & 1);
  auto q6 = [&](uint32_t lv, uint32_t hv) -> uint32_t { return (lv & lmask) | M | ((hv << hs) & hmask); };
  const f16x2 off = splat((g >= 2) ? (f16)-1536.0f : (f16)-1056.0f);
  f16x2 w0 = (as_f16x2(q6(l.x, h.x)) + off) * scale;
  f16x2 w1 = (as_f16x2(q6(l.x >> 8, h.x >> 8)) + off) * scale;
  f16x2 w2 = (as_f16x2(q6(l.y, h.y)) + off) * scale;
  f16x2 w3 = (as_f16x2(q6(l.y >> 8, h.y >> 8)) + off) * scale;
  f16x8 r = {w0.x, w0.y, w1.x, w1.y, w2.x, w2.y, w3.x, w3.y};
  return r;
}

// Fragment of step t for lane half hh from the LDS row (same arithmetic as weight_frag).
template <int TYPE>
SK_DEV f16x8 lds_frag(const uint32_t *row, int t, uint32_t hh, f16x2 scale, f16x2 negmin) {
  if constexpr (TYPE == 1) {
    return q4k_frag(*(const uint2 *)(row + 2 * t), hh, scale, negmin);  // qs bytes [8t, 8t + 8)
  } else {
    const int hf = t >> 3, g = (t >> 1) & 3;
    const uint32_t l0 = 16 * (t & 1) + 8 * hh;
    const uint2 l = *(const uint2 *)(row + (hf * 64 + ((g & 1) ? 32 : 0) + l0) / 4);
    const uint2 h = *(const uint2 *)(row + (128 + hf * 32 + l0) / 4);
    (void)negmin;
    return q6k_frag(l, h, t, scale);
  }
}

// Stage scales of a lane from its LDS row (header / scales + d), as stage_scales.
template <int TYPE>
SK_DEV void lds_scales(const uint32_t *row, uint32_t hh, StageScales<TYPE> &o) {
  WStage<TYPE> s;
  if constexpr (TYPE == 1) {
    const uint2 a = *(const uint2 *)(row + 32), b = *(const uint2 *)(row + 34);
    s.hd = make_uint4(a.x, a.y, b.x, b.y);
  } else {
    const uint2 a = *(const uint2 *)(row + 48), b = *(const uint2 *)(row + 50);
    s.sc = make_uint4(a.x, a.y, b.x, b.y);
    s.d = row[52] & 0xffffu;
  }
  stage_scales<TYPE>(s, hh, o);
}

// Dense tile with LDS-staged K-quant weights (Q4_K, Q6_K), 128 rows x 128 tokens.
//   NW = 8: waves of 32 rows x 64 tokens (two per SIMD), 256-k activation chunks.
//   NW = 4: waves of 32 rows x all 128 tokens, 128-k chunks: each dequantised weight
//     fragment feeds four MFMAs instead of two (half the VALU per MFMA) and the ~54 KB of
//     LDS lets two workgroups share a CU.
// K split: with S > 1, grid.z = token tiles x S and workgroup (row tile, token tile, split)
// runs its share of the super-blocks.  Each writes its f32 partial tile to `ws` with
// coherent (sc1) stores, drains them, and counts itself in cnt[tile]; the last of the S
// sums the partials in split order (deterministic) and writes y, then resets the count
// for the next launch.  No workgroup ever waits for another.
// Balanced grid (HYB): grid.x = hf + 2 (tiles - hf) workgroups for a launch of more tiles
// than one round of workgroup slots holds; workgroup b < hf runs tile b whole, the others
// run tile hf + (b - hf) / 2 in two K halves (ws and cnt indexed from tile hf), so every CU
// gets about the same work; hz token tiles per row tile.
// Segments (SEG): up to four matrices on the same rows in one launch (the runtime fuses
// matmuls with no barrier between them that read the same activations); the row tiles of
// segment s follow those of segment s - 1, and each takes its own push words (regions,
// y_off, n_out, y_stride); x_off, n_in and x_stride are the same for all.
// Per-lane state of the direct-to-LDS tile: buffer resources, this lane's load offsets
// (activation pieces, weight pieces) and its read swizzles.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Weight stage layout of the direct-to-LDS tile (byte offsets in one stage buffer; each
// region is whole 1 KiB blocks, loaded block by block, one 16 B piece per lane):
//   Q4_K, 18 blocks: qs rows (128 B) at 128 r, headers (16 B) at 16384 + 16 r
//   Q6_K, 28 blocks: ql rows (128 B) at 128 r, qh rows (64 B) at 16384 + 64 r, scales (16 B)
//                    at 24576 + 16 r, and at 26624 + 16 r the 16 B-aligned 16 B that hold the
//                    row's d (at byte dpos: regions and buffers are 16 B-aligned, so those
//                    16 B lie inside the buffer)
template <int TYPE>
constexpr uint32_t dl_wblocks() {
  return TYPE == 1 ? 18 : 28;
}
// 16 B unit slot swizzle of a 64 B qh row (4 units): the 8 B reads of 32 rows at one
// position meet at most twice on a bank (64 or 32 banks)
SK_DEV uint32_t dl_swz4(uint32_t r) { return ((r >> 1) ^ (r >> 3)) & 3u; }

// Per-lane state of the direct-to-LDS tile: buffer resources, this lane's load offsets for
// its activation blocks (wave + NW i) and weight blocks (the same), the bytes a weight
// block's source moves per super-block, and the read swizzles.
template <int NW, int TYPE, int TN = TN2>
struct DLLanes {
  static constexpr int XS = TN / 8 / NW;                                 // activation blocks per wave
  static constexpr int WS = (dl_wblocks<TYPE>() + NW - 1) / NW;      // weight block slots per wave
  static constexpr int WMIN = dl_wblocks<TYPE>() / NW;               // weight loads of every wave
  static_assert(XS >= 1 && XS * NW * 8 == TN, "whole 1 KiB activation blocks per wave");
  u32x4 xres, wres, dres, nres;  // nres: no bytes (every load past its end reads zeros)
  uint32_t xo[XS], wo[WS], wm[WS];
  uint32_t wv, lane, lrow, hh, tb, wsw, wsw4, xsw;
  uint32_t dpos0;  // Q6_K: byte offset of this lane's row's d at super-block 0
};

// Buffer resource words over [base, base + bytes) (as buf_res builds them: stride 0, raw
// 32-bit data), for the loads below, which take it as an SGPR quad.
SK_DEV u32x4 dl_res(const void *base, uint64_t bytes) {
  const uint64_t a = (uint64_t)base;
  u32x4 r = {(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, (uint32_t)(bytes < 0xffffffffull ? bytes : 0xffffffffull),
             0x00020000u};
  return r;
}
// One 16 B-per-lane buffer load into LDS: lane l's 16 B land at byte lds + 16 l (wave-
// uniform lds, in M0); a load past the resource's end writes zeros.  Written as assembly on
// purpose: with the compiler's own form of this load, every later LDS read waits until all
// such loads in flight are done (the compiler cannot tell which LDS bytes they write),
// which serialises the double buffering; here the explicit waits of dl_stage order each
// buffer's loads before its reads, and the compiler's own waits (it does not count these
// loads) can only wait longer than needed, never less.
// (m0 is declared clobbered; the compiler warns that it reserves m0, which these kernels
// use for nothing else)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
SK_DEV void dl_load16(const u32x4 &res, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(res), "s"(soff)
               : "memory", "m0");
}
#pragma clang diagnostic pop
SK_DEV uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)(dl_lds *)p; }

// Source of weight block b for this lane: byte offset (super-block 0) and bytes per
// super-block, with rows past n_out clamped to the last row.
template <int TYPE>
SK_DEV void dl_wpiece(uint32_t b, uint32_t lane, const MatmulPush &p, uint32_t row0, uint32_t &off, uint32_t &per) {
  const uint32_t supers = p.n_in >> 8, last = p.n_out - 1;
  auto R = [&](uint32_t r) { return min(row0 + r, last); };
  if (b < 16) {  // qs / ql: 8 rows, lane = 8 r + unit slot
    const uint32_t r = 8 * b + (lane >> 3);
    off = 16u * (p.o0 + R(r) * supers * 8 + ((lane & 7) ^ dl_swz(r)));
    per = 128;
  } else if (TYPE == 1) {  // headers: 64 rows
    off = 16u * (p.o1 + R(64 * (b - 16) + lane) * supers);
    per = 16;
  } else if (b < 24) {  // qh: 16 rows, lane = 4 r + unit slot
    const uint32_t r = 16 * (b - 16) + (lane >> 2);
    off = 16u * (p.o1 + R(r) * supers * 4 + ((lane & 3) ^ dl_swz4(r)));
    per = 64;
  } else if (b < 26) {  // scales: 64 rows
    off = 16u * (p.o2 + R(64 * (b - 24) + lane) * supers);
    per = 16;
  } else {  // d: 64 rows (the 16 B-aligned piece that holds d: see dl_issue_w)
    off = 2u * (p.o3 + R(64 * (b - 26) + lane) * supers);
    per = 2;
  }
}

// A 64-k activation chunk (at k) into buffer dst.
template <int NW, int TYPE, int TN>
SK_DEV void dl_issue_x(const DLLanes<NW, TYPE, TN> &L, f16 *__restrict__ dst, uint32_t k) {
#pragma unroll
  for (int i = 0; i < L.XS; i++) dl_load16(L.xres, lds_addr(dst + (NW * i + L.wv) * 512), L.xo[i], 2u * k);
}
// The weights of super-block sb into buffer dst.
template <int NW, int TYPE, int TN>
SK_DEV void dl_issue_w(const DLLanes<NW, TYPE, TN> &L, uint32_t *__restrict__ dst, uint32_t sb) {
#pragma unroll
  for (int i = 0; i < L.WS; i++) {
    const uint32_t b = NW * i + L.wv;
    if (i < L.WMIN || b < dl_wblocks<TYPE>()) {
      if (TYPE == 2 && b >= 26)  // d: 2 B-aligned, so the piece is the aligned 16 B around it
        dl_load16(L.dres, lds_addr(dst + b * 256), (L.wo[i] + 2u * sb) & ~15u, 0);
      else
        dl_load16(L.wres, lds_addr(dst + b * 256), L.wo[i], L.wm[i] * sb);
    }
  }
}

// One 256-k stage of the direct-to-LDS tile: four 64-k chunks alternating between the
// activation buffers x0 (chunks 0, 2) and x1 (1, 3), weights in wc; the loads of the next
// chunk go to the other activation buffer, and at chunk 0 (when `more`) the next stage's
// weights (super-block nsb) go to wn.  The waits that order a buffer's loads before its
// reads are the explicit ones here (the loads are assembly the compiler does not count).
template <int NW, int TYPE, int NB, int TN>
SK_DEV void dl_stage(const DLLanes<NW, TYPE, TN> &L, f32x16 (&acc)[NB], f16 *__restrict__ x0, f16 *__restrict__ x1,
                     const uint32_t *__restrict__ wc, uint32_t *__restrict__ wn, bool more, uint32_t k0,
                     uint32_t nsb) {
  // (wc holds super-block nsb - 1)
  StageScales<TYPE> ss;
#pragma unroll
  for (int c4 = 0; c4 < KC / DL_KX; c4++) {
    // this wave's loads of chunk c4 (and, at c4 = 0, of the stage's weights) are in LDS; at
    // c4 = 1 the next stage's weight loads, issued after the chunk's, may stay in flight
    if (c4 == 1 && more)
      dl_wait_vm<DLLanes<NW, TYPE, TN>::WMIN>();
    else
      dl_wait_vm<0>();
    __syncthreads();
    if (c4 + 1 < KC / DL_KX)
      dl_issue_x(L, (c4 & 1) ? x0 : x1, k0 + DL_KX * (c4 + 1));
    else if (more)
      dl_issue_x(L, x0, k0 + KC);
    if (c4 == 0) {
      __builtin_amdgcn_sched_barrier(0);  // the weight loads stay behind the chunk's
      if (more) dl_issue_w(L, wn, nsb);
      WStage<TYPE> hs;
      if constexpr (TYPE == 1) {
        hs.hd = *(const uint4 *)(wc + 4096 + 4 * L.lrow);
      } else {
        hs.sc = *(const uint4 *)(wc + 6144 + 4 * L.lrow);
        const uint32_t pos = (L.dpos0 + 2u * (nsb - 1)) & 15u;  // d's byte in its 16 B
        const uint4 dq = *(const uint4 *)(wc + 6656 + 4 * L.lrow);
        const uint32_t dw = pos < 8 ? (pos < 4 ? dq.x : dq.y) : (pos < 12 ? dq.z : dq.w);
        hs.d = (dw >> (8 * (pos & 2))) & 0xffffu;
      }
      stage_scales<TYPE>(hs, L.hh, ss);
    }
    const f16 *xb = (c4 & 1) ? x1 : x0;
    f16x8 xf0[NB], xf1[NB], wf0, wf1;
    auto frags = [&](int ts, f16x8(&xf)[NB], f16x8 &wf) {
      const int t = 4 * c4 + ts;  // chunk c4 holds steps 4 c4 .. 4 c4 + 3 (their koff lie in it)
      f16x2 sc, nm;
      ss.get(t, sc, nm);
      if constexpr (TYPE == 1) {
        wf = q4k_frag(*(const uint2 *)(wc + L.lrow * 32 + 4 * ((t >> 1) ^ L.wsw) + 2 * (t & 1)), L.hh, sc, nm);
      } else {  // ql unit 4 hf + 2 (g & 1) + (t & 1), qh unit 2 hf + (t & 1); lane half hh: bytes 8 hh..
        const int hf = t >> 3, g = (t >> 1) & 3;
        const uint2 l = *(const uint2 *)(wc + L.lrow * 32 + 4 * ((4 * hf + 2 * (g & 1) + (t & 1)) ^ L.wsw) + 2 * L.hh);
        const uint2 h = *(const uint2 *)(wc + 4096 + L.lrow * 16 + 4 * ((2 * hf + (t & 1)) ^ L.wsw4) + 2 * L.hh);
        wf = q6k_frag(l, h, t, sc);
      }
      const uint32_t xu = ((koff<TYPE>(t, L.hh) - DL_KX * c4) >> 3) ^ L.xsw;
#pragma unroll
      for (int j = 0; j < NB; j++)
        xf[j] = *(const f16x8 *)(xb + (32 * (L.tb + j) + (L.lane & 31)) * DL_KX + 8 * xu);
    };
    frags(0, xf0, wf0);
#pragma unroll
    for (int ts = 0; ts < 4; ts++) {
      if (ts + 1 < 4) {
        if (ts & 1)
          frags(ts + 1, xf0, wf0);
        else
          frags(ts + 1, xf1, wf1);
      }
#pragma unroll
      for (int j = 0; j < NB; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16((ts & 1) ? xf1[j] : xf0[j], (ts & 1) ? wf1 : wf0, acc[j],
                                                        0, 0, 0);
    }
  }
}

struct NoSegments {};
template <int TYPE, int ACCUM, int XHALF, int NW, int TN = TN2, int MOE = 0, int HYB = 0, int SEG = 0,
          typename SG = NoSegments>
SK_DEV void matmul_tile128_w(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd, const void *x,
                             float *y, const uint32_t *ctl, const MatmulPush &p0, float *ws = nullptr,
                             uint32_t *cnt = nullptr, uint32_t S = 1, uint32_t hf = 0, uint32_t hz = 1,
                             const SG &segs = SG{}) {
  static_assert(NW == 4 || TN == TN2, "eight waves split a 128-token tile");
  // XHALF = 3: the f16 rows of x_half_rows and the K-quant weights loaded straight into LDS
  constexpr bool DL = XHALF == 3;
  static_assert(!DL || (TYPE != 0 && TN == TN2 && !MOE), "direct-to-LDS form");
  constexpr bool W2 = NW == 8;  // two waves per row block
  constexpr int NT = 64 * NW;
  constexpr int NB = W2 ? 2 : TN / 32;  // 32-token blocks per wave
  constexpr int KX = DL ? DL_KX : (NW == 8 || TN < TN2) ? KX_W : 128, PITCH2 = pitch2<KX>();
  constexpr uint32_t PW = WLds<TYPE, NT>::PW;
  __shared__ __attribute__((aligned(16))) f16 xs[DL ? 2 * TN * DL_KX : TN * PITCH2];
  __shared__ __attribute__((aligned(16))) uint32_t wl[DL ? 2 * 256 * dl_wblocks<TYPE>() : TM * PW / 4];
  __shared__ uint32_t xrow[TN];
  __shared__ uint32_t yrow[TN];
  __shared__ int xexp[TN];
  __shared__ uint32_t xflag[NW];
  __shared__ uint32_t last;

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63, wave = tid >> 6;
  const uint32_t hh = lane >> 5;
  const uint32_t rb = W2 ? (wave & 3) : wave, tb = W2 ? 2 * (wave >> 2) : 0;
  // Tile order: workgroups are dealt to the 8 XCDs round-robin by linear id, and
  // consecutive ids take consecutive token tiles (then splits), so the workgroups of one
  // XCD share a token tile's activations in that XCD's L2.
  // Expert groups (MOE): grid.y = expert e, whose group of (count, start) = table[e] tokens
  // is listed in list[]; tile z takes group tokens [z TN, z TN + TN), token i being slot
  // s = list[start + i] that reads x row s / x_div and writes y row s (matmul.comp:124-150).
  uint32_t rt, tt, sp, kt;  // row tile, token tile, split, the tile's slot in ws / cnt
  if constexpr (HYB) {
    const uint32_t b = blockIdx.x;
    const uint32_t t = b < hf ? b : hf + ((b - hf) >> 1);
    S = b < hf ? 1u : 2u;
    sp = b < hf ? 0u : ((b - hf) & 1u);
    rt = t / hz;
    tt = t % hz;
    kt = t - hf;
  } else {
    const uint32_t gx = gridDim.x, gz = gridDim.z, Z = gz / S;
    const uint32_t lin = blockIdx.x + gx * blockIdx.z;
    const uint32_t rem = lin % gz;
    rt = MOE ? blockIdx.x : lin / gz;
    tt = MOE ? blockIdx.z : rem % Z;
    sp = MOE ? 0 : rem / Z;
    kt = rt * Z + tt;
  }
  // MOE = 2: the tile map entry (grid.y, a multiple of 8).  The XCDs take workgroups
  // round-robin by linear id, so ids of one residue mod 8 walk all the row tiles of one entry
  // before the next: every row tile of an entry (the same slots' activation rows, in every
  // segment) runs on one XCD and reads the rows through its L2 once
  uint32_t ent = blockIdx.y;
  if constexpr (MOE == 2) {
    const uint32_t lin = blockIdx.x + gridDim.x * blockIdx.y, k8 = lin / 8;
    rt = k8 % gridDim.x;
    ent = (k8 / gridDim.x) * 8 + lin % 8;
  }
  MatmulPush p = p0;
  if constexpr (SEG) {  // kt stays the launch-wide tile index (ws and cnt span every segment)
    // field by field, with the (wave-uniform) segment in an SGPR: selecting whole push
    // structs made the compiler copy the table to scratch and index it
    const uint32_t sg = __builtin_amdgcn_readfirstlane(segment_of(segs, rt));
    auto pick = [&](uint32_t MatmulPush::*f) -> uint32_t {
      const uint32_t a = segs.p[0].*f, b = segs.p[1].*f, c = segs.p[2].*f, d = segs.p[3].*f;
      return sg == 0 ? a : sg == 1 ? b : sg == 2 ? c : d;
    };
    p.o0 = pick(&MatmulPush::o0);
    p.o1 = pick(&MatmulPush::o1);
    p.o2 = pick(&MatmulPush::o2);
    p.o3 = pick(&MatmulPush::o3);
    p.y_off = pick(&MatmulPush::y_off);
    p.n_out = pick(&MatmulPush::n_out);
    p.y_stride = pick(&MatmulPush::y_stride);
    rt -= sg == 0 ? 0u : sg == 1 ? segs.start[1] : sg == 2 ? segs.start[2] : segs.start[3];
  }
  uint32_t e = MOE ? blockIdx.y : 0, n_all, lstart;
  if constexpr (MOE == 2) {
    // grid.y walks moe_sort's tile map (TILE_MAP words before the table) instead of every
    // expert times every token tile: the count and this workgroup's entry (e | z << 16,
    // then the expert's list start | its slot count << 16) are read together, so the slots
    // are one dependent load away (an entry past the count is never used; the grid stays
    // within the map: at most 280 entries)
    const uint32_t *map = ctl + p.table_off - TILE_MAP;
    const uint32_t cnt = map[0], va = map[1 + 2 * ent], vb = map[2 + 2 * ent];
    if (ent >= cnt) return;
    e = va & 0xffffu;
    tt = va >> 16;
    lstart = vb & 0xffffu;
    n_all = vb >> 16;
  } else {
    n_all = MOE ? ctl[p.table_off + 2 * e] : ctl[2];
    lstart = MOE ? ctl[p.table_off + 2 * e + 1] : 0;
  }
  const uint32_t base = MOE ? e * p.n_out : 0;
  const uint32_t row0 = rt * TM;
  const uint32_t col0 = tt * TN;
  if (col0 >= n_all) return;
  const uint32_t n_tok = min(n_all - col0, (uint32_t)TN);
  if (tid < TN) {
    const uint32_t i = min(tid, n_tok - 1);
    const uint32_t slot = MOE ? ctl[p.list_off + lstart + col0 + i] : col0 + i;
    xrow[tid] = MOE ? slot / p.x_div : slot;
    yrow[tid] = slot;
  }
  const uint32_t lrow = rb * 32 + (lane & 31);
  const uint32_t my_row = row0 + lrow;
  const uint32_t *wrow = wl + lrow * PW / 4;

  f32x16 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int i = 0; i < 16; i++) acc[j][i] = 0.0f;

  const uint32_t n_stage_all = p.n_in / KC;
  const uint32_t st0 = sp * n_stage_all / S, st1 = (sp + 1) * n_stage_all / S;
  const uint32_t n_stage = st1 - st0;
  const uint32_t n_chunk = n_stage * (KC / KX);
  const uint32_t kbase = st0 * KC;
  if constexpr (DL) {
    // Every operand byte goes from global memory straight into LDS (buffer loads with the
    // LDS bit), double buffered: 64-k activation chunks (128 tokens x 128 B) and 256-k
    // weight stages (the layout at dl_wblocks).  One wave-instruction fills 1 KiB, lane l the
    // 16 B at 16 l, so rows are unpadded and their 16 B units are stored XOR-swizzled.  One
    // barrier per chunk: after it, chunk c + 1 loads into the other activation buffer (last
    // read in chunk c - 1) and, at a stage's first chunk, the next stage's weights into the
    // other weight buffer (last read in the stage before).  vmcnt counts a wave's loads in
    // issue order, so before each barrier a wave waits for its loads of the chunk, letting
    // only the weight loads issued after them stay in flight.
    constexpr uint32_t XB = TN * DL_KX, WB = 256 * dl_wblocks<TYPE>();
    using DL_L = DLLanes<NW, TYPE, TN>;
    DL_L L;
    L.wv = __builtin_amdgcn_readfirstlane(wave);
    L.lane = lane;
    L.lrow = lrow;
    L.hh = hh;
    L.tb = tb;
    L.wsw = dl_swz(lrow);
    L.wsw4 = dl_swz4(lrow);
    L.xsw = dl_swz(lane & 31);
    __syncthreads();  // xrow
    L.xres = dl_res(x, 2ull * ((uint64_t)p.x_off + (uint64_t)n_all * p.x_stride));
    L.wres = dl_res(w, 0xffffffffull);
    // d pieces: the 16 B-aligned 16 B around each d, to the end of the d region's last 16 B
    L.dres = dl_res(wd, (2ull * ((uint64_t)p.o3 + (uint64_t)p.n_out * (p.n_in >> 8)) + 15) & ~15ull);
    L.nres = dl_res(nullptr, 0);
    L.dpos0 = 2u * (p.o3 + min(row0 + lrow, p.n_out - 1) * (p.n_in >> 8));
#pragma unroll
    for (int i = 0; i < DL_L::XS; i++) {
      const uint32_t r = 8 * (NW * i + L.wv) + (lane >> 3);  // token
      L.xo[i] = 2u * (p.x_off + xrow[r] * p.x_stride + 8u * ((lane & 7) ^ dl_swz(r)));
    }
#pragma unroll
    for (int i = 0; i < DL_L::WS; i++) dl_wpiece<TYPE>(NW * i + L.wv, lane, p, row0, L.wo[i], L.wm[i]);
    dl_issue_x(L, xs, kbase);
    dl_issue_w(L, wl, st0);
    for (uint32_t st = 0; st < n_stage; st++) {
      const uint32_t b = st & 1;
      dl_stage<NW, TYPE, NB, TN>(L, acc, xs, xs + XB, wl + b * WB, wl + (b ^ 1) * WB, st + 1 < n_stage,
                                 kbase + KC * st, st0 + st + 1);
    }
  } else if constexpr (MOE != 0 && XHALF == 2) {
    // Expert groups on f16 rows: the stage weights are loaded two stages ahead, alternating
    // between two register sets (WBuf: unconditional buffer loads), and each stage issues
    // the next chunk's activations before the weights of the stage after next, so the waits
    // for the data of stage st + 1 (at the end of stage st) leave those in flight.
    static_assert(KX == KC, "one activation chunk per stage");
    const WBuf<TYPE, NT> wb = make_wbuf<TYPE, NT>(w, wd, p, base, row0, tid);
    WLds<TYPE, NT> wa, wc;
    wb.load(wa, st0, true);
    __syncthreads();  // xrow
    XChunk<KX, XHALF, NT, TN> xn;
    load_chunk<KX, XHALF, NT, TN, true>(xn, x, xrow, p.x_off, p.x_stride, kbase, p.n_in, n_tok);
    wa.store(wa, wl, tid);
    store_chunk<KX, XHALF, NT, TN>(xs, xn, xexp, kbase, p.n_in);
    wb.load(wa, st0 + 1, 1 < n_stage);
    __syncthreads();
    // stage st: `held` holds the weights of stage st + 1, `fill` receives those of st + 2
    auto stage = [&](uint32_t st, WLds<TYPE, NT> &held, WLds<TYPE, NT> &fill) {
      StageScales<TYPE> ss;
      lds_scales<TYPE>(wrow, hh, ss);
      load_chunk<KX, XHALF, NT, TN, true>(xn, x, xrow, p.x_off, p.x_stride, kbase + (st + 1) * KC, p.n_in, n_tok);
      wb.load(fill, st0 + st + 2, st + 2 < n_stage);
      constexpr int SPC = KX / 16;
      f16x8 xf0[NB], xf1[NB], wf0, wf1;
      auto frags = [&](int t, f16x8(&xf)[NB], f16x8 &wf) {
        f16x2 sc, nm;
        ss.get(t, sc, nm);
        wf = lds_frag<TYPE>(wrow, t, hh, sc, nm);
        const uint32_t ko = koff<TYPE>(t, hh);
#pragma unroll
        for (int j = 0; j < NB; j++) xf[j] = *(const f16x8 *)(xs + (32 * (tb + j) + (lane & 31)) * PITCH2 + ko);
      };
      frags(0, xf0, wf0);
#pragma unroll
      for (int ts = 0; ts < SPC; ts++) {
        if (ts + 1 < SPC) {
          if (ts & 1)
            frags(ts + 1, xf0, wf0);
          else
            frags(ts + 1, xf1, wf1);
        }
#pragma unroll
        for (int j = 0; j < NB; j++)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16((ts & 1) ? xf1[j] : xf0[j], (ts & 1) ? wf1 : wf0,
                                                          acc[j], 0, 0, 0);
      }
      __syncthreads();  // every wave is done with this stage's weights and activations
      // stored unconditionally (past the last stage: zeros no one reads), and the stage pairs
      // below run unconditionally, so that on every path the loads a stage waits for are
      // complete at the loop's back edge; with a branch around either, the compiler waited
      // at the top of each pair for the weights issued two stages ahead
      held.store(held, wl, tid);
      store_chunk<KX, XHALF, NT, TN>(xs, xn, xexp, kbase + (st + 1) * KC, p.n_in);
      __syncthreads();
    };
    uint32_t st = 0;
    for (; st + 1 < n_stage; st += 2) {
      stage(st, wa, wc);
      stage(st + 1, wc, wa);
    }
    if (st < n_stage) stage(st, wa, wc);
  } else {
  WLds<TYPE, NT> wr;
  if constexpr (TYPE == 1) wr.load(wr, w, p, row0, st0, tid, base);
  else wr.load(wr, w, wd, p, row0, st0, tid, base);
  __syncthreads();  // xrow
  XChunk<KX, XHALF, NT, TN> xn;  // the chunk in flight; expert groups: padding rows stay zero
  if constexpr (MOE != 0 && !XHALF) zero_chunk(xn);
  load_chunk<KX, XHALF, NT, TN, MOE != 0>(xn, x, xrow, p.x_off, p.x_stride, kbase, p.n_in, n_tok);
  wr.store(wr, wl, tid);
  {
    const bool r = store_chunk<KX, XHALF, NT, TN>(xs, xn, xexp, kbase, p.n_in);
    if (lane == 0) xflag[wave] = r;
  }
  __syncthreads();

  uint32_t chunk = 0;
  for (uint32_t st = 0; st < n_stage; st++) {
    StageScales<TYPE> ss;
    lds_scales<TYPE>(wrow, hh, ss);
    const bool more = st + 1 < n_stage;
    if (more) {
      if constexpr (TYPE == 1) wr.load(wr, w, p, row0, st0 + st + 1, tid, base);
      else wr.load(wr, w, wd, p, row0, st0 + st + 1, tid, base);
    }
#pragma unroll
    for (int c4 = 0; c4 < KC / KX; c4++) {
      const bool next = chunk + 1 < n_chunk;
      if (next)
        load_chunk<KX, XHALF, NT, TN, MOE != 0>(xn, x, xrow, p.x_off, p.x_stride, kbase + (chunk + 1) * KX, p.n_in,
                                                n_tok);
      bool rescaled = false;  // f16 rows never rescale (store_chunk returns false)
      if constexpr (!XHALF)
#pragma unroll
        for (int q = 0; q < NW; q++) rescaled |= xflag[q] != 0;
      if (rescaled) {
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int i = 0; i < 16; i++)
            acc[j][i] = __builtin_ldexpf(acc[j][i], -xexp[32 * (tb + j) + 8 * (i >> 2) + 4 * hh + (i & 3)]);
      }
      constexpr int SPC = KX / 16;
      f16x8 xf0[NB], xf1[NB], wf0, wf1;
      auto frags = [&](int ts, f16x8(&xf)[NB], f16x8 &wf) {
        const int t = SPC * c4 + ts;
        f16x2 sc, nm;
        ss.get(t, sc, nm);
        wf = lds_frag<TYPE>(wrow, t, hh, sc, nm);
        const uint32_t ko = koff<TYPE>(t, hh) - KX * c4;
#pragma unroll
        for (int j = 0; j < NB; j++) xf[j] = *(const f16x8 *)(xs + (32 * (tb + j) + (lane & 31)) * PITCH2 + ko);
      };
      frags(0, xf0, wf0);
#pragma unroll
      for (int ts = 0; ts < SPC; ts++) {
        if (ts + 1 < SPC) {
          if (ts & 1)
            frags(ts + 1, xf0, wf0);
          else
            frags(ts + 1, xf1, wf1);
        }
#pragma unroll
        for (int j = 0; j < NB; j++)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16((ts & 1) ? xf1[j] : xf0[j], (ts & 1) ? wf1 : wf0,
                                                          acc[j], 0, 0, 0);
      }
      if (rescaled) {
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int i = 0; i < 16; i++)
            acc[j][i] = __builtin_ldexpf(acc[j][i], xexp[32 * (tb + j) + 8 * (i >> 2) + 4 * hh + (i & 3)]);
      }
      __syncthreads();  // every wave is done with this chunk (and, at the stage end, the weights)
      if (next) {
        if (c4 == KC / KX - 1 && more) wr.store(wr, wl, tid);
        const bool r = store_chunk<KX, XHALF, NT, TN>(xs, xn, xexp, kbase + (chunk + 1) * KX, p.n_in);
        if (lane == 0) xflag[wave] = r;
        __syncthreads();
      }
      chunk++;
    }
  }
  }

  if (S > 1) {
    const uint32_t tile = kt;
    constexpr uint32_t PART = NW * NB * 16 * 64;  // floats of one partial tile
    float *mine = ws + (size_t)(tile * S + sp) * PART + wave * (NB * 16 * 64);
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int i = 0; i < 16; i++)
        __hip_atomic_store(mine + (j * 16 + i) * 64 + lane, acc[j][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // each wave's partial stores complete before the barrier
    __syncthreads();
    // Release at agent scope: the count is made after this workgroup's partial stores are
    // visible device-wide (buffer_wbl2 sc1 and a wait, by one thread).  Only the last
    // workgroup of a tile reads the partials, with agent-scope loads; a full __threadfence in
    // every workgroup (release and acquire) made the split 2x slower.
    if (tid == 0) last = __hip_atomic_fetch_add(&cnt[tile], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    __syncthreads();
    if (!last) return;
    // No acquire fence here: the partials are read with agent-scope loads (sc1, served past
    // the XCD's non-coherent L2 state) that issue only after the count's result is back and
    // the workgroup has met at the barrier.  An agent-scope acquire (buffer_inv sc1 in the
    // last workgroup of each tile) invalidates the L2 the other workgroups stream through:
    // M = 512 q 51 -> 59 us, config-5 prefill 13.7k -> 12.4k tok/s.
    // The partials added in split order.  Split by split, all of a lane's values are loaded
    // before any is added (a wave-uniform branch per split), so a partial costs one round
    // trip past the L2; a branch per value made the compiler wait for every load in turn
    // (~11 us per partial tile: M = 128, K split 8, 103 -> 41 us).
    float t[NB][16];
    for (uint32_t q = 0; q < S; q++) {
      float v[NB][16];
      if (q == sp) {
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int i = 0; i < 16; i++) v[j][i] = acc[j][i];
      } else {
        const float *src = ws + (size_t)(tile * S + q) * PART + wave * (NB * 16 * 64) + lane;
#pragma unroll
        for (int j = 0; j < NB; j++)
#pragma unroll
          for (int i = 0; i < 16; i++)
            v[j][i] = __hip_atomic_load(src + (j * 16 + i) * 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < 16; i++) t[j][i] = q == 0 ? v[j][i] : t[j][i] + v[j][i];
    }
#pragma unroll
    for (int j = 0; j < NB; j++)
#pragma unroll
      for (int i = 0; i < 16; i++) acc[j][i] = t[j][i];
    if (tid == 0) __hip_atomic_store(&cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (my_row < p.n_out) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t tok = 32 * (tb + j) + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (tok < n_tok) {
          float *o = y + p.y_off + (size_t)yrow[tok] * p.y_stride + my_row;
          float v = acc[j][i];
          // XHALF = 2, 3: the rows came from x_half_rows as x * 2^-e; scale back (exact) by
          // the exponent of the token's input row (its output row for dense launches)
          if constexpr (XHALF >= 2) v = __builtin_ldexpf(v, ((const int *)x)[xrow[tok]]);
          *o = ACCUM ? *o + v : v;
        }
      }
    }
  }
}

template <int TYPE, int ACCUM, int XHALF>
SK_DEV void matmul_tile128(const uint4 *__restrict__ w, const uint16_t *__restrict__ wd, const void *x,
                           float *y, const uint32_t *ctl, const MatmulPush &p) {
  // wave w: rows 32 (w % 4) + [0, 32), tokens 64 (w / 4) + [0, 64) of the tile; the two
  // waves of a row block dequantise the same fragments (VALU) but share one weight stream
  constexpr int NB = 2;
  constexpr int KX = KX_Q8, PITCH2 = pitch2<KX>();
  __shared__ __attribute__((aligned(16))) f16 xs[TN2 * PITCH2];
  __shared__ uint32_t xrow[TN2];
  __shared__ int xexp[TN2];
  __shared__ uint32_t xflag[NT2 / 64];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63, wave = tid >> 6;
  const uint32_t hh = lane >> 5;
  const uint32_t rb = wave & 3, tb = 2 * (wave >> 2);  // row block, first token block
  // Tile order: blocks are dealt to the 8 XCDs round-robin by linear id, so consecutive ids
  // take consecutive token tiles; every workgroup of an XCD then shares one token tile of
  // activations in that XCD's L2 (the row tiles, read once per token tile, stream past).
  const uint32_t gx = gridDim.x, gz = gridDim.z;
  const uint32_t lin = blockIdx.x + gx * blockIdx.z;
  const uint32_t row0 = (lin / gz) * TM;
  const uint32_t n_all = ctl[2];
  const uint32_t col0 = (lin % gz) * TN2;
  if (col0 >= n_all) return;
  const uint32_t n_tok = min(n_all - col0, (uint32_t)TN2);
  if (tid < TN2) xrow[tid] = col0 + min(tid, n_tok - 1);
  __syncthreads();

  const uint32_t my_row = row0 + rb * 32 + (lane & 31);
  const uint32_t wrow = min(my_row, p.n_out - 1);

  f32x16 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int i = 0; i < 16; i++) acc[j][i] = 0.0f;

  const uint32_t n_stage = (p.n_in + KC - 1) / KC;
  const uint32_t n_chunk = (p.n_in + KX - 1) / KX;
  WStage<TYPE> ws;
  load_stage<TYPE>(ws, w, wd, p, wrow, 0, min(p.n_in, (uint32_t)KC));
  {
    XChunk<KX, XHALF, NT2> c0;
    load_chunk<KX, XHALF, NT2>(c0, x, xrow, p.x_off, p.x_stride, 0, p.n_in);
    const bool r = store_chunk<KX, XHALF, NT2>(xs, c0, xexp, 0, p.n_in);
    if (lane == 0) xflag[wave] = r;
  }
  __syncthreads();

  uint32_t chunk = 0;
  for (uint32_t st = 0; st < n_stage; st++) {
    const uint32_t kc = st * KC;
    const uint32_t nk = min(p.n_in - kc, (uint32_t)KC);
    StageScales<TYPE> ss;
    stage_scales<TYPE>(ws, hh, ss);
    WStage<TYPE> wn;
    const bool more = st + 1 < n_stage;
#pragma unroll
    for (int c4 = 0; c4 < KC / KX; c4++) {
      if ((uint32_t)(KX * c4) < nk) {
        // the next chunk is loaded into registers while this one runs from LDS; the next
        // super-block's weights are requested during the stage's last chunk, after it
        XChunk<KX, XHALF, NT2> xn;
        const bool next = chunk + 1 < n_chunk;
        if (next) load_chunk<KX, XHALF, NT2>(xn, x, xrow, p.x_off, p.x_stride, (chunk + 1) * KX, p.n_in);
        if (c4 == KC / KX - 1 && more) load_stage<TYPE>(wn, w, wd, p, wrow, kc + KC, min(p.n_in - kc - KC, (uint32_t)KC));
        bool rescaled = false;  // f16 rows never rescale (store_chunk returns false)
        if constexpr (!XHALF)
#pragma unroll
          for (int q = 0; q < NT2 / 64; q++) rescaled |= xflag[q] != 0;
        const f16 *cur = xs;
        if (rescaled) {  // acc *= 2^-e(token) before this chunk (exact)
#pragma unroll
          for (int j = 0; j < NB; j++)
#pragma unroll
            for (int i = 0; i < 16; i++)
              acc[j][i] = __builtin_ldexpf(acc[j][i], -xexp[32 * (tb + j) + 8 * (i >> 2) + 4 * hh + (i & 3)]);
        }
        // Software-pipelined steps: the LDS reads and the dequantisation of step tt+1 are
        // issued before the MFMAs of step tt, so their latency hides behind the matrix cores.
        // K-quant stages are always whole (n_in % 256 == 0); Q8_0's last stage may be short.
        constexpr int SPC = KX / 16;  // steps per chunk
        const int nsteps = TYPE == 0 ? min(SPC, (int)(nk - KX * c4) / 16) : SPC;
        f16x8 xf0[NB], xf1[NB], wf0, wf1;
        auto frags = [&](int tt, f16x8(&xf)[NB], f16x8 &wf) {
          const int t = SPC * c4 + tt;
          f16x2 sc, nm;
          ss.get(t, sc, nm);
          wf = weight_frag<TYPE>(ws, t, hh, sc, nm);
          const uint32_t ko = koff<TYPE>(t, hh) - KX * c4;
#pragma unroll
          for (int j = 0; j < NB; j++) xf[j] = *(const f16x8 *)(cur + (32 * (tb + j) + (lane & 31)) * PITCH2 + ko);
        };
        frags(0, xf0, wf0);
#pragma unroll
        for (int tt = 0; tt < SPC; tt++) {
          if (tt < nsteps) {
            if (tt + 1 < nsteps) {
              if (tt & 1)
                frags(tt + 1, xf0, wf0);
              else
                frags(tt + 1, xf1, wf1);
            }
#pragma unroll
            for (int j = 0; j < NB; j++)
              acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16((tt & 1) ? xf1[j] : xf0[j], (tt & 1) ? wf1 : wf0,
                                                              acc[j], 0, 0, 0);
          }
        }
        if (rescaled) {
#pragma unroll
          for (int j = 0; j < NB; j++)
#pragma unroll
            for (int i = 0; i < 16; i++)
              acc[j][i] = __builtin_ldexpf(acc[j][i], xexp[32 * (tb + j) + 8 * (i >> 2) + 4 * hh + (i & 3)]);
        }
        __syncthreads();  // every wave is done with this chunk
        if (next) {
          const bool r = store_chunk<KX, XHALF, NT2>(xs, xn, xexp, (chunk + 1) * KX, p.n_in);
          if (lane == 0) xflag[wave] = r;
          __syncthreads();
        }
        chunk++;
      }
    }
    if (more) ws = wn;
  }

  if (my_row < p.n_out) {
#pragma unroll
    for (int j = 0; j < NB; j++) {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t tok = 32 * (tb + j) + 8 * (i >> 2) + 4 * hh + (i & 3);
        if (tok < n_tok) {
          float *o = y + p.y_off + (size_t)(col0 + tok) * p.y_stride + my_row;
          *o = ACCUM ? *o + acc[j][i] : acc[j][i];
        }
      }
    }
  }
}

}  // namespace

// Dense (MOE = 0) launches use the 128 x 128 tile; expert groups (MOE = 1) 128 x 32 tiles
// (K-quants: LDS-staged weights, four waves of 32 rows; Q8_0: register weights).
#define MM_BODY(T, A, M, H)                                                     \
  if constexpr (M == 0 && T != 0)                                               \
    matmul_tile128_w<T, A, H, 8>(w, wd, x, y, ctl, p);                          \
  else if constexpr (M == 0)                                                    \
    matmul_tile128<T, A, H>(w, wd, x, y, ctl, p);                               \
  else if constexpr (T != 0)                                                    \
    matmul_tile128_w<T, A, H, 4, 32, 1>(w, wd, x, y, ctl, p);                   \
  else                                                                          \
    matmul_body<T, A, M, H>(w, wd, x, y, ctl, p);

#define MM(T, A, M)                                                                          \
  extern "C" __global__ __launch_bounds__(M ? 256 : NT2) void matmul__##T##_##A##_##M(       \
      const uint4 *w, const uint16_t *wd, const float *x, float *y, const uint32_t *ctl,     \
      MatmulPush p) {                                                                        \
    MM_BODY(T, A, M, 0)                                                                      \
  }                                                                                          \
  extern "C" __global__ __launch_bounds__(M ? 256 : NT2) void matmul__##T##_##A##_##M##_1(   \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,       \
      MatmulPush p) {                                                                        \
    MM_BODY(T, A, M, 1)                                                                      \
  }

#define MM_TYPE(T) \
  MM(T, 0, 0)      \
  MM(T, 1, 0)      \
  MM(T, 0, 1)      \
  MM(T, 1, 1)

MM_TYPE(0)
MM_TYPE(1)
MM_TYPE(2)

// Runtime-internal dense K-quant variants (not engine symbols): NW = 4 or 8 waves, with a
// K split over workspace `ws` and counters `cnt` (zeroed once; each launch leaves them zero).
#define MMX(T, A, H, XT)                                                                          \
  extern "C" __global__ __launch_bounds__(256) void matmul_w4__##T##_##A##_##H(                   \
      const uint4 *w, const uint16_t *wd, const XT *x, float *y, const uint32_t *ctl,             \
      MatmulPush p, float *ws, uint32_t *cnt, uint32_t S) {                                       \
    matmul_tile128_w<T, A, H, 4>(w, wd, x, y, ctl, p, ws, cnt, S);                                \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(512) void matmul_w8__##T##_##A##_##H(                   \
      const uint4 *w, const uint16_t *wd, const XT *x, float *y, const uint32_t *ctl,             \
      MatmulPush p, float *ws, uint32_t *cnt, uint32_t S) {                                       \
    matmul_tile128_w<T, A, H, 8>(w, wd, x, y, ctl, p, ws, cnt, S);                                \
  }
MMX(1, 0, 0, float)
MMX(1, 1, 0, float)
MMX(1, 0, 1, f16)
MMX(1, 1, 1, f16)
MMX(2, 0, 0, float)
MMX(2, 1, 0, float)
MMX(2, 0, 1, f16)
MMX(2, 1, 1, f16)

// Dense K-quant tiles on f16 rows that x_half_rows wrote (XHALF = 2): x is that buffer (the
// per-row exponents first, then the rows), same arguments as matmul_w8.
#define MMH(T, A)                                                                                 \
  extern "C" __global__ __launch_bounds__(512) void matmul_x8__##T##_##A(                          \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      MatmulPush p, float *ws, uint32_t *cnt, uint32_t S) {                                       \
    matmul_tile128_w<T, A, 2, 8>(w, wd, x, y, ctl, p, ws, cnt, S);                                \
  }
MMH(1, 0)
MMH(1, 1)
MMH(2, 0)
MMH(2, 1)

// Expert groups (128 x 32 tiles, four waves) on the f16 rows x_half_rows wrote: the rows of
// the launch's inputs (tokens for gate and up, slots for down), no K split.  MOE = 2: grid
// (row tiles, at least the tile map's entries, 1), grid.y indexing moe_sort's tile map.
#define MMXM(T, A)                                                                                \
  extern "C" __global__ __launch_bounds__(256) void matmul_xm__##T##_##A(                          \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl, MatmulPush p) { \
    matmul_tile128_w<T, A, 2, 4, 32, 2>(w, wd, x, y, ctl, p);                                     \
  }
MMXM(1, 0)
MMXM(1, 1)
MMXM(2, 0)
MMXM(2, 1)
// the same over up to four matrices on the same rows (gate and up): row tiles of segment s
// after those of s - 1, each with its own regions, y_off, n_out and y_stride
#define MMXMS(T, A)                                                                               \
  extern "C" __global__ __launch_bounds__(256) void matmul_xms__##T##_##A(                         \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      Segments<MatmulPush> m) {                                                                   \
    matmul_tile128_w<T, A, 2, 4, 32, 2, 0, 1>(w, wd, x, y, ctl, m.p[0], nullptr, nullptr, 1, 0, 1, m); \
  }
MMXMS(1, 0)
MMXMS(1, 1)
MMXMS(2, 0)
MMXMS(2, 1)

// The four-wave tile on the same f16 rows (128 tokens per wave, 128-k chunks).
#define MMH4(T, A)                                                                                \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void       \
      matmul_x4__##T##_##A(                                                                       \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      MatmulPush p, float *ws, uint32_t *cnt, uint32_t S) {                                       \
    matmul_tile128_w<T, A, 2, 4>(w, wd, x, y, ctl, p, ws, cnt, S);                                \
  }
MMH4(1, 0)
MMH4(1, 1)
MMH4(2, 0)
MMH4(2, 1)

// The four-wave tile on f16 rows over a balanced grid (HYB): hf whole tiles, the rest in
// two K halves; hz token tiles per row tile.
#define MMH4B(T, A)                                                                               \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void       \
      matmul_x4b__##T##_##A(                                                                      \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      MatmulPush p, float *ws, uint32_t *cnt, uint32_t S, uint32_t hf, uint32_t hz) {             \
    matmul_tile128_w<T, A, 2, 4, TN2, 0, 1>(w, wd, x, y, ctl, p, ws, cnt, S, hf, hz);             \
  }
MMH4B(1, 0)
MMH4B(1, 1)
MMH4B(2, 0)
MMH4B(2, 1)

// The four-wave Q4_K tile with activations and weights loaded straight into LDS (XHALF 3),
// on a plain grid (x4d) and on the balanced grid (x4db).  (Q6_K's 28 KiB weight stages,
// double buffered, would leave one four-wave workgroup per CU: it keeps the x4 tiles.)
#define MMH4D(A)                                                                                  \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void       \
      matmul_x4d__1_##A(                                                                          \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      MatmulPush p, float *ws, uint32_t *cnt, uint32_t S) {                                       \
    matmul_tile128_w<1, A, 3, 4>(w, wd, x, y, ctl, p, ws, cnt, S);                                \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void       \
      matmul_x4db__1_##A(                                                                         \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      MatmulPush p, float *ws, uint32_t *cnt, uint32_t S, uint32_t hf, uint32_t hz) {             \
    matmul_tile128_w<1, A, 3, 4, TN2, 0, 1>(w, wd, x, y, ctl, p, ws, cnt, S, hf, hz);             \
  }
MMH4D(0)
MMH4D(1)

// The eight-wave tile with operands loaded straight into LDS: K-split launches (x8d) and
// segments (x8ds), Q4_K and Q6_K.
#define MMH8D(T, A)                                                                               \
  extern "C" __global__ __launch_bounds__(512) void matmul_x8d__##T##_##A(                         \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      MatmulPush p, float *ws, uint32_t *cnt, uint32_t S) {                                       \
    matmul_tile128_w<T, A, 3, 8>(w, wd, x, y, ctl, p, ws, cnt, S);                                \
  }                                                                                               \
  extern "C" __global__ __launch_bounds__(512) void matmul_x8ds__##T##_##A(                        \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      Segments<MatmulPush> m, float *ws, uint32_t *cnt, uint32_t S) {                              \
    matmul_tile128_w<T, A, 3, 8, TN2, 0, 0, 1>(w, wd, x, y, ctl, m.p[0], ws, cnt, S, 0, 1, m);     \
  }
MMH8D(1, 0)
MMH8D(1, 1)
MMH8D(2, 0)
MMH8D(2, 1)

// The eight-wave tile on f16 rows over up to four matrices that read the same rows
// (segment table as the matvecs take it; start[] counts row tiles).
#define MMHS(T, A)                                                                                \
  extern "C" __global__ __launch_bounds__(512) void matmul_x8s__##T##_##A(                         \
      const uint4 *w, const uint16_t *wd, const f16 *x, float *y, const uint32_t *ctl,            \
      Segments<MatmulPush> m, float *ws, uint32_t *cnt, uint32_t S) {                              \
    matmul_tile128_w<T, A, 2, 8, TN2, 0, 0, 1>(w, wd, x, y, ctl, m.p[0], ws, cnt, S, 0, 1, m);     \
  }
MMHS(1, 0)
MMHS(1, 1)
MMHS(2, 0)
MMHS(2, 1)

// f32 activation rows to f16 rows for the dense K-quant tiles, once per launch instead of
// in every tile (the runtime inserts it before dense K-quant matmuls with f32 inputs; one
// conversion serves every matmul that reads the same rows before the next barrier).  Row t
// (t < ctl[2]) of x -- x_off + t * x_stride, n_in values -- becomes h[t * n_in ..] =
// f16(x * 2^-e_t), each four values k..k+3 stored in the order k, k+2, k+1, k+3 (the
// order of the packed-quant extraction, so the tiles copy the rows as they are), with e_t = 0 unless the row's largest |x| reaches 2^15, then its
// exponent - 14 (the tile's range guard, applied to the whole row): e[t] = e_t, and the tile
// multiplies its sums back by 2^e_t.  With e_t = 0 the f16 values, and so the GEMM's bits,
// are those of the tile's own conversion (round to nearest even).  Grid: one workgroup per
// row of the launch's token tiles; out = [e: one int32 per row][rows: f16 from u32 h_off,
// n_in per row, 16-byte aligned].
struct XHalfPush {
  uint32_t x_off, x_stride, n_in, h_off;
  uint32_t rows_per_token;  // input rows per token of ctl[2]: 1, or the slots of an expert down
};
// One row of f16 for the tiles from its values v (n_in <= 12288 at 4 per thread and 256
// threads), with e = 0 unless the row's largest |x| reaches 2^15 (then the row is x * 2^-e,
// e putting it below 2^15): the rows at out + h_off (f16 row t at t * n_in), pairs (0,2),
// (1,3) of every four values as the tiles' LDS rows hold them; the exponent at out[t].
constexpr int HALF_ROW_V = 48;  // values per thread: n_in <= 12288
SK_DEV void store_half_row(const float4 (&v)[HALF_ROW_V / 4], uint32_t *out, uint32_t h_off, uint32_t n_in,
                           uint32_t t) {
  const uint32_t tid = threadIdx.x;
  float m = 0.0f;
#pragma unroll
  for (int i = 0; i < HALF_ROW_V / 4; i++)
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  // the row's largest |x| (NaN counts as big, as in the tile's guard)
  __shared__ uint32_t big[4];
  __shared__ float wm[4];
  const bool b = !(m < 32768.0f);
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  const uint64_t anyb = __ballot(b);
  if ((tid & 63) == 0) {
    wm[tid >> 6] = m;
    big[tid >> 6] = anyb != 0;
  }
  __syncthreads();
  const float tm = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
  const bool any = big[0] | big[1] | big[2] | big[3];
  const int e = any && tm >= 32768.0f ? (int)((__builtin_bit_cast(uint32_t, tm) >> 23) & 255u) - 127 - 14 : 0;
  const float sc = __builtin_ldexpf(1.0f, -e);
  f16 *h = (f16 *)(out + h_off) + (size_t)t * n_in;
#pragma unroll
  for (int i = 0; i < HALF_ROW_V / 4; i++) {
    const uint32_t k = 4 * (tid + 256 * i);
    if (k < n_in) {
      float4 a = v[i];
      if (e) a = make_float4(a.x * sc, a.y * sc, a.z * sc, a.w * sc);
      *(uint2 *)(h + k) = make_uint2(as_u32(pack_f16x2(a.x, a.z)), as_u32(pack_f16x2(a.y, a.w)));
    }
  }
  if (tid == 0) out[t] = (uint32_t)e;
}

extern "C" __global__ __launch_bounds__(256) void x_half_rows(const float *x, uint32_t *out, const uint32_t *ctl,
                                                              XHalfPush p) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  if (t >= ctl[2] * p.rows_per_token) return;
  const float *xr = x + p.x_off + (size_t)t * p.x_stride;
  float4 v[HALF_ROW_V / 4];
#pragma unroll
  for (int i = 0; i < HALF_ROW_V / 4; i++) {
    const uint32_t k = 4 * (tid + 256 * i);
    v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (k < p.n_in) v[i] = *(const float4 *)(xr + k);
  }
  store_half_row(v, out, p.h_off, p.n_in, t);
}

// silu_mul (silu_mul.comp:15-23) on the rows an expert down projection reads, with that
// matmul's f16 row prepass in the same launch: slot row t (t < ctl[2] x rows_per_token)
// becomes g / (1 + e^-g) * u in place, in silu_mul's expression (the same f32 values), and
// its f16 row and exponent go to the workspace as x_half_rows writes them.  The columns
// past n_in of a row and the rows past the slots are not computed: no later launch reads
// them.
struct SiluHalfPush {
  uint32_t g_off, u_off, x_stride, n_in, h_off, rows_per_token;
};
extern "C" __global__ __launch_bounds__(256) void silu_half_rows(float *a, uint32_t *out, const uint32_t *ctl,
                                                                 SiluHalfPush p) {
  const uint32_t t = blockIdx.x, tid = threadIdx.x;
  if (t >= ctl[2] * p.rows_per_token) return;
  // every load in flight before the first is used: the passes the row needs (uniform), a
  // lane past the row's end reading its last four values (n_in is a multiple of 4)
  const uint32_t n_pass = (p.n_in + 1023) / 1024;
  float *gr = a + p.g_off + (size_t)t * p.x_stride;
  const float *ur = a + p.u_off + (size_t)t * p.x_stride;
  float4 g[HALF_ROW_V / 4], u[HALF_ROW_V / 4];
#pragma unroll
  for (int i = 0; i < HALF_ROW_V / 4; i++)
    if ((uint32_t)i < n_pass) {
      const uint32_t k = min(4 * (tid + 256 * i), p.n_in - 4);
      g[i] = *(const float4 *)(gr + k);
      u[i] = *(const float4 *)(ur + k);
    }
  float4 v[HALF_ROW_V / 4];
#pragma unroll
  for (int i = 0; i < HALF_ROW_V / 4; i++) {
    const uint32_t k = 4 * (tid + 256 * i);
    v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    if ((uint32_t)i < n_pass && k < p.n_in) {
      {
#pragma clang fp contract(off)
        v[i] = make_float4(g[i].x / (1.0f + expf(-g[i].x)) * u[i].x, g[i].y / (1.0f + expf(-g[i].y)) * u[i].y,
                           g[i].z / (1.0f + expf(-g[i].z)) * u[i].z, g[i].w / (1.0f + expf(-g[i].w)) * u[i].w);
      }
      *(float4 *)(gr + k) = v[i];
    }
  }
  store_half_row(v, out, p.h_off, p.n_in, t);
}

// rmsnorm (rmsnorm.comp; ops.rs:1-16) on the rows a dense matmul reads next, with that
// matmul's f16 row prepass in the same launch: token row tok (tok < ctl[2]) of x becomes
// y = x * r * w in rmsnorm's expression (the same f32 values, written to y_off as rmsnorm
// writes them), and its f16 row and exponent go to the workspace as x_half_rows writes them.
// The runtime uses it only for rows of at most 4096 values with x_off, y_off, w_off, n and
// stride multiples of 4 (rmsnorm's float4 path).  Grid [1, tokens, 1], as rmsnorm's.
struct NormHalfPush {
  uint32_t x_off, w_off, y_off, n;
  float eps;
  uint32_t stride, h_off;
};
extern "C" __global__ __launch_bounds__(256) void rmsnorm_half_rows(const float *w, float *a, uint32_t *out,
                                                                    const uint32_t *ctl, NormHalfPush p) {
  const uint32_t tok = blockIdx.y, t = threadIdx.x;
  if (tok >= ctl[2]) return;
  float4 v[HALF_ROW_V / 4];
#pragma unroll
  for (int i = 4; i < HALF_ROW_V / 4; i++) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  float4 y4[4];
  norm_row4(a + p.x_off + tok * p.stride, w + p.w_off, p.n, p.eps, y4);
  float4 *yr = (float4 *)(a + p.y_off + tok * p.stride);
#pragma unroll
  for (int k = 0; k < 4; k++) {
    v[k] = y4[k];
    if (t + 256 * k < (p.n >> 2)) yr[t + 256 * k] = y4[k];
  }
  store_half_row(v, out, p.h_off, p.n, tok);
}

// Workspace of skyla_hip_dispatch_noalloc, the entry point that allocates nothing: the K
// split's f32 partial tiles (SCRATCH_TILES of 128 x 128), then its per-tile arrival
// counters (SCRATCH_COUNTERS).  A K-split launch holds at most 256 partial tiles (row tiles
// x token tiles x S <= 256, skyla_hip.cpp split_of) and 128 counters.  Each loaded copy of
// this code object (one per context, so one per device) owns its array until it is
// unloaded.  Kernels never name it: the runtime looks its device address up once per
// context and passes that as the `ws` and `cnt` arguments, as it passes its own workspace.
#define SCRATCH_TILES 256
#define SCRATCH_COUNTERS 1024
__device__ __attribute__((used)) __align__(256) unsigned char
    scratch[SCRATCH_TILES * 128 * 128 * 4 + SCRATCH_COUNTERS * 4];

// p[0, n) = v: clears the counters before an allocation-free launch (a kernel, not
// hipMemsetAsync, so that a caller may capture it into a HIP graph)
extern "C" __global__ __launch_bounds__(256) void fill_u32(uint32_t *p, uint32_t n, uint32_t v) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}
