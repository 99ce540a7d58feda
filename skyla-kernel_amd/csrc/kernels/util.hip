// Measurement and checking kernels.
#include "common.h"

struct BandwidthPush { uint32_t n_vec4; };

// bandwidth (bandwidth.comp:1-23): grid-stride XOR stream over n_vec4 uint4; writes only
// if the fold hits a fixed constant, which keeps the loads live.  Roofline probe for the
// HBM-bound kernels.  spec [threads per workgroup] is the reference's form (four loads in
// flight per lane); spec [threads, depth] keeps `depth` loads in flight, and a third word 1
// issues them non-temporal, so the probe can sweep for the device's stream-read ceiling.
// Each uint4 is folded by thread (index mod grid threads) whatever the depth.
template <int THREADS, int DEPTH, bool NT>
SK_DEV void bandwidth_body(const uint4 *src, uint32_t *dst, BandwidthPush p) {
  const uint32_t gid = blockIdx.x * THREADS + threadIdx.x;
  const uint32_t stride = gridDim.x * THREADS;
  uint4 acc = make_uint4(0, 0, 0, 0);
  uint32_t i = gid;
  for (; i + (DEPTH - 1) * stride < p.n_vec4; i += DEPTH * stride) {
    uint4 v[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; d++)
      if constexpr (NT) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const u32x4 t = __builtin_nontemporal_load((const u32x4 *)(src + i + d * stride));
        v[d] = make_uint4(t.x, t.y, t.z, t.w);
      } else {
        v[d] = src[i + d * stride];
      }
#pragma unroll
    for (int d = 0; d < DEPTH; d++) {
      acc.x ^= v[d].x;
      acc.y ^= v[d].y;
      acc.z ^= v[d].z;
      acc.w ^= v[d].w;
    }
  }
  for (; i < p.n_vec4; i += stride) {
    const uint4 a = src[i];
    acc.x ^= a.x;
    acc.y ^= a.y;
    acc.z ^= a.z;
    acc.w ^= a.w;
  }
  const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
  if (r == 0x9e3779b9u) dst[gid] = r;
}

#define BW(NAME, T, D, NT)                                                                  \
  extern "C" __global__ __launch_bounds__(T) void NAME(const uint4 *src, uint32_t *dst,      \
                                                       BandwidthPush p) {                   \
    bandwidth_body<T, D, NT>(src, dst, p);                                                  \
  }
BW(bandwidth__64, 64, 4, false)
BW(bandwidth__128, 128, 4, false)
BW(bandwidth__256, 256, 4, false)
BW(bandwidth__512, 512, 4, false)
BW(bandwidth__1024, 1024, 4, false)
BW(bandwidth__256_8, 256, 8, false)
BW(bandwidth__256_16, 256, 16, false)
BW(bandwidth__512_8, 512, 8, false)
BW(bandwidth__1024_8, 1024, 8, false)
BW(bandwidth__256_4_1, 256, 4, true)
BW(bandwidth__256_8_1, 256, 8, true)
BW(bandwidth__256_16_1, 256, 16, true)
BW(bandwidth__512_8_1, 512, 8, true)
BW(bandwidth__1024_8_1, 1024, 8, true)

// dequant: the bit-exact dequantisation the path's arithmetic is judged against
// (quant.rs:5-89), run on the GPU over planner regions.  One thread per 32-value group,
// output row-major f32: y[y_off + row * n_in + k].  spec [TYPE] (0/1/2 = Q8_0/Q4_K/Q6_K).
// Push: o0..o3 region offsets (as the matmul push), n_in, n_rows, y_off.
struct DequantPush { uint32_t o0, o1, o2, o3, n_in, n_rows, y_off; };

// The 32 values of group gi (32-value groups in row order) of row `row`; returns the index
// of the first value within the row.
template <int TYPE>
SK_DEV uint32_t dequant_group(const uint4 *w, const uint16_t *wd, uint32_t o0, uint32_t o1, uint32_t o2,
                              uint32_t o3, uint32_t n_in, uint32_t row, uint32_t gi, float o[32]) {
  if (TYPE == 1) {
    const uint32_t sb = gi >> 3, sub = gi & 7;
    const uint32_t rs = row * (n_in >> 8) + sb;
    const uint4 *qs = w + o0 + rs * 8 + (sub >> 1) * 2;
    dequant_q4k_sub(w[o1 + rs], qs[0], qs[1], sub, o);
    return sb * 256 + (sub >> 1) * 64 + (sub & 1) * 32;
  } else if (TYPE == 2) {
    const uint32_t sb = gi >> 3, hf = (gi >> 2) & 1, g = gi & 3;
    const uint32_t rs = row * (n_in >> 8) + sb;
    uint4 ql[4], qh[2];
    for (int i = 0; i < 4; i++) ql[i] = w[o0 + rs * 8 + hf * 4 + i];
    for (int i = 0; i < 2; i++) qh[i] = w[o1 + rs * 4 + hf * 2 + i];
    dequant_q6k_group(ql, qh, w[o2 + rs], f16_bits_to_f32(wd[o3 + rs]), hf, g, o);
    return sb * 256 + hf * 128 + g * 32;
  } else {
    const uint4 *q = w + o0 + row * (n_in >> 4) + gi * 2;
    dequant_q8_0_block(q[0], q[1], f16_bits_to_f32(wd[o1 + row * (n_in >> 5) + gi]), o);
    return gi * 32;
  }
}

SK_DEV void store32(float *dst, const float o[32]) {
#pragma unroll
  for (int i = 0; i < 8; i++) ((float4 *)dst)[i] = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
}

template <int TYPE>
SK_DEV void dequant_body(const uint4 *w, const uint16_t *wd, float *y, DequantPush p) {
  const uint32_t groups = p.n_in >> 5;
  const uint32_t gid = blockIdx.x * 256 + threadIdx.x;
  if (gid >= groups * p.n_rows) return;
  const uint32_t row = gid / groups, gi = gid % groups;
  float o[32];
  const uint32_t first = dequant_group<TYPE>(w, wd, p.o0, p.o1, p.o2, p.o3, p.n_in, row, gi, o);
  store32(y + p.y_off + (size_t)row * p.n_in + first, o);
}

// embed: the activation rows of a chunk's tokens from the HBM copy of token_embd.  The
// reference dequantises the rows on the host and writes them into the mapped arena
// (engine.rs:100-117, skyla_gguf::dequantize); here the engine writes only the token ids
// (u32, at ids_off of the arena) and this gathers and dequantises row ids[tok] into
// a[x_off + tok * stride ..] for tok < ctl[2], with the same bit-exact arithmetic as
// dequant.  One thread per 32-value group; grid [ceil(n_embd / 32 / 256), tokens, 1].
// spec [TYPE]; push: o0..o3 of the matrix, n_embd, ids_off, x_off, stride.
struct EmbedPush { uint32_t o0, o1, o2, o3, n_embd, ids_off, x_off, stride; };

template <int TYPE>
SK_DEV void embed_body(const uint4 *w, const uint16_t *wd, float *a, const uint32_t *ctl, EmbedPush p) {
  const uint32_t tok = blockIdx.y, gi = blockIdx.x * 256 + threadIdx.x;
  if (tok >= ctl[2] || gi >= (p.n_embd >> 5)) return;
  const uint32_t row = ctl[p.ids_off + tok];
  float o[32];
  const uint32_t first = dequant_group<TYPE>(w, wd, p.o0, p.o1, p.o2, p.o3, p.n_embd, row, gi, o);
  store32(a + p.x_off + tok * p.stride + first, o);
}

#define EMB(T)                                                                               \
  extern "C" __global__ __launch_bounds__(256) void embed__##T(                                \
      const uint4 *w, const uint16_t *wd, float *a, const uint32_t *ctl, EmbedPush p) {       \
    embed_body<T>(w, wd, a, ctl, p);                                                         \
  }
EMB(0)
EMB(1)
EMB(2)

#define DQ(T)                                                                                \
  extern "C" __global__ __launch_bounds__(256) void dequant__##T(const uint4 *w,              \
                                                                  const uint16_t *wd,        \
                                                                  float *y, DequantPush p) {  \
    dequant_body<T>(w, wd, y, p);                                                            \
  }
DQ(0)
DQ(1)
DQ(2)
