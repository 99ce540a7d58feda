// The rest of the decode step around the weight matvecs, gfx950: RMSNorm, the QK-norm +
// RoPE + KV-cache write, split-K attention over the cache and its merge, and the last-row
// copy of a prefill chunk (graph.rs:48-113, 200-233; the kernels of kernels.rs:186-193).
//
// Contract (bindings, push words, grids) as the engine dispatches them:
//   rmsnorm          [W, A, C]            6 words  grid [1, tokens, 1]
//   qkv_prep         [W, A, C, KV, KV8]  16 words  grid [n_head + 2 n_kv, tokens, 1]
//   attention        [A, C, KV, KV8, KVS] 11 words grid [n_kv, n_split, tokens]
//   attention_merge  [A, C]               6 words  grid [n_head, tokens, 1]
//   take_last        [A, C]               4 words  grid [ceil(n / 256), 1, 1]
// W is a weight buffer (f32 tables: norm weights, RoPE frequencies), A the f32 arena and C
// its u32 view (ctl[1] = position of the first token, ctl[2] = token count), KV the cache
// buffer as f16 (keys, f16 values, the per-32 scales of 8-bit entries) and KV8 as i8.
// Offsets are element indices of the view they index.  Heads are 128 wide (head_dim =
// n_rot = 128, no gate: the plain Qwen3 layout Engine::new accepts, engine.rs:27-39).
//
// KV layout (kv.rs): a layer's keys at kc_off + pos * kv_dim + head * 128, values likewise
// at vc_off; an 8-bit row keeps one f16 scale per 32 values at
// scales + pos * kv_dim / 32 + head * 4 + block.  An entry is quantised as
// s = max|y| over its block / 127, q = round(y / s) (qkv_prep.comp:44-65; ties to even).
#include "common.h"

namespace {

constexpr uint32_t HD = 128;     // head width
constexpr uint32_t CHUNK = 64;   // positions per attention split (arena.rs:6)
constexpr uint32_t PART = HD + 2;  // one (head, split) partial: m, l, acc[128]

struct NormPush { uint32_t x_off, w_off, y_off, n; float eps; uint32_t stride; };
struct QkvPush {
  uint32_t q_off, k_off, v_off, qn_off, kn_off, kc_off, vc_off, n_head, n_kv;
  float eps;
  uint32_t rope_off;
  float mscale;
  uint32_t q_stride, kv_stride, ks_off, vs_off;
};
struct AttnPush {
  uint32_t q_off, part_off, kc_off, vc_off, n_kv, n_split;
  float scale;
  uint32_t q_stride, part_stride, ks_off, vs_off;
};
struct MergePush { uint32_t part_off, o_off, n_split, chunk, part_stride, o_stride; };
struct LastPush { uint32_t src_off, dst_off, n, stride; };

SK_DEV float wave_sum(float v) { return group_sum<64>(v); }

SK_DEV float wave_max(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
  return v;
}

// max |v| over the 32-lane half of the wave that holds v (one quantisation block)
SK_DEV float block_max(float v) {
  v = fabsf(v);
#pragma unroll
  for (int d = 16; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
  return v;
}

// Writes y0 (element t) and y1 (element t + 64) of one head's cache row.
template <int Q8>
SK_DEV void store_kv(f16 *kv, int8_t *kv8, uint32_t cache, uint32_t scales, uint32_t kv_dim, uint32_t pos,
                     uint32_t head, uint32_t t, float y0, float y1) {
  const uint32_t dst = cache + pos * kv_dim + head * HD;
  if constexpr (!Q8) {
    kv[dst + t] = (f16)y0;
    kv[dst + t + 64] = (f16)y1;
  } else {
    const float s0 = block_max(y0) / 127.0f, s1 = block_max(y1) / 127.0f;
    kv8[dst + t] = (int8_t)(s0 > 0.0f ? __builtin_rintf(y0 / s0) : 0.0f);
    kv8[dst + t + 64] = (int8_t)(s1 > 0.0f ? __builtin_rintf(y1 / s1) : 0.0f);
    if ((t & 31) == 0) {
      const uint32_t sd = scales + pos * (kv_dim / 32) + head * 4 + t / 32;
      kv[sd] = (f16)s0;
      kv[sd + 2] = (f16)s1;
    }
  }
}

template <int K8, int V8>
SK_DEV void qkv_body(const float *w, float *a, const uint32_t *ctl, f16 *kv, int8_t *kv8, const QkvPush &p) {
#pragma clang fp contract(off)
  const uint32_t h = blockIdx.x, tok = blockIdx.y;
  if (tok >= ctl[2]) return;
  const uint32_t t = threadIdx.x, pos = ctl[1] + tok, kv_dim = p.n_kv * HD;
  if (h >= p.n_head + p.n_kv) {  // value head: cache it as it is
    const uint32_t vh = h - p.n_head - p.n_kv;
    const uint32_t src = p.v_off + tok * p.kv_stride + vh * HD;
    store_kv<V8>(kv, kv8, p.vc_off, p.vs_off, kv_dim, pos, vh, t, a[src + t], a[src + t + 64]);
    return;
  }
  const bool is_q = h < p.n_head;
  const uint32_t head = is_q ? h : h - p.n_head;
  const uint32_t src = (is_q ? p.q_off + tok * p.q_stride : p.k_off + tok * p.kv_stride) + head * HD;
  const uint32_t nw = is_q ? p.qn_off : p.kn_off;
  const float x0 = a[src + t], x1 = a[src + t + 64];
  const float r = 1.0f / sqrtf(wave_sum(x0 * x0 + x1 * x1) / (float)HD + p.eps);
  const float n0 = x0 * r * w[nw + t], n1 = x1 * r * w[nw + t + 64];
  // NeoX rotation of the pair (t, t + 64) by pos * freq[t] (rope.rs:60-68)
  const float angle = (float)pos * w[p.rope_off + t];
  const float c = cosf(angle) * p.mscale, s = sinf(angle) * p.mscale;
  const float y0 = n0 * c - n1 * s, y1 = n0 * s + n1 * c;
  if (is_q) {
    a[src + t] = y0;
    a[src + t + 64] = y1;
  } else {
    store_kv<K8>(kv, kv8, p.kc_off, p.ks_off, kv_dim, pos, head, t, y0, y1);
  }
}

// Element d of cache row `pos` of head kvh.
template <int Q8>
SK_DEV float load_kv(const f16 *kv, const int8_t *kv8, uint32_t cache, uint32_t scales, uint32_t kv_dim,
                     uint32_t pos, uint32_t kvh, uint32_t d) {
  const uint32_t at = cache + pos * kv_dim + kvh * HD + d;
  if constexpr (!Q8)
    return (float)kv[at];
  else
    return (float)kv8[at] * (float)kv[scales + pos * (kv_dim / 32) + kvh * 4 + d / 32];
}

// One wave per (kv head, split of CHUNK positions, token).  The N_REP query heads that share
// the kv head are held in LDS (scaled).  Scores: lane p takes position split * CHUNK + p and
// dots its key row with every query head.  The chunk's softmax numerators e_p = exp(s_p - m)
// then weight the value rows, lane d owning output elements d and d + 64.  The partial
// (m, l = sum e_p, acc = sum e_p v_p) goes to the part region for attention_merge; it is the
// same quantity as the reference's running (m, l, acc) over the chunk (attention.comp:83-97).
template <int N_REP, int K8, int V8>
SK_DEV void attention_body(float *a, const uint32_t *ctl, const f16 *kv, const int8_t *kv8, const AttnPush &p) {
  __shared__ float qs[N_REP][HD];
  const uint32_t kvh = blockIdx.x, split = blockIdx.y, tok = blockIdx.z;
  const uint32_t n_pos = ctl[1] + tok + 1;
  if (tok >= ctl[2] || split * CHUNK >= n_pos) return;
  const uint32_t lane = threadIdx.x, kv_dim = p.n_kv * HD;
  const uint32_t q_base = p.q_off + tok * p.q_stride;
#pragma unroll
  for (int j = 0; j < N_REP; j++) {
    const uint32_t qb = q_base + (kvh * N_REP + j) * HD;
    qs[j][lane] = a[qb + lane] * p.scale;
    qs[j][lane + 64] = a[qb + lane + 64] * p.scale;
  }
  __syncthreads();
  const uint32_t begin = split * CHUNK, cnt = min(CHUNK, n_pos - begin);
  const bool live = lane < cnt;
  const uint32_t pos = begin + (live ? lane : 0);
  float s[N_REP];
#pragma unroll
  for (int j = 0; j < N_REP; j++) s[j] = 0.0f;
  for (uint32_t d0 = 0; d0 < HD; d0 += 8) {
    float k[8];
    if constexpr (!K8) {
      const uint4 raw = *(const uint4 *)(kv + p.kc_off + pos * kv_dim + kvh * HD + d0);
      const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const f16x2 h = as_f16x2(wd[i]);
        k[2 * i] = (float)h.x;
        k[2 * i + 1] = (float)h.y;
      }
    } else {
      const uint2 raw = *(const uint2 *)(kv8 + p.kc_off + pos * kv_dim + kvh * HD + d0);
      const float sc = (float)kv[p.ks_off + pos * (kv_dim / 32) + kvh * 4 + d0 / 32];
      const uint32_t wd[2] = {raw.x, raw.y};
#pragma unroll
      for (int i = 0; i < 8; i++) k[i] = (float)(int8_t)((wd[i >> 2] >> (8 * (i & 3))) & 255u) * sc;
    }
#pragma unroll
    for (int j = 0; j < N_REP; j++)
#pragma unroll
      for (int i = 0; i < 8; i++) s[j] = __builtin_fmaf(qs[j][d0 + i], k[i], s[j]);
  }
  float e[N_REP], m[N_REP], l[N_REP];
#pragma unroll
  for (int j = 0; j < N_REP; j++) {
    m[j] = wave_max(live ? s[j] : -INFINITY);
    e[j] = live ? expf(s[j] - m[j]) : 0.0f;
    l[j] = wave_sum(e[j]);
  }
  float acc0[N_REP], acc1[N_REP];
#pragma unroll
  for (int j = 0; j < N_REP; j++) acc0[j] = acc1[j] = 0.0f;
  for (uint32_t q = 0; q < cnt; q++) {
    const float v0 = load_kv<V8>(kv, kv8, p.vc_off, p.vs_off, kv_dim, begin + q, kvh, lane);
    const float v1 = load_kv<V8>(kv, kv8, p.vc_off, p.vs_off, kv_dim, begin + q, kvh, lane + 64);
#pragma unroll
    for (int j = 0; j < N_REP; j++) {
      const float ep = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e[j]), (int)q));
      acc0[j] = __builtin_fmaf(ep, v0, acc0[j]);
      acc1[j] = __builtin_fmaf(ep, v1, acc1[j]);
    }
  }
  const uint32_t part_base = p.part_off + tok * p.part_stride;
#pragma unroll
  for (int j = 0; j < N_REP; j++) {
    const uint32_t base = part_base + ((kvh * N_REP + j) * p.n_split + split) * PART;
    if (lane == 0) {
      a[base] = m[j];
      a[base + 1] = l[j];
    }
    a[base + 2 + lane] = acc0[j];
    a[base + 2 + lane + 64] = acc1[j];
  }
}

}  // namespace

// rmsnorm (rmsnorm.comp; ops.rs:1-16): y = x * r * w, r = 1 / sqrt(mean(x^2) + eps), per
// token below ctl[2].  256 threads; partial sums of squares per wave, added in wave order.
extern "C" __global__ __launch_bounds__(256) void rmsnorm(const float *w, float *a, const uint32_t *ctl,
                                                           NormPush p) {
#pragma clang fp contract(off)
  __shared__ float part[4];
  const uint32_t tok = blockIdx.y, t = threadIdx.x;
  if (tok >= ctl[2]) return;
  const uint32_t x = p.x_off + tok * p.stride, y = p.y_off + tok * p.stride;
  float ss = 0.0f;
  for (uint32_t i = t; i < p.n; i += 256) {
    const float v = a[x + i];
    ss += v * v;
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) part[t >> 6] = ss;
  __syncthreads();
  const float total = ((part[0] + part[1]) + part[2]) + part[3];
  const float r = 1.0f / sqrtf(total / (float)p.n + p.eps);
  for (uint32_t i = t; i < p.n; i += 256) a[y + i] = a[x + i] * r * w[p.w_off + i];
}

// qkv_prep (qkv_prep.comp): per (head, token) wave, QK-norm + RoPE of the q and k heads (q
// rewritten in place, k into the cache) and the value heads copied to the cache.
// Spec [K_Q8, V_Q8, head_dim, n_rot, gated]; exported for head_dim = n_rot = 128, gated 0.
#define QKV(K8, V8)                                                                            \
  extern "C" __global__ __launch_bounds__(64) void qkv_prep__##K8##_##V8##_128_128_0(         \
      const float *w, float *a, const uint32_t *ctl, f16 *kv, int8_t *kv8, QkvPush p) {       \
    qkv_body<K8, V8>(w, a, ctl, kv, kv8, p);                                                   \
  }
QKV(0, 0)
QKV(0, 1)
QKV(1, 1)

// attention (attention.comp): spec [N_REP, CHUNK, K_Q8, V_Q8, head_dim, q_head].
#define ATTN(R, K8, V8)                                                                          \
  extern "C" __global__ __launch_bounds__(64) void attention__##R##_64_##K8##_##V8##_128_128(    \
      float *a, const uint32_t *ctl, const f16 *kv, const int8_t *kv8, const f16 *kvs, AttnPush p) { \
    (void)kvs;                                                                                   \
    attention_body<R, K8, V8>(a, ctl, kv, kv8, p);                                               \
  }
#define ATTN_REP(K8, V8) ATTN(1, K8, V8) ATTN(2, K8, V8) ATTN(4, K8, V8) ATTN(8, K8, V8)
ATTN_REP(0, 0)
ATTN_REP(0, 1)
ATTN_REP(1, 1)

// attention_merge (attention_merge.comp): o = sum_s w_s acc_s / sum_s w_s l_s with
// w_s = exp(m_s - max m) over the splits that hold positions, in split order.  Spec
// [head_dim, gated] = [128, 0].
extern "C" __global__ __launch_bounds__(128) void attention_merge__128_0(float *a, const uint32_t *ctl,
                                                                          MergePush p) {
  const uint32_t h = blockIdx.x, tok = blockIdx.y, t = threadIdx.x;
  if (tok >= ctl[2]) return;
  const uint32_t used = (ctl[1] + tok + p.chunk) / p.chunk;
  const uint32_t first = p.part_off + tok * p.part_stride + h * p.n_split * PART;
  float big = -1e30f;
  for (uint32_t s = 0; s < used; s++) big = fmaxf(big, a[first + s * PART]);
  float total = 0.0f, o = 0.0f;
  for (uint32_t s = 0; s < used; s++) {
    const uint32_t base = first + s * PART;
    const float wgt = expf(a[base] - big);
    total += wgt * a[base + 1];
    o += wgt * a[base + 2 + t];
  }
  a[p.o_off + tok * p.o_stride + h * HD + t] = o / total;
}

// take_last (take_last.comp): the last token row of a chunk, for the output head.
extern "C" __global__ __launch_bounds__(256) void take_last(float *a, const uint32_t *ctl, LastPush p) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < p.n) a[p.dst_off + i] = a[p.src_off + (ctl[2] - 1) * p.stride + i];
}
