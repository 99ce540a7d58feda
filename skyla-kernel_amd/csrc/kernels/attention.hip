// The rest of the decode step around the weight matvecs, gfx950: RMSNorm, the QK-norm +
// RoPE + KV-cache write, split-K attention over the cache and its merge, and the last-row
// copy of a prefill chunk (graph.rs:48-113, 200-233; the kernels of kernels.rs:186-193).
//
// Contract (bindings, push words, grids) as the engine dispatches them:
//   rmsnorm          [W, A, C]            6 words  grid [1, tokens, 1]
//   qkv_prep         [W, A, C, KV, KV8]  16 words  grid [n_head + 2 n_kv, tokens, 1]
//   attention        [A, C, KV, KV8, KVS] 11 words grid [n_kv, n_split, tokens], 256 threads
//   attention_merge  [A, C]               6 words  grid [n_head, tokens, 1], 1024 threads
//   attention_prep   [W, A, C, KV, KV8]  17 words  grid [n_kv, n_split, 1], 256 threads:
//                    qkv_prep + attention of a single-token step
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
// attention_prep: qkv_prep's and attention's words for a single-token step (17 words)
struct PrepPush {
  uint32_t q_off, k_off, v_off, qn_off, kn_off, kc_off, vc_off, n_kv;
  float eps;
  uint32_t rope_off;
  float mscale;
  uint32_t ks_off, vs_off, part_off, n_split;
  float scale;
  uint32_t part_stride;
  uint32_t cs_off;  // the step's rope pairs (rope_table) in the arena, or NO_TABLE: computed here
};
constexpr uint32_t NO_TABLE = 0xffffffffu;
// attention_prep1: attention_prep's words, then attention_merge's output offset and stride
struct PrepPush1 {
  PrepPush pp;
  uint32_t o_off, o_stride;
};
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

// Writes y0 (element t) and y1 (element t + 64) of one head's cache row.  With `raw`, the
// stored row also goes to LDS as the cache holds it (128 f16, or 128 i8 and the four block
// scales in `sc`), for a reader in the same workgroup.
template <int Q8>
SK_DEV void store_kv(f16 *kv, int8_t *kv8, uint32_t cache, uint32_t scales, uint32_t kv_dim, uint32_t pos,
                     uint32_t head, uint32_t t, float y0, float y1, uint32_t *raw = nullptr,
                     float *sc = nullptr) {
  const uint32_t dst = cache + pos * kv_dim + head * HD;
  if constexpr (!Q8) {
    const f16 h0 = (f16)y0, h1 = (f16)y1;
    kv[dst + t] = h0;
    kv[dst + t + 64] = h1;
    if (raw) {
      ((f16 *)raw)[t] = h0;
      ((f16 *)raw)[t + 64] = h1;
    }
  } else {
    const float s0 = block_max(y0) / 127.0f, s1 = block_max(y1) / 127.0f;
    const int8_t q0 = (int8_t)(s0 > 0.0f ? __builtin_rintf(y0 / s0) : 0.0f);
    const int8_t q1 = (int8_t)(s1 > 0.0f ? __builtin_rintf(y1 / s1) : 0.0f);
    kv8[dst + t] = q0;
    kv8[dst + t + 64] = q1;
    if ((t & 31) == 0) {
      const uint32_t sd = scales + pos * (kv_dim / 32) + head * 4 + t / 32;
      kv[sd] = (f16)s0;
      kv[sd + 2] = (f16)s1;
    }
    if (raw) {
      ((int8_t *)raw)[t] = q0;
      ((int8_t *)raw)[t + 64] = q1;
      if ((t & 31) == 0) {
        sc[t / 32] = (float)(f16)s0;
        sc[t / 32 + 2] = (float)(f16)s1;
      }
    }
  }
}

// QK-norm (rmsnorm.comp over one 128-wide head, weights at nw) and NeoX RoPE (rope.rs:60-68)
// of the pair (element t, element t + 64), one wave per head.
SK_DEV void norm_rope(const float *w, uint32_t nw, uint32_t rope_off, float eps, float mscale, uint32_t pos,
                      uint32_t t, float x0, float x1, float &y0, float &y1, const float *cs = nullptr) {
#pragma clang fp contract(off)
  const float r = 1.0f / sqrtf(wave_sum(x0 * x0 + x1 * x1) / (float)HD + eps);
  const float n0 = x0 * r * w[nw + t], n1 = x1 * r * w[nw + t + 64];
  float c, s;
  if (cs) {  // rope_table's pairs for this position: the same two products
    c = cs[2 * t];
    s = cs[2 * t + 1];
  } else {
    const float angle = (float)pos * w[rope_off + t];
    c = cosf(angle) * mscale;
    s = sinf(angle) * mscale;
  }
  y0 = n0 * c - n1 * s;
  y1 = n0 * s + n1 * c;
}

// rope_table: the (cos, sin) x mscale pairs of the step's position (ctl[1]) for the 64
// rotation frequencies, computed once per decode step into the arena for every layer's
// attention_prep -- its workgroups (one per kv head and split) would each reduce the same
// large angles otherwise.  norm_rope's expressions, so the same values.
struct RopePush { uint32_t rope_off, o_off; float mscale; };
extern "C" __global__ __launch_bounds__(64) void rope_table(const float *w, float *a, const uint32_t *ctl, RopePush p) {
#pragma clang fp contract(off)
  const uint32_t t = threadIdx.x;
  const float angle = (float)ctl[1] * w[p.rope_off + t];
  a[p.o_off + 2 * t] = cosf(angle) * p.mscale;
  a[p.o_off + 2 * t + 1] = sinf(angle) * p.mscale;
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
  float y0, y1;
  norm_rope(w, nw, p.rope_off, p.eps, p.mscale, pos, t, a[src + t], a[src + t + 64], y0, y1);
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

// One workgroup of four waves per (kv head, split of CHUNK positions, token); every load of
// the split is issued up front.  Scores with f16 keys run on the matrix cores: wave w
// computes the N_REP query heads (A, from LDS) against its 16 positions (B, one key row's
// 32 dims per lane group and k-step) in four v_mfma_f32_16x16x32_f16 k-steps, once with
// the heads' f16 high parts and once with their low parts (the heads scaled by a power of
// two first, so hi + lo carries each value to 2^-22 of the head's largest and the products
// with the f16 keys are exact in the f32 sums).  With 8-bit keys, thread t takes dims
// 8 (t % 16) ... of the key rows of positions t / 16 + 16 k (k < 4) and dots them with the
// heads in f32; the 16 partial dots of a row meet in a DPP sum.  The chunk's softmax numerators
// e_p = exp(s_p - m) go through LDS to the value phase, where thread t weights 8 dims
// (8 (t % 16) ...) of the value rows of positions 4 (t / 16) ... 4 (t / 16) + 3; the 16
// position groups are then summed in LDS.  The partial (m, l = sum e_p, acc = sum e_p v_p)
// goes to the part region for attention_merge; it is the same quantity as the reference's
// running (m, l, acc) over the chunk (attention.comp:83-97).  Positions past the token's
// own are masked (e = 0) and read a live row instead, so no load leaves the cache.
//
// PREP (attention_prep, single-token steps): qkv_prep folded in.  Each workgroup norms and
// rotates its own query heads from the raw q rows (one wave per head, the same arithmetic
// as qkv_prep), and the workgroup whose split holds the new position writes that
// position's key and value rows to the cache as qkv_prep would, keeping the stored bytes
// in LDS: its threads take them from there in place of the rows they loaded from the cache
// before the write (the new row and the masked slots clamped to it).
//
// DIRECT (attention_prep1, a grid of one split: every position of the step in the first 64):
// the workgroup writes the merged output itself, o = (acc + 0) / l per dim -- what
// attention_merge computes over one split (its weight is exp(0) = 1 and every other term
// adds zero), so the same bits -- and no partial; o_off / o_stride are the merge's.
template <int N_REP, int K8, int V8, bool PREP = false, bool DIRECT = false>
SK_DEV void attention_body(const float *w, float *a, const uint32_t *ctl, f16 *kv, int8_t *kv8, const AttnPush &p,
                           const PrepPush *pp, uint32_t o_off = 0, uint32_t o_stride = 0) {
  // heads per value reduction round: two keep vp at 16 KB and the workgroup near 20 KB of
  // LDS, so six share a CU (with four heads, 32 KB, LDS allowed four, and a 16k-position
  // step's 2056 workgroups took a third round of eight)
  constexpr int HG = N_REP < 2 ? N_REP : 2;
  // f16 keys: the scores on the matrix cores (MQ); 8-bit keys keep the VALU dots
  constexpr bool MQ = !K8;
  // the A operand's rows: head m % N_REP in row m (rows past the heads repeat them, and
  // their products are not used); a row pitch of 320 B (80 banks) puts the 16 distinct
  // 16 B pieces that a k-step's lanes read (four heads x four dim groups) on distinct banks
  constexpr int QP = HD + 32;
  __shared__ float qs[MQ ? 1 : N_REP][HD];
  __shared__ __attribute__((aligned(16))) f16 qh[2][MQ ? N_REP : 1][MQ ? QP : 8];
  __shared__ int qsh[MQ ? N_REP : 1];
  __shared__ __attribute__((aligned(16))) uint32_t nk[PREP ? 64 : 1], nv[PREP ? 64 : 1];
  __shared__ float nks[PREP ? 4 : 1], nvs[PREP ? 4 : 1];
  __shared__ float es[N_REP][CHUNK];
  __shared__ float wm[4][N_REP];
  __shared__ float4 vp[16][HG * HD / 4];
  __shared__ float lsh[DIRECT ? N_REP : 1];
  const uint32_t kvh = blockIdx.x, split = blockIdx.y, tok = blockIdx.z;
  const uint32_t n_pos = ctl[1] + tok + 1;
  if (tok >= ctl[2] || split * CHUNK >= n_pos) return;
  const uint32_t t = threadIdx.x, wave = t >> 6, kv_dim = p.n_kv * HD;
  const uint32_t begin = split * CHUNK, cnt = min(CHUNK, n_pos - begin);

  // keys: dims [8 kd, 8 kd + 8) of positions kg + 16 k, k < 4 (16 lanes cover a row: every
  // load instruction reads whole cache lines)
  // MQ: lane i of wave w takes position mp = 16 w + i % 16 and dims 8 (mg + 4 k), mg = i / 16:
  // its B operand of k-step k (32 dims) of v_mfma_f32_16x16x32_f16
  const uint32_t kd = t & 15, kg = t >> 4;
  const uint32_t lane = t & 63, mp = 16 * wave + (lane & 15), mg = lane >> 4;
  uint4 kr[4];
  float ksc[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    if constexpr (MQ) {
      const uint32_t kpos = begin + min(mp, cnt - 1);
      kr[k] = *(const uint4 *)(kv + p.kc_off + kpos * kv_dim + kvh * HD + 8 * (mg + 4 * k));
      ksc[k] = 1.0f;
    } else {
      const uint32_t kpos = begin + min(kg + 16 * k, cnt - 1);
      const uint2 r = *(const uint2 *)(kv8 + p.kc_off + kpos * kv_dim + kvh * HD + 8 * kd);
      kr[k] = make_uint4(r.x, r.y, 0u, 0u);
      ksc[k] = (float)kv[p.ks_off + kpos * (kv_dim / 32) + kvh * 4 + (kd >> 2)];
    }
  }
  // values: dims [8 vg, 8 vg + 8) of positions 4 vq + [0, 4)
  const uint32_t vg = t & 15, vq = t >> 4;
  uint4 vr[4];
  float vsc[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const uint32_t vpos = begin + min(4 * vq + q, cnt - 1);
    if constexpr (!V8) {
      vr[q] = *(const uint4 *)(kv + p.vc_off + vpos * kv_dim + kvh * HD + 8 * vg);
      vsc[q] = 1.0f;
    } else {
      const uint2 r = *(const uint2 *)(kv8 + p.vc_off + vpos * kv_dim + kvh * HD + 8 * vg);
      vr[q] = make_uint4(r.x, r.y, 0u, 0u);
      vsc[q] = (float)kv[p.vs_off + vpos * (kv_dim / 32) + kvh * 4 + (vg >> 2)];
    }
  }
  // the scaled query head j (this lane's dims lane and lane + 64; the caller's wave holds
  // the whole head).  MQ: as f16 hi + lo parts of v 2^sh, sh putting the head's largest
  // |v| in [2^10, 2^11): hi + lo is v 2^sh to 2^-22 of that largest value, nothing
  // overflows, and each product with an f16 key is exact in the f32 accumulation
  auto put_q = [&](uint32_t j, float v0, float v1) {
    if constexpr (MQ) {
      const float big = wave_max(fmaxf(fabsf(v0), fabsf(v1)));
      const int sh = big > 0.0f ? 11 - __builtin_amdgcn_frexp_expf(big) : 0;
      const float s0 = ldexpf(v0, sh), s1 = ldexpf(v1, sh);
      const f16 h0 = (f16)s0, h1 = (f16)s1;
      qh[0][j][lane] = h0;
      qh[0][j][lane + 64] = h1;
      qh[1][j][lane] = (f16)(s0 - (float)h0);
      qh[1][j][lane + 64] = (f16)(s1 - (float)h1);
      if (lane == 0) qsh[j] = sh;
    } else {
      qs[j][lane] = v0;
      qs[j][lane + 64] = v1;
    }
  };
  // the query heads of this kv head, scaled
  const uint32_t q_base = p.q_off + tok * p.q_stride + kvh * N_REP * HD;
  if constexpr (PREP) {
    const uint32_t pos = ctl[1];
    const float *cs = pp->cs_off != NO_TABLE ? a + pp->cs_off : nullptr;
    for (uint32_t j = wave; j < (uint32_t)N_REP; j += 4) {
      float y0, y1;
      norm_rope(w, pp->qn_off, pp->rope_off, pp->eps, pp->mscale, pos, lane, a[q_base + j * HD + lane],
                a[q_base + j * HD + lane + 64], y0, y1, cs);
      put_q(j, y0 * p.scale, y1 * p.scale);
    }
    if (pos / CHUNK == split) {
      if (wave == 0) {
        float y0, y1;
        const uint32_t src = pp->k_off + kvh * HD;
        norm_rope(w, pp->kn_off, pp->rope_off, pp->eps, pp->mscale, pos, lane, a[src + lane], a[src + lane + 64], y0,
                  y1, cs);
        store_kv<K8>(kv, kv8, p.kc_off, p.ks_off, kv_dim, pos, kvh, lane, y0, y1, nk, nks);
      } else if (wave == 1) {
        const uint32_t src = pp->v_off + kvh * HD;
        store_kv<V8>(kv, kv8, p.vc_off, p.vs_off, kv_dim, pos, kvh, lane, a[src + lane], a[src + lane + 64], nv, nvs);
      }
    }
  } else if constexpr (MQ) {
    for (uint32_t j = wave; j < (uint32_t)N_REP; j += 4)
      put_q(j, a[q_base + j * HD + lane] * p.scale, a[q_base + j * HD + lane + 64] * p.scale);
  } else {
    for (uint32_t i = t; i < N_REP * HD; i += 256) qs[i / HD][i % HD] = a[q_base + i] * p.scale;
  }
  __syncthreads();
  if constexpr (PREP) {
    if (ctl[1] / CHUNK == split) {  // the new row (pl = cnt - 1) and the masked slots clamped to it
      const uint32_t pl = cnt - 1;
      if constexpr (MQ) {
        if (mp >= pl)
#pragma unroll
          for (int k = 0; k < 4; k++) kr[k] = ((const uint4 *)nk)[mg + 4 * k];
      } else {
#pragma unroll
        for (int k = 0; k < 4; k++)
          if (kg + 16 * k >= pl) {
            const uint2 u = ((const uint2 *)nk)[kd];
            kr[k] = make_uint4(u.x, u.y, 0u, 0u);
            ksc[k] = nks[kd >> 2];
          }
      }
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (4 * vq + q >= pl) {
          if constexpr (!V8) {
            vr[q] = ((const uint4 *)nv)[vg];
          } else {
            const uint2 u = ((const uint2 *)nv)[vg];
            vr[q] = make_uint4(u.x, u.y, 0u, 0u);
            vsc[q] = nvs[vg >> 2];
          }
        }
    }
  }

  float mx[N_REP];
  if constexpr (MQ) {
    // scores on the matrix cores: A rows are the query heads (hi, then lo parts, each k-step
    // 32 dims), B columns the wave's 16 positions; lane i then holds the scores of heads
    // 4 (i / 16) + r (r < 4, those below N_REP) at position mp
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t m = lane & (N_REP - 1);  // A row lane % 16 holds head (lane % 16) % N_REP
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const f16x8 bk = __builtin_bit_cast(f16x8, kr[k]);
#pragma unroll
      for (int part = 0; part < 2; part++)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const f16x8 *)&qh[part][m][8 * (mg + 4 * k)], bk, acc, 0, 0, 0);
    }
    // heads of this lane: 4 mg + r; with at most four heads, only mg = 0 holds any
    constexpr int MGS = N_REP > 4 ? 2 : 1;
    float sr[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const uint32_t h = 4 * mg + r;
      sr[r] = -INFINITY;
      if (h < (uint32_t)N_REP && mp < cnt) sr[r] = ldexpf(acc[r], -qsh[h < (uint32_t)N_REP ? h : 0]);
      // the head's maximum over the wave's 16 positions (one DPP row)
      float v = sr[r];
      v = fmaxf(v, dpp_f<0xb1>(v));
      v = fmaxf(v, dpp_f<0x4e>(v));
      v = fmaxf(v, dpp_f<0x141>(v));
      v = fmaxf(v, dpp_f<0x140>(v));
      if ((lane & 15) == 0 && h < (uint32_t)N_REP) wm[wave][h] = v;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < N_REP; j++) mx[j] = fmaxf(fmaxf(wm[0][j], wm[1][j]), fmaxf(wm[2][j], wm[3][j]));
    if (mg < (uint32_t)MGS) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int h = MGS == 1 ? r : (mg ? 4 + r : r);
        if (h < N_REP) {
          const float mh = MGS == 1 ? mx[r < N_REP ? r : 0] : (mg ? mx[(4 + r) % N_REP] : mx[r % N_REP]);
          es[h][mp] = mp < cnt ? expf(sr[r] - mh) : 0.0f;
        }
      }
    }
    __syncthreads();
  } else {
    float sc[4][N_REP];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float key[8];
      const uint32_t wd[2] = {kr[k].x, kr[k].y};
#pragma unroll
      for (int bb = 0; bb < 8; bb++) key[bb] = (float)(int8_t)((wd[bb >> 2] >> (8 * (bb & 3))) & 255u) * ksc[k];
#pragma unroll
      for (int j = 0; j < N_REP; j++) {
        const float4 q0 = *(const float4 *)&qs[j][8 * kd], q1 = *(const float4 *)&qs[j][8 * kd + 4];
        float s = 0.0f;
        s = __builtin_fmaf(q0.x, key[0], s);
        s = __builtin_fmaf(q0.y, key[1], s);
        s = __builtin_fmaf(q0.z, key[2], s);
        s = __builtin_fmaf(q0.w, key[3], s);
        s = __builtin_fmaf(q1.x, key[4], s);
        s = __builtin_fmaf(q1.y, key[5], s);
        s = __builtin_fmaf(q1.z, key[6], s);
        s = __builtin_fmaf(q1.w, key[7], s);
        sc[k][j] = lane_sum<16>(s);  // the row's dot, in all 16 lanes
      }
    }
    // The 16 lanes of a group hold the same 4 x N_REP scores, so the wave maximum needs only
    // the two cross-group steps, and each lane then exponentiates its own share of them.
#pragma unroll
    for (int j = 0; j < N_REP; j++) {
      float m = -INFINITY;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if (kg + 16 * k >= cnt) sc[k][j] = -INFINITY;
        m = fmaxf(m, sc[k][j]);
      }
      m = fmaxf(m, __shfl_xor(m, 16, 64));
      m = fmaxf(m, __shfl_xor(m, 32, 64));
      if ((t & 63) == 0) wm[wave][j] = m;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < N_REP; j++) mx[j] = fmaxf(fmaxf(wm[0][j], wm[1][j]), fmaxf(wm[2][j], wm[3][j]));
    constexpr int NS = 4 * N_REP;  // scores of a lane group: (position k, head j) = (i / N_REP, i % N_REP)
#pragma unroll
    for (int i0 = 0; i0 < NS; i0 += 16) {
      const int i = i0 + (int)kd;
      if (i < NS) {
        float s = -INFINITY, m = 0.0f;
#pragma unroll
        for (int u = i0; u < (i0 + 16 < NS ? i0 + 16 : NS); u++)
          if (u == i) {
            s = sc[u / N_REP][u % N_REP];
            m = mx[u % N_REP];
          }
        const uint32_t pk = kg + 16 * (uint32_t)(i / N_REP);
        es[i % N_REP][pk] = pk < cnt ? expf(s - m) : 0.0f;
      }
    }
    __syncthreads();
  }
  // l = sum of the split's e per head: wave 0 adds the LDS rows while the others go on
  float lrow[N_REP];
  if (wave == 0) {
#pragma unroll
    for (int j = 0; j < N_REP; j++) lrow[j] = wave_sum(es[j][t]);
    if constexpr (DIRECT) {  // every thread divides by l (read after the value round's barrier)
#pragma unroll
      for (int j = 0; j < N_REP; j++)
        if (t == 0) lsh[j] = lrow[j];
    }
  }

  float v[4][8];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    if constexpr (!V8) {
      const uint32_t wd[4] = {vr[q].x, vr[q].y, vr[q].z, vr[q].w};
#pragma unroll
      for (int h = 0; h < 4; h++) {
        const f16x2 x = as_f16x2(wd[h]);
        v[q][2 * h] = (float)x.x;
        v[q][2 * h + 1] = (float)x.y;
      }
    } else {
      const uint32_t wd[2] = {vr[q].x, vr[q].y};
#pragma unroll
      for (int bb = 0; bb < 8; bb++) v[q][bb] = (float)(int8_t)((wd[bb >> 2] >> (8 * (bb & 3))) & 255u) * vsc[q];
    }
  }
  const uint32_t part_base = p.part_off + tok * p.part_stride;
#pragma unroll
  for (int h0 = 0; h0 < N_REP; h0 += HG) {
    if (h0 != 0) __syncthreads();  // the previous round's sums are read
#pragma unroll
    for (int j = 0; j < HG; j++) {
      float acc[8];
#pragma unroll
      for (int i = 0; i < 8; i++) acc[i] = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float ep = es[h0 + j][4 * vq + q];
#pragma unroll
        for (int i = 0; i < 8; i++) acc[i] = __builtin_fmaf(ep, v[q][i], acc[i]);
      }
      vp[vq][(j * HD + 8 * vg) / 4] = make_float4(acc[0], acc[1], acc[2], acc[3]);
      vp[vq][(j * HD + 8 * vg) / 4 + 1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
    }
    __syncthreads();
    for (uint32_t o = t; o < HG * HD; o += 256) {
      float sum = 0.0f;
#pragma unroll
      for (int g = 0; g < 16; g++) sum += ((const float *)vp[g])[o];
      const uint32_t j = h0 + o / HD;
      if constexpr (DIRECT)
        a[o_off + tok * o_stride + (kvh * N_REP + j) * HD + o % HD] = (sum + 0.0f) / lsh[j];
      else
        a[part_base + ((kvh * N_REP + j) * p.n_split + split) * PART + 2 + o % HD] = sum;
    }
  }
  if constexpr (DIRECT) return;
  if (t < N_REP) {
    const uint32_t base = part_base + ((kvh * N_REP + t) * p.n_split + split) * PART;
    float l = 0.0f, m = 0.0f;
#pragma unroll
    for (int j = 0; j < N_REP; j++)
      if ((uint32_t)j == t) {
        m = mx[j];
        l = lrow[j];
      }
    a[base] = m;
    a[base + 1] = l;
  }
}

}  // namespace

// rmsnorm (rmsnorm.comp; ops.rs:1-16): y = x * r * w, r = 1 / sqrt(mean(x^2) + eps), per
// token below ctl[2].  256 threads; rows of at most 4096 floats at 16-byte aligned offsets
// (every arena row and norm table) are read once as float4, all loads in flight together,
// and kept in registers for the scaling; other rows take a plain loop.  Partial sums of
// squares per wave, added in wave order.
extern "C" __global__ __launch_bounds__(256) void rmsnorm(const float *w, float *a, const uint32_t *ctl,
                                                           NormPush p) {
#pragma clang fp contract(off)
  __shared__ float part[4];
  const uint32_t tok = blockIdx.y, t = threadIdx.x;
  if (tok >= ctl[2]) return;
  const uint32_t x = p.x_off + tok * p.stride, y = p.y_off + tok * p.stride;
  if (((x | y | p.w_off | p.n) & 3u) == 0 && p.n <= 4096) {
    float4 yv[4];
    norm_row4(a + x, w + p.w_off, p.n, p.eps, yv);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t i = t + 256 * k;
      if (i < (p.n >> 2)) ((float4 *)(a + y))[i] = yv[k];
    }
    return;
  }
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
// Six waves per SIMD for the forms of at most four query heads per kv head (at most 80
// VGPRs, no spill; about 20 KB of LDS, six workgroups per CU); eight heads keep their
// registers.
#define ATTN(R, K8, V8)                                                                          \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(R == 8 ? 1 : 6))) void attention__##R##_64_##K8##_##V8##_128_128(   \
      float *a, const uint32_t *ctl, const f16 *kv, const int8_t *kv8, const f16 *kvs, AttnPush p) { \
    (void)kvs;                                                                                   \
    attention_body<R, K8, V8>(nullptr, a, ctl, const_cast<f16 *>(kv), const_cast<int8_t *>(kv8), p, nullptr); \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(R == 8 ? 1 : 6))) void attention_prep__##R##_64_##K8##_##V8##_128_128( \
      const float *w, float *a, const uint32_t *ctl, f16 *kv, int8_t *kv8, PrepPush pp) {        \
    const AttnPush p = {pp.q_off, pp.part_off, pp.kc_off, pp.vc_off, pp.n_kv, pp.n_split,         \
                        pp.scale, 0u, pp.part_stride, pp.ks_off, pp.vs_off};                     \
    attention_body<R, K8, V8, true>(w, a, ctl, kv, kv8, p, &pp);                                 \
  }                                                                                              \
  extern "C" __global__ __launch_bounds__(256) void attention_prep1__##R##_64_##K8##_##V8##_128_128( \
      const float *w, float *a, const uint32_t *ctl, f16 *kv, int8_t *kv8, PrepPush1 q) {        \
    const PrepPush &pp = q.pp;                                                                   \
    const AttnPush p = {pp.q_off, pp.part_off, pp.kc_off, pp.vc_off, pp.n_kv, pp.n_split,         \
                        pp.scale, 0u, pp.part_stride, pp.ks_off, pp.vs_off};                     \
    attention_body<R, K8, V8, true, true>(w, a, ctl, kv, kv8, p, &pp, q.o_off, q.o_stride);      \
  }
#define ATTN_REP(K8, V8) ATTN(1, K8, V8) ATTN(2, K8, V8) ATTN(4, K8, V8) ATTN(8, K8, V8)
ATTN_REP(0, 0)
ATTN_REP(0, 1)
ATTN_REP(1, 1)

// attention_merge (attention_merge.comp): o = sum_s w_s acc_s / sum_s w_s l_s with
// w_s = exp(m_s - max m) over the splits that hold positions.  Spec [head_dim, gated] =
// [128, 0].  One workgroup of 1024 threads per (head, token).  Wave w takes the splits
// s = w + 16 i; lane l holds dims 2 l and 2 l + 1.  Every load of a round of 1024 splits is
// issued before any arithmetic: lane j loads (m, l) of the wave's split i = j, and each lane
// its two dims of the wave's splits, MG at a time.  A wave keeps its own running maximum
// M_w, and its sums over its splits weighted by exp(m_s - M_w); the waves then meet in LDS:
// M = max M_w, and each wave's sums are scaled by exp(M_w - M) before they are added in
// wave order.  That is the same quantity as the reference's single pass with M from the
// start, in another rounding: exp(m_s - M_w) exp(M_w - M) for exp(m_s - M).  Over a single
// split every factor is exp(0) = 1, so o = (acc + 0) / l, the bits attention_prep1 writes.
constexpr uint32_t MAX_SPLITS = 4096;  // 262144 positions; the engine's arena stays below
constexpr uint32_t MG = 24;            // a wave's splits whose loads are in flight together

extern "C" __global__ __launch_bounds__(1024) void attention_merge__128_0(float *a, const uint32_t *ctl,
                                                                           MergePush p) {
  __shared__ float wmax[16], wl[16];
  __shared__ float2 sums[16][HD / 2];
  const uint32_t h = blockIdx.x, tok = blockIdx.y, t = threadIdx.x, wave = t >> 6, lane = t & 63;
  if (tok >= ctl[2]) return;
  const uint32_t used = min(min((ctl[1] + tok + p.chunk) / p.chunk, p.n_split), MAX_SPLITS);
  const uint32_t first = p.part_off + tok * p.part_stride + h * p.n_split * PART;
  float mw = -INFINITY, lw = 0.0f, ax = 0.0f, ay = 0.0f;
  for (uint32_t base = 0; base < used; base += 1024) {
    // this pass's splits of the wave: s_i = base + wave + 16 i, i < n_i
    const uint32_t s0 = base + wave;
    const uint32_t n_i = s0 < used ? min(64u, (used - s0 + 15) / 16) : 0u;
    if (n_i == 0) break;  // wave-uniform; no later round holds a split of this wave either
    const uint32_t sj = s0 + 16 * lane;
    const bool live = lane < n_i;
    const float mj = live ? a[first + sj * PART] : -INFINITY;
    const float lj = live ? a[first + sj * PART + 1] : 0.0f;
    float2 v[MG];
#pragma unroll
    for (uint32_t i = 0; i < MG; i++)
      v[i] = i < n_i ? *(const float2 *)(a + first + (s0 + 16 * i) * PART + 2 + 2 * lane) : make_float2(0.f, 0.f);
    const float mn = fmaxf(mw, wave_max(mj));
    const float r = expf(mw - mn);  // 0 in the first round (mw = -inf)
    const float wj = expf(mj - mn);  // 0 for lanes past n_i
    lw = __builtin_fmaf(lw, r, wave_sum(wj * lj));
    ax *= r;
    ay *= r;
#pragma unroll
    for (uint32_t i = 0; i < MG; i++) {
      const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wj), (int)i));
      ax = __builtin_fmaf(wi, v[i].x, ax);
      ay = __builtin_fmaf(wi, v[i].y, ay);
    }
    for (uint32_t i = MG; i < n_i; i++) {  // past MG splits of the wave in one round (long contexts)
      const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wj), (int)i));
      const float2 u = *(const float2 *)(a + first + (s0 + 16 * i) * PART + 2 + 2 * lane);
      ax = __builtin_fmaf(wi, u.x, ax);
      ay = __builtin_fmaf(wi, u.y, ay);
    }
    mw = mn;
  }
  if (lane == 0) wmax[wave] = mw;
  __syncthreads();
  float big = wmax[0];
#pragma unroll
  for (int w = 1; w < 16; w++) big = fmaxf(big, wmax[w]);
  const float f = expf(mw - big);  // 0 for a wave without splits (mw = -inf)
  sums[wave][lane] = make_float2(ax * f, ay * f);
  if (lane == 0) wl[wave] = lw * f;
  __syncthreads();
  if (t < HD) {
    float o = 0.0f, total = 0.0f;
#pragma unroll
    for (int g = 0; g < 16; g++) {
      o += ((const float *)sums[g])[t];
      total += wl[g];
    }
    a[p.o_off + tok * p.o_stride + h * HD + t] = o / total;
  }
}

// attention_merge for batched steps (prefill chunks, grid [ceil(n_head / 4), tokens] by the
// runtime): one wave per (head, token), lane l the head's dims 2l and 2l + 1.  The split
// weights exp(m_s - M) are formed 64 at a time, one per lane, and broadcast by readlane (the
// split index is wave-uniform).  The same quantity as attention_merge__128_0 in another
// summation order; a prefill token has few splits, which the 1024-thread form leaves idle.
extern "C" __global__ __launch_bounds__(256) void attention_merge_t__128_0(float *a, const uint32_t *ctl,
                                                                             MergePush p, uint32_t n_head,
                                                                             uint32_t n_tok) {
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t h = blockIdx.x * 4 + wave, tok = blockIdx.y;
  (void)n_tok;
  if (tok >= ctl[2] || h >= n_head) return;
  const uint32_t used = min(min((ctl[1] + tok + p.chunk) / p.chunk, p.n_split), MAX_SPLITS);
  const uint32_t first = p.part_off + tok * p.part_stride + h * p.n_split * PART;
  float *o = a + p.o_off + tok * p.o_stride + h * HD + 2 * lane;
  if (used <= 16) {
    // at most 16 splits (a prefill chunk within 1024 positions): every load in flight at
    // once, then the arithmetic below in the same order (the same bits)
    float ml = -INFINITY, ll = 0.0f, vx[16], vy[16];
    if (lane < used) {
      ml = a[first + lane * PART];
      ll = a[first + lane * PART + 1];
    }
#pragma unroll
    for (uint32_t j = 0; j < 16; j++)
      if (j < used) {
        vx[j] = a[first + j * PART + 2 + 2 * lane];
        vy[j] = a[first + j * PART + 3 + 2 * lane];
      }
    const float big = wave_max(ml);
    const float wl = lane < used ? expf(ml - big) : 0.0f;
    float total = lane < used ? __builtin_fmaf(wl, ll, 0.0f) : 0.0f;
    float ox = 0.0f, oy = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < 16; j++)
      if (j < used) {
        const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), (int)j));
        ox = __builtin_fmaf(wj, vx[j], ox);
        oy = __builtin_fmaf(wj, vy[j], oy);
      }
    total = wave_sum(total);
    o[0] = ox / total;
    o[1] = oy / total;
    return;
  }
  float big = -INFINITY;
  for (uint32_t s = lane; s < used; s += 64) big = fmaxf(big, a[first + s * PART]);
  big = wave_max(big);
  float total = 0.0f, ox = 0.0f, oy = 0.0f;
  for (uint32_t s0 = 0; s0 < used; s0 += 64) {
    const uint32_t s = s0 + lane;
    const float wl = s < used ? expf(a[first + s * PART] - big) : 0.0f;
    if (s < used) total = __builtin_fmaf(wl, a[first + s * PART + 1], total);
    const uint32_t n = min(used - s0, 64u);
    for (uint32_t j = 0; j < n; j++) {
      const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), (int)j));
      const float *v = a + first + (s0 + j) * PART + 2 + 2 * lane;
      ox = __builtin_fmaf(wj, v[0], ox);
      oy = __builtin_fmaf(wj, v[1], oy);
    }
  }
  total = wave_sum(total);
  o[0] = ox / total;
  o[1] = oy / total;
}

// take_last (take_last.comp): the last token row of a chunk, for the output head.
extern "C" __global__ __launch_bounds__(256) void take_last(float *a, const uint32_t *ctl, LastPush p) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i < p.n) a[p.dst_off + i] = a[p.src_off + (ctl[2] - 1) * p.stride + i];
}
