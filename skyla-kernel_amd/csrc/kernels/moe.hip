// MoE top-k dispatch and the elementwise kernels around the expert matvec/matmul, gfx950.
//
// All of them address one f32 arena `a` (plus its u32 and f16 views); offsets are element
// indices (arena.rs:85-113).  The arena's control words are ctl[0] = first token,
// ctl[1] = position, ctl[2] = token count (engine.rs:119-123).
#include "common.h"
#include "route.h"

namespace {

constexpr uint32_t MAX_SLOTS = 1024;  // moe_sort.comp:15 (BATCH * n_used <= 1024)
constexpr uint32_t TILE_MAP = 640;    // words of the tile map before the table (matmul.hip)
constexpr uint32_t TILE_SLOTS = 32;   // slots per expert tile of the grouped matmuls

struct LogitsPush { uint32_t x_off, router_off, logits_off, n_embd, x_stride; };
struct SortPush { uint32_t ids_off, table_off, list_off, n_expert, n_used; };
struct CombinePush { uint32_t x_off, y_off, weights_off, n, stride, n_used; };
struct SiluPush { uint32_t g_off, u_off, n, stride; };
struct HalfPush { uint32_t src_off, dst_off, n, src_stride, dst_stride, per_token; };
}  // namespace

// moe_logits (moe_logits.comp:18-31): logits[tok * n_expert + e] = router_e . x_tok, one
// workgroup of 256 threads per (expert, token); grid [n_expert, tokens, 1].
extern "C" __global__ __launch_bounds__(256) void moe_logits(const float *w, const float *a,
                                                              float *logits, LogitsPush p) {
  __shared__ float part[4];
  const uint32_t e = blockIdx.x, tok = blockIdx.y, tid = threadIdx.x;
  const float4 *row = (const float4 *)(w + p.router_off + e * p.n_embd);
  const float4 *x = (const float4 *)(a + p.x_off + tok * p.x_stride);
  const uint32_t n4 = p.n_embd / 4;
  // one float4's product, its rounding order fixed: ((y y + x x) + z z) + w w as three fmas
  auto dot4 = [](float4 r, float4 v) {
    return __builtin_fmaf(r.w, v.w, __builtin_fmaf(r.z, v.z, __builtin_fmaf(r.x, v.x, r.y * v.y)));
  };
  float s = 0.0f;
  if (n4 != 0 && n4 <= 512) {
    // up to two float4 per thread: both loads issued before the first product (clamped
    // addresses, products kept only where in range), the same sums as the loop below
    const uint32_t i0 = min(tid, n4 - 1), i1 = min(tid + 256, n4 - 1);
    const float4 r0 = row[i0], v0 = x[i0], r1 = row[i1], v1 = x[i1];
    const float t0 = dot4(r0, v0), t1 = dot4(r1, v1);
    s = tid < n4 ? s + t0 : s;
    s = tid + 256 < n4 ? s + t1 : s;
  } else {
    for (uint32_t i = tid; i < n4; i += 256) s += dot4(row[i], x[i]);
  }
  s = group_sum<64>(s);
  if ((tid & 63) == 0) part[tid >> 6] = s;
  __syncthreads();
  if (tid == 0) logits[p.logits_off + tok * gridDim.x + e] = part[0] + part[1] + part[2] + part[3];
}

// moe_logits_t: the runtime's form of moe_logits for a batch (same logits, another grid and
// summation order).  Workgroup (g, h) computes the LG x LG block of experts LG g + [0, LG)
// and tokens LG h + [0, LG): each lane accumulates all LG x LG dot products over its own
// float4 columns (the four waves take interleaved column ranges), the 64 sums are spread
// one per lane by a halving exchange across the wave, and the four waves' sums are added
// in wave order.  Per workgroup that reads 2 LG rows once instead of one expert row and
// one token row per (expert, token): ~32 MB of L2 traffic at 128 x 128 x 2048 instead of
// ~256 MB, which bounded the one-workgroup-per-logit form.
constexpr uint32_t LG = 8;
extern "C" __global__ __launch_bounds__(256) void moe_logits_t(const float *w, const float *a,
                                                                float *logits, LogitsPush p,
                                                                uint32_t n_expert, uint32_t n_tok) {
  __shared__ float part[4][64];
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t e0 = blockIdx.x * LG, t0 = blockIdx.y * LG;
  const uint32_t n4 = p.n_embd / 4;
  const float4 *xr[LG], *rr[LG];
#pragma unroll
  for (uint32_t i = 0; i < LG; i++) {
    xr[i] = (const float4 *)(a + p.x_off + min(t0 + i, n_tok - 1) * p.x_stride);
    rr[i] = (const float4 *)(w + p.router_off + min(e0 + i, n_expert - 1) * p.n_embd);
  }
  float v[LG * LG];  // v[LG ti + ei]
#pragma unroll
  for (uint32_t j = 0; j < LG * LG; j++) v[j] = 0.0f;
  for (uint32_t c = wave * 64 + lane; c < n4; c += 256) {
    float4 xv[LG], rv[LG];
#pragma unroll
    for (uint32_t i = 0; i < LG; i++) {
      xv[i] = xr[i][c];
      rv[i] = rr[i][c];
    }
#pragma unroll
    for (uint32_t ti = 0; ti < LG; ti++)
#pragma unroll
      for (uint32_t ei = 0; ei < LG; ei++)
        v[LG * ti + ei] += xv[ti].x * rv[ei].x + xv[ti].y * rv[ei].y + xv[ti].z * rv[ei].z + xv[ti].w * rv[ei].w;
  }
  // halving exchange: after the step of distance d, lane l holds the sums of the outputs
  // whose index has l's bits >= d; lane l ends with output l
#pragma unroll
  for (uint32_t d = 32, n = 64; d >= 1; d >>= 1, n >>= 1) {
    const bool upper = (lane & d) != 0;
#pragma unroll
    for (uint32_t j = 0; j < n / 2; j++) {
      const float keep = upper ? v[j + n / 2] : v[j], send = upper ? v[j] : v[j + n / 2];
      v[j] = keep + __shfl_xor(send, (int)d, 64);
    }
  }
  part[wave][lane] = v[0];
  __syncthreads();
  if (threadIdx.x < 64) {
    const uint32_t tok = t0 + lane / LG, e = e0 + lane % LG;
    const float sum = ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane];
    if (tok < n_tok && e < n_expert) logits[p.logits_off + tok * n_expert + e] = sum;
  }
}

// moe_route (moe_route.comp:23-74): one workgroup of four waves per token ranks its logits
// (route_ranked), then wave 0 computes the routing weights; tokens at or beyond ctl[2] do
// nothing.
extern "C" __global__ __launch_bounds__(256) void moe_route(float *a, uint32_t *ids, RoutePush p) {
  __shared__ uint32_t sid[16];
  __shared__ float sval[16];
  const uint32_t tok = blockIdx.y;
  const uint32_t n_tok = __builtin_bit_cast(uint32_t, a[2]);
  if (tok >= n_tok) return;
  route_ranked(a, p, tok, threadIdx.x, sid, sval);
  if (threadIdx.x < 64) {
    const uint32_t n_used = min(p.n_used, 16u), t = threadIdx.x;
    const float wt = route_weight(t < n_used ? sval[t] : 0.0f, n_used);
    if (t < n_used) {
      ids[p.ids_off + tok * p.n_used + t] = sid[t];
      a[p.weights_off + tok * p.n_used + t] = wt;
    }
  }
}

// moe_sort (moe_sort.comp:21-55): slot s = tok * n_used + k is routed to ids[s].  Writes
// table[2e] = count, table[2e+1] = start (exclusive scan in expert order) and list[start +
// rank] = s with rank = number of earlier slots of the same expert (stable).  One
// workgroup of four waves; wave w owns the slots [256 w, 256 w + 256) and counts them per
// expert in its own LDS row, so its first slot of expert e goes after the table's start of
// e plus the earlier waves' counts of e.  Each wave then ranks its slots 64 at a time in
// slot order, using ballots to find the lanes that share an expert.  The ids are read once
// (the list writes go to the same arena, so reads from it could not be hoisted past them).
// Beside the table it writes the tile map the grouped matmuls launch over, TILE_MAP words
// before the table: map[0] = the number of (expert, 32-slot tile) entries, and entry i, in
// expert order, as map[1 + 2i] = e | z << 16 and map[2 + 2i] = the expert's list start |
// its slot count << 16 (at most 280 entries: the sum of ceil(c_e / 32) over the experts
// with slots is at most (MAX_SLOTS + 31 * 256) / 32).
extern "C" __global__ __launch_bounds__(256) void moe_sort(uint32_t *a, SortPush p) {
  __shared__ uint32_t count[4][256];  // per wave and expert; then that wave's cursor
  __shared__ uint32_t wsum[4];
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t n = min(a[2] * p.n_used, MAX_SLOTS);
  const uint32_t n_expert = min(p.n_expert, 256u);
  constexpr uint32_t PER_WAVE = MAX_SLOTS / 4, CHUNKS = PER_WAVE / 64;
#pragma unroll
  for (uint32_t w = 0; w < 4; w++) count[w][t] = 0;
  uint32_t mine[CHUNKS];
#pragma unroll
  for (uint32_t j = 0; j < CHUNKS; j++) {
    const uint32_t i = PER_WAVE * wave + 64 * j + lane;
    mine[j] = i < n ? a[p.ids_off + i] : 0xffffffffu;
  }
  __syncthreads();
#pragma unroll
  for (uint32_t j = 0; j < CHUNKS; j++)
    if (mine[j] < n_expert) atomicAdd(&count[wave][mine[j]], 1u);
  __syncthreads();
  // thread t: expert e = t.  Its total over the waves and its tiles, the exclusive scans of
  // both in expert order (one scan of tot | tiles << 16: the totals sum to at most 1024 and
  // the tiles to at most 289, so neither half carries), and each wave's cursor.
  const uint32_t c0 = count[0][t], c1 = count[1][t], c2 = count[2][t], c3 = count[3][t];
  const uint32_t tot = c0 + c1 + c2 + c3;
  const uint32_t tiles = (tot + TILE_SLOTS - 1) / TILE_SLOTS;
  const uint32_t pk = tot | (tiles << 16);
  uint32_t incl = pk;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint32_t o = __shfl_up(incl, d, 64);
    if (lane >= (uint32_t)d) incl += o;
  }
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  uint32_t first = incl - pk;
  for (uint32_t w = 0; w < wave; w++) first += wsum[w];
  const uint32_t start = first & 0xffffu, tile0 = first >> 16;
  // the map only where the arena has room for it before the table (a caller's own layout
  // may put the table first; the runtime then keeps the grouped matmuls off the map)
  const bool has_map = p.table_off >= TILE_MAP;
  uint32_t *map = a + (has_map ? p.table_off - TILE_MAP : 0u);
  if (t < n_expert) {
    a[p.table_off + 2 * t] = tot;
    a[p.table_off + 2 * t + 1] = start;
    if (has_map)
      for (uint32_t z = 0; z < tiles; z++) {
        map[1 + 2 * (tile0 + z)] = t | (z << 16);
        map[2 + 2 * (tile0 + z)] = start | (tot << 16);
      }
  }
  if (t == 0 && has_map) map[0] = (wsum[0] + wsum[1] + wsum[2] + wsum[3]) >> 16;
  count[0][t] = start;
  count[1][t] = start + c0;
  count[2][t] = start + c0 + c1;
  count[3][t] = start + c0 + c1 + c2;
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1;
#pragma unroll
  for (uint32_t j = 0; j < CHUNKS; j++) {
    const uint32_t i = PER_WAVE * wave + 64 * j + lane;
    const uint32_t e = mine[j];
    const bool ok = e < n_expert;  // slots past n hold 0xffffffff
    // lanes with the same expert: intersect the ballots of all 8 expert bits
    uint64_t same = __ballot(ok);
#pragma unroll
    for (int bit = 0; bit < 8; bit++) {
      const uint64_t ones = __ballot(ok && ((e >> bit) & 1u));
      same &= ((e >> bit) & 1u) ? ones : ~ones;
    }
    if (ok) {
      const uint32_t rank = __popcll(same & below);
      const uint32_t at = count[wave][e] + rank;
      a[p.list_off + at] = i;
      // the highest lane of the group advances the wave's cursor
      if ((same >> lane) == 1ull) count[wave][e] = at + 1;
    }
    // a single wave's LDS accesses complete in program order; the fence only keeps the
    // compiler from moving the next step's cursor reads above these writes
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  }
}

// moe_combine (moe_combine.comp:16-27): x[tok] += sum_s w[tok, s] * down[tok * n_used + s],
// summed in route order from 0 as the oracle does (ffn.rs:67-74, model.rs:113-114).
extern "C" __global__ __launch_bounds__(256) void moe_combine(float *a, CombinePush p) {
#pragma clang fp contract(off)
  const uint32_t i = blockIdx.x * 256 + threadIdx.x, tok = blockIdx.y;
  if (i >= p.n) return;
  // the first 16 slots' loads (the engine routes at most 16) all in flight before the sum,
  // which adds them in the same order; any further slots one by one
  constexpr uint32_t MAXU = 16;
  const uint32_t nb = min(p.n_used, MAXU);
  float wv[MAXU], yv[MAXU];
#pragma unroll
  for (uint32_t s = 0; s < MAXU; s++)
    if (s < nb) {
      const uint32_t slot = tok * p.n_used + s;
      wv[s] = a[p.weights_off + slot];
      yv[s] = a[p.y_off + slot * p.stride + i];
    }
  const float x0 = a[p.x_off + tok * p.stride + i];
  float sum = 0.0f;
#pragma unroll
  for (uint32_t s = 0; s < MAXU; s++)
    if (s < nb) sum += wv[s] * yv[s];
  for (uint32_t s = MAXU; s < p.n_used; s++) {
    const uint32_t slot = tok * p.n_used + s;
    sum += a[p.weights_off + slot] * a[p.y_off + slot * p.stride + i];
  }
  a[p.x_off + tok * p.stride + i] = x0 + sum;
}

// silu_mul (silu_mul.comp:15-23): g <- g / (1 + e^-g) * u for tokens below ctl[2].
extern "C" __global__ __launch_bounds__(256) void silu_mul(float *a, const uint32_t *ctl,
                                                            SiluPush p) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x, tok = blockIdx.y;
  if (i >= p.n || tok >= ctl[2]) return;
  const uint32_t g = p.g_off + tok * p.stride + i;
  const float x = a[g];
  a[g] = x / (1.0f + expf(-x)) * a[p.u_off + tok * p.stride + i];
}

// to_half (to_half.metal:13-28): f32 -> f16 copy of the GEMM input rows, 4 per thread,
// rows below ctl[2] * per_token.
extern "C" __global__ __launch_bounds__(256) void to_half(const float *a, f16 *h,
                                                           const uint32_t *ctl, HalfPush p) {
  const uint32_t i = (blockIdx.x * 256 + threadIdx.x) * 4, row = blockIdx.y;
  if (i >= p.n || row >= ctl[2] * p.per_token) return;
  const float4 v = *(const float4 *)(a + p.src_off + row * p.src_stride + i);
  const f16x4 o = {(f16)v.x, (f16)v.y, (f16)v.z, (f16)v.w};
  *(f16x4 *)(h + p.dst_off + row * p.dst_stride + i) = o;
}
