// Chained decode matvecs for gfx950: matvec_chain runs a run of dependent dense decode
// matvec launches (the stages: q+k+v, o, gate+up, down, ... as the engine records them,
// graph.rs:23-34, each a fused launch of one to four dispatches) as one persistent launch.
//
// Why.  Each kernel launch on MI355X costs ~2.3 us before any work, and a small decode
// matvec ramps up and drains: a Qwen3-8B decode layer's four matvec launches take ~37 us
// for 122 MB that the HBM streams in ~21 us.  Here one workgroup per CU streams its share
// of every stage's weights into an LDS ring with direct-to-LDS buffer loads, issued by two
// loader waves that run up to AHEAD chunks ahead of the computation, across stage
// boundaries.  Eight consumer waves compute each chunk from LDS.  Between stages the
// workgroups meet at a grid barrier (a device-scope arrival count); while they wait, the
// next stage's weights are already in flight.
//
// Stage kinds (chain_table.h; the runtime chains only launches of these shapes):
//   CHAIN_Q4K_4096   Q4_K, n_in = 4096, chunk = 8 rows.  The arithmetic is the K-split
//                    form's (matvec_q4k_ks_body, matvec.hip): wave w takes super-blocks
//                    2w and 2w + 1, lane = (row pair, 16-byte unit), f32 FMAs of exact
//                    integer quants, the eight wave partials added in wave order; so each
//                    output is bit-identical to that kernel's.
//   CHAIN_Q6K_12288  Q6_K, n_in = 12288, chunk = 2 rows.  Wave w takes super-blocks
//                    [6w, 6w + 6) of both rows, lane = (row, 64-value unit) (48 of 64 lanes
//                    busy); the unit's arithmetic is matvec_q6k_body's (quants rebuilt as
//                    bytes, f32 FMAs, -32 * sum(x) bias, d * sc per 16 values).
//
// Chunk layout in a ring slot (bytes; every piece is 16 B, loaded in piece order):
//   Q4_K: [0, 16384) qs of rows 0..7 (2048 B each), [16384, 18432) their headers (256 B)
//   Q6_K: [0, 12288) ql of rows 0..1, [12288, 18432) qh, [18432, 19968) scales,
//         [19968, 20160) d
// Pieces past a chunk's data load from past the buffer's end and read zero; rows past
// n_out are clamped to the last row (their outputs are not stored).
//
// Synchronisation.
//   * Ring: every wave runs the same sequence of workgroup barriers (one per chunk, one per
//     stage boundary).  A loader waits for its own loads of chunk c (vmcnt counts them, in
//     order) before the barrier of chunk c, and after it refills the slot of chunk c - 1,
//     which every consumer finished before that barrier.
//   * Grid: activations are read with device-coherent loads, since the previous stage's
//     outputs come from other workgroups, on other XCDs; outputs are written with
//     device-coherent stores by wave 0, which waits for them to complete, counts its
//     workgroup, then waits until the count reaches (stage + 1) x workgroups.
//     The wait is bounded (time-out flag in sync[1], then the launch runs on): every wave
//     exits even if the workgroups were not all resident.  The last workgroup to count
//     itself at the last stage resets the count, so each launch starts at zero.
// The runtime launches one workgroup per CU (the ring holds one per CU).
#include "common.h"
#include "chain_table.h"

namespace {

constexpr int CONSUMERS = 8, LOADERS = 2;
static_assert(64 * (CONSUMERS + LOADERS) == CHAIN_THREADS, "chain workgroup shape");
constexpr int KL = 11;                                    // loads per chunk per loader wave
constexpr uint32_t SLOT = LOADERS * KL * 1024;            // bytes per ring slot
constexpr int RING = 6, AHEAD = RING - 1;                 // slots; chunks in flight
constexpr uint32_t OOB = 0xfffffff0u;                     // a load offset past any buffer
constexpr uint32_t SPIN_LIMIT = 1u << 20;                 // polls before a time-out (~1-2 s)
static_assert(KL * (AHEAD - 1) < 64, "vmcnt holds at most 63");

typedef __attribute__((address_space(3))) void lds_void;
typedef const __attribute__((address_space(4))) ChainStage CStage;
typedef __attribute__((address_space(1))) float gfloat;

// vmcnt(N) with the other counters unconstrained (gfx9 s_waitcnt encoding)
template <int N>
SK_DEV void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}
// until at most m chunks' loads of this loader wave are outstanding
SK_DEV void wait_chunks(uint32_t m) {
  switch (m) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<KL>(); break;
    case 2: wait_vm<2 * KL>(); break;
    case 3: wait_vm<3 * KL>(); break;
    default: wait_vm<4 * KL>(); break;
  }
}
static_assert(AHEAD - 1 == 4, "wait_chunks covers 0..AHEAD-1");

// workgroup barrier after this wave's LDS accesses (global memory is not waited for)
SK_DEV void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

SK_DEV float4 ld_coherent(BufRes r, uint32_t off) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));  // sc1
}

// chunks of a stage that workgroup wg computes (chunk g goes to workgroup g % nwg)
SK_DEV uint32_t chunks_of(uint32_t n_chunks, uint32_t wg, uint32_t nwg) {
  return n_chunks > wg ? (n_chunks - wg + nwg - 1) / nwg : 0;
}

// The fields of a stage that a wave uses per chunk, read once per stage into scalar
// registers (a table read per chunk would put a scalar-memory round trip in every chunk).
// Segments past n_seg have g_end = ~0, so the segment of chunk g is the number of g_end <= g.
struct LoaderView {
  uint32_t kind, w_records, nc;
  uint64_t w;
  uint32_t o[4][4], n_out[4], g_end[4];
};
struct ConsumerView {
  uint32_t kind, accum, x_off, nc;
  uint64_t x, y;
  uint32_t n_out[4], y_off[4], g_end[4];
};

SK_DEV LoaderView loader_view(CStage *st, uint32_t wg, uint32_t nwg) {
  LoaderView v;
  v.kind = st->kind;
  v.w_records = st->w_records;
  v.nc = chunks_of(st->n_chunks, wg, nwg);
  v.w = st->w;
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int k = 0; k < 4; k++) v.o[i][k] = st->seg[i].o[k];
    v.n_out[i] = st->seg[i].n_out;
    v.g_end[i] = st->seg[i].g_end;
  }
  return v;
}

SK_DEV ConsumerView consumer_view(CStage *st, uint32_t wg, uint32_t nwg) {
  ConsumerView v;
  v.kind = st->kind;
  v.accum = st->accum;
  v.x_off = st->x_off;
  v.nc = chunks_of(st->n_chunks, wg, nwg);
  v.x = st->x;
  v.y = st->y;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    v.n_out[i] = st->seg[i].n_out;
    v.y_off[i] = st->seg[i].y_off;
    v.g_end[i] = st->seg[i].g_end;
  }
  return v;
}

// v[i] selected by a wave-uniform or per-lane index, without indexing an array
SK_DEV uint32_t pick(const uint32_t (&v)[4], uint32_t i) {
  return i == 0 ? v[0] : i == 1 ? v[1] : i == 2 ? v[2] : v[3];
}

// segment of chunk g, and its first row
template <typename V>
SK_DEV void locate(const V &v, uint32_t g, uint32_t &seg, uint32_t &row0) {
  const uint32_t i = (uint32_t)(g >= v.g_end[0]) + (uint32_t)(g >= v.g_end[1]) + (uint32_t)(g >= v.g_end[2]);
  const uint32_t g0 = i == 0 ? 0u : i == 1 ? v.g_end[0] : i == 2 ? v.g_end[1] : v.g_end[2];
  seg = i;
  row0 = (g - g0) * (v.kind == CHAIN_Q4K_4096 ? 8u : 2u);
}

// Loader wave L's share of chunk g, into ring slot `dst`: 1 KiB blocks L, L + 2, .., one
// 16-byte piece per lane.  The block index is a compile-time constant in each step, so
// which region (and, for most blocks, which row) a block holds is too, and a step costs a
// few scalar operations and one or two vector ones.
template <int L>
SK_DEV void issue(const LoaderView &v, uint32_t g, unsigned char *dst, uint32_t lane) {
  uint32_t si, row0;
  locate(v, g, si, row0);
  const uint32_t o0 = si == 0 ? v.o[0][0] : si == 1 ? v.o[1][0] : si == 2 ? v.o[2][0] : v.o[3][0];
  const uint32_t o1 = si == 0 ? v.o[0][1] : si == 1 ? v.o[1][1] : si == 2 ? v.o[2][1] : v.o[3][1];
  const uint32_t o2 = si == 0 ? v.o[0][2] : si == 1 ? v.o[1][2] : si == 2 ? v.o[2][2] : v.o[3][2];
  const uint32_t o3 = si == 0 ? v.o[0][3] : si == 1 ? v.o[1][3] : si == 2 ? v.o[2][3] : v.o[3][3];
  const uint32_t last = pick(v.n_out, si) - 1;
  const BufRes r = buf_res((const void *)v.w, v.w_records);
  auto row = [&](uint32_t i) { return min(row0 + i, last); };
  if (v.kind == CHAIN_Q4K_4096) {
#pragma unroll
    for (int k = 0; k < KL; k++) {
      const int blk = LOADERS * k + L;
      uint32_t off = OOB;
      if (blk < 16)  // qs: row blk / 2, units 64 (blk % 2) + lane
        off = 16u * (o0 + row(blk >> 1) * 128u + (blk & 1) * 64u + lane);
      else if (blk < 18)  // headers: rows 4 (blk - 16) + lane / 16
        off = 16u * (o1 + row(4 * (blk - 16) + (lane >> 4)) * 16u + (lane & 15u));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(dst + blk * 1024), 16, off, 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int k = 0; k < KL; k++) {
      const int blk = LOADERS * k + L;
      uint32_t off = OOB;
      if (blk < 12) {  // ql: row blk / 6, units 64 (blk % 6) + lane
        off = 16u * (o0 + row(blk / 6) * 384u + (blk % 6) * 64u + lane);
      } else if (blk < 18) {  // qh: row (blk - 12) / 3
        off = 16u * (o1 + row((blk - 12) / 3) * 192u + ((blk - 12) % 3) * 64u + lane);
      } else if (blk == 18) {  // scales: pieces 0..63 of 96 (row = piece / 48)
        const uint32_t i = lane >= 48;
        off = 16u * (o2 + row(i) * 48u + lane - 48u * i);
      } else if (blk == 19) {  // scales 64..95 (row 1), then d: 12 pieces, 6 per row
        if (lane < 32) {
          off = 16u * (o2 + row(1) * 48u + 16u + lane);
        } else if (lane < 44) {
          const uint32_t q = lane - 32, i = q >= 6;
          off = 2u * (o3 + row(i) * 48u) + 16u * (q - 6 * i);
        }
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(dst + blk * 1024), 16, off, 0, 0, 0);
    }
  }
}

// Outputs.  Wave 0 writes a chunk's rows after the barrier that follows its computation:
// the eight wave partials of a row added in wave order (as the K-split form), stored with
// device-coherent stores.  An accumulating stage adds them to the old y, which wave 0
// loads when the stage starts, lane i holding row i % R of the workgroup's chunk i / R
// (R rows per chunk) while i < 64; rows past the first 64 of a stage are loaded when they
// are written.
struct Pending {  // a computed chunk whose rows are not written yet (wave-uniform)
  uint32_t valid, k, parity, row0, n_out, rows, accum;
  gfloat *y;  // the segment's outputs (y + y_off)
};

SK_DEV Pending pending(const ConsumerView &v, uint32_t k, uint32_t g, uint32_t c) {
  uint32_t si, row0;
  locate(v, g, si, row0);
  return {1, k, c & 1, row0, pick(v.n_out, si), v.kind == CHAIN_Q4K_4096 ? 8u : 2u, v.accum,
          (gfloat *)v.y + pick(v.y_off, si)};
}

// lane i of wave 0 at a stage start: the old y of its row (zero if none or not accumulating)
SK_DEV float old_y(const ConsumerView &v, uint32_t wg, uint32_t nwg, uint32_t lane) {
  const uint32_t rows = v.kind == CHAIN_Q4K_4096 ? 8u : 2u;
  const uint32_t k = lane / rows, j = lane - k * rows;
  if (!v.accum || k >= v.nc) return 0.0f;
  uint32_t si, row0;
  locate(v, wg + k * nwg, si, row0);
  if (row0 + j >= pick(v.n_out, si)) return 0.0f;
  return __hip_atomic_load((gfloat *)v.y + pick(v.y_off, si) + row0 + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

SK_DEV void flush(const Pending &pd, const float (*part)[CONSUMERS][8], uint32_t lane, float old) {
  if (!pd.valid) return;
  const bool pre = (pd.k + 1) * pd.rows <= 64;  // the old values sit in lanes k R .. k R + R - 1
  const uint32_t j = pre ? lane - pd.k * pd.rows : lane;
  if (j >= pd.rows || pd.row0 + j >= pd.n_out) return;
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < CONSUMERS; i++) t += part[pd.parity][i][j];
  gfloat *yp = pd.y + pd.row0 + j;
  if (pd.accum) t = (pre ? old : __hip_atomic_load(yp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) + t;
  __hip_atomic_store(yp, t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Smem {
  unsigned char ring[RING * SLOT] __attribute__((aligned(16)));
  float4 hp[CONSUMERS][8][2][4];  // per wave: header products of (row, super-block, chunk)
  float part[2][CONSUMERS][8];     // wave partials of the last two chunks
};

// One Q4_K chunk: wave wv's two super-blocks of 8 rows.  xl/xh: the lane's 16 low- and 16
// high-nibble activations, sl/sh their sums (matvec_q4k_ks_body's operands).
SK_DEV void compute_q4k(Smem &sm, const unsigned char *sl, uint32_t par, uint32_t wv, uint32_t l,
                        const float4 (&xl)[4], const float4 (&xh)[4], float xsl, float xsh, uint32_t LO4,
                        uint32_t HI4) {
  const uint32_t ul = l & 15, pair = l >> 4;
  const uint32_t unit = wv * 16 + ul, sbl = ul >> 3, c = (unit >> 1) & 3;
  {  // this lane's quarter of one header: (row l / 8, super-block 2 wv + (l / 4) % 2)
    const uint32_t hr = l >> 3, hs = (l >> 2) & 1, cc = l & 3;
    const uint4 hc = *(const uint4 *)(sl + 16384 + hr * 256 + (2 * wv + hs) * 16);
    const float d = f16_bits_to_f32(hc.x & 0xffffu), dmin = f16_bits_to_f32(hc.x >> 16);
    const float d16 = d * 0.0625f;
    const uint32_t sw[2] = {hc.y & 0x3f3f3f3fu, (hc.w & 0x0f0f0f0fu) | ((hc.y >> 2) & 0x30303030u)};
    const uint32_t mw[2] = {hc.z & 0x3f3f3f3fu, ((hc.w >> 4) & 0x0f0f0f0fu) | ((hc.z >> 2) & 0x30303030u)};
    const uint32_t sv = (cc < 2 ? sw[0] : sw[1]) >> (16 * (cc & 1));
    const uint32_t mv = (cc < 2 ? mw[0] : mw[1]) >> (16 * (cc & 1));
    sm.hp[wv][hr][hs][cc] = make_float4(d * (float)(sv & 255u), d16 * (float)((sv >> 8) & 255u),
                                        dmin * (float)(mv & 255u), dmin * (float)((mv >> 8) & 255u));
  }
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const uint32_t row = pair * 2 + r;
    const uint4 q = *(const uint4 *)(sl + row * 2048 + unit * 16);
    const float sa = fma_bytes16(q, LO4, xl, 0.0f);
    const float sb = fma_bytes16(q, HI4, xh, 0.0f);
    const float4 f = sm.hp[wv][row][sbl][c];
    float v = f.x * sa;
    v = __builtin_fmaf(f.y, sb, v);
    v = __builtin_fmaf(-f.z, xsl, v);
    v = __builtin_fmaf(-f.w, xsh, v);
    v = lane_sum<16>(v);
    if (ul == 0) sm.part[par][wv][row] = v;
  }
}

// One Q6_K chunk: wave wv's six super-blocks of 2 rows; lane (row l / 32, unit l % 32 < 24).
// xq[g][k]: the unit's activations 32 g + 4 k .. + 3 within its 128-value half; ib[g] = -32
// times the sum of group g's 16 values.
SK_DEV void compute_q6k(Smem &sm, const unsigned char *sl, uint32_t par, uint32_t wv, uint32_t l,
                        const float4 (&xq)[4][4], const float (&ib)[4], uint32_t LO4, uint32_t H2) {
  const uint32_t j = l & 31, r = l >> 5;
  float acc = 0.0f;
  if (j < 24) {
    const uint32_t s = wv * 6 + (j >> 2), hf = (j >> 1) & 1, li = j & 1;
    const uint4 qa = *(const uint4 *)(sl + r * 6144 + s * 128 + hf * 64 + li * 16);
    const uint4 qb = *(const uint4 *)(sl + r * 6144 + s * 128 + hf * 64 + 32 + li * 16);
    const uint4 qh = *(const uint4 *)(sl + 12288 + r * 3072 + s * 64 + hf * 32 + li * 16);
    const uint4 scw = *(const uint4 *)(sl + 18432 + r * 768 + s * 16);
    const float d = f16_bits_to_f32(*(const uint16_t *)(sl + 19968 + r * 96 + s * 2));
    const uint32_t sw[4] = {scw.x, scw.y, scw.z, scw.w};
    const uint32_t hv[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint4 qv = (g & 1) ? qb : qa;
      const uint32_t wv4[4] = {qv.x, qv.y, qv.z, qv.w};
      float tg = ib[g];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const uint32_t lo = g < 2 ? wv4[k] : wv4[k] >> 4;
        const uint32_t hb = g == 0 ? hv[k] << 4 : g == 1 ? hv[k] << 2 : g == 2 ? hv[k] : hv[k] >> 2;
        tg = fma_bytes((lo & LO4) | (hb & H2), xq[g][k], tg);
      }
      // scale 8 hf + li + 2 g: word 2 hf + g / 2, byte li + 2 (g % 2) (selected, not indexed)
      const uint32_t sword = hf ? (g < 2 ? sw[2] : sw[3]) : (g < 2 ? sw[0] : sw[1]);
      const int s8 = (int)(int8_t)((sword >> (8 * (li + 2 * (g & 1)))) & 255u);
      acc = __builtin_fmaf(d * (float)s8, tg, acc);
      __builtin_amdgcn_sched_barrier(0);  // one group's operands live at a time
    }
  }
  const float v = lane_sum<32>(acc);
  if (j == 0) sm.part[par][wv][r] = v;
}

template <int L>
SK_DEV void loader(CStage *tab, uint32_t n_stages, uint32_t wg, uint32_t nwg, Smem &sm, uint32_t lane) {
  // issue cursor: stage ls (its view lv), its chunk lk; `issued` chunks so far (slot =
  // index % RING)
  uint32_t ls = 0, lk = 0, issued = 0;
  LoaderView lv = loader_view(tab, wg, nwg);
  auto skip = [&]() {
    while (ls < n_stages && lk >= lv.nc) {
      ls++;
      lk = 0;
      if (ls < n_stages) lv = loader_view(tab + ls, wg, nwg);
    }
  };
  auto next = [&]() {
    if (ls >= n_stages) return;
    issue<L>(lv, wg + lk * nwg, sm.ring + (issued % RING) * SLOT, lane);
    issued++;
    lk++;
    skip();
  };
  if (n_stages) skip();
  for (int i = 0; i < AHEAD; i++) next();
  uint32_t c = 0;
  for (uint32_t s = 0; s < n_stages; s++) {
    const uint32_t nc = chunks_of(tab[s].n_chunks, wg, nwg);
    for (uint32_t k = 0; k < nc; k++, c++) {
      wait_chunks(issued - c - 1);
      bar();
      next();
    }
    bar();
  }
}

SK_DEV void consumer(CStage *tab, uint32_t n_stages, uint32_t wg, uint32_t nwg, Smem &sm, uint32_t *sync,
                     uint32_t wv, uint32_t l) {
  const uint32_t LO4 = opaque_mask(0x0f0f0f0fu), HI4 = opaque_mask(0xf0f0f0f0u), H2 = opaque_mask(0x30303030u);
  Pending pd = {0, 0, 0, 0, 0, 0, 0, nullptr};
  float old = 0.0f;  // wave 0: the old y values of the pending chunk's stage (old_y)
  uint32_t c = 0;    // chunks so far: ring slot c % RING, partials parity c % 2
  ConsumerView v = consumer_view(tab, wg, nwg);
  for (uint32_t s = 0; s < n_stages; s++) {
    const uint32_t nc = v.nc;
    const bool q4 = v.kind == CHAIN_Q4K_4096;
    const BufRes xr = buf_res((const float *)v.x + v.x_off, 4ull * (q4 ? 4096u : 12288u));
    // Chunk k: the barrier that hands its slot over, the previous chunk's outputs, the
    // computation.  The stage's activations (and old outputs) are read once, after the
    // first chunk's barrier, so after the grid barrier wave 0 waited at.
    if (nc && q4) {
      bar();
      if (wv == 0) {
        flush(pd, sm.part, l, old);
        old = old_y(v, wg, nwg, l);
        asm volatile("" ::"v"(old));  // wait for it here, with the activations, not per chunk
      }
      const uint32_t unit = wv * 16 + (l & 15);
      const uint32_t at = (unit >> 3) * 256 + ((unit >> 1) & 3) * 64 + (unit & 1) * 16;
      float4 xl[4], xh[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        xl[i] = ld_coherent(xr, 4 * (at + 4 * i));
        xh[i] = ld_coherent(xr, 4 * (at + 32 + 4 * i));
      }
      const float xsl = (sum4(xl[0]) + sum4(xl[1])) + (sum4(xl[2]) + sum4(xl[3]));
      const float xsh = (sum4(xh[0]) + sum4(xh[1])) + (sum4(xh[2]) + sum4(xh[3]));
      for (uint32_t k = 0; k < nc; k++, c++) {
        if (k) {
          bar();
          if (wv == 0) flush(pd, sm.part, l, old);
        }
        compute_q4k(sm, sm.ring + (c % RING) * SLOT, c & 1, wv, l, xl, xh, xsl, xsh, LO4, HI4);
        pd = pending(v, k, wg + k * nwg, c);
      }
    } else if (nc) {
      bar();
      if (wv == 0) {
        flush(pd, sm.part, l, old);
        old = old_y(v, wg, nwg, l);
        asm volatile("" ::"v"(old));
      }
      const uint32_t j = l & 31;
      const uint32_t at = (wv * 6 + (j >> 2)) * 256 + ((j >> 1) & 1) * 128 + (j & 1) * 16;
      float4 xq[4][4];
      float ib[4];
#pragma unroll
      for (int g = 0; g < 4; g++) {
#pragma unroll
        for (int i = 0; i < 4; i++) xq[g][i] = ld_coherent(xr, 4 * (at + 32 * g + 4 * i));
        ib[g] = -32.0f * ((sum4(xq[g][0]) + sum4(xq[g][1])) + (sum4(xq[g][2]) + sum4(xq[g][3])));
      }
      for (uint32_t k = 0; k < nc; k++, c++) {
        if (k) {
          bar();
          if (wv == 0) flush(pd, sm.part, l, old);
        }
        compute_q6k(sm, sm.ring + (c % RING) * SLOT, c & 1, wv, l, xq, ib, LO4, H2);
        pd = pending(v, k, wg + k * nwg, c);
      }
    }
    // the next stage's view, read while this one finishes
    if (s + 1 < n_stages) v = consumer_view(tab + s + 1, wg, nwg);
    bar();  // the stage's last partials are in LDS
    if (wv == 0) {
      flush(pd, sm.part, l, old);
      pd.valid = 0;
      if (l == 0) {
        const uint32_t target = (s + 1) * nwg;
        // this wave's device-coherent stores are complete before the count (an agent-scope
        // release would also write back the XCD's L2, which costs ~1.5 us a stage here and
        // is not needed: every value another workgroup reads was stored device-coherent)
        __builtin_amdgcn_s_waitcnt(0);
        const uint32_t prev = __hip_atomic_fetch_add(&sync[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (s + 1 < n_stages) {
          // every 256 polls: give up past the limit, or at once after a time-out elsewhere
          uint32_t n = 0;
          while (__hip_atomic_load(&sync[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if ((++n & 255u) == 0 &&
                (n > SPIN_LIMIT || __hip_atomic_load(&sync[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
              __hip_atomic_store(&sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
        } else if (prev == target - 1) {
          __hip_atomic_store(&sync[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
}

}  // namespace

// table: device address of n_stages ChainStage entries; sync: CHAIN_SYNC_WORDS words, zero
// at the first launch (every launch leaves sync[0] zero).
extern "C" __global__ __launch_bounds__(CHAIN_THREADS) void matvec_chain(uint64_t table, uint32_t n_stages,
                                                                          uint32_t *sync) {
  __shared__ Smem sm;
  CStage *tab = (CStage *)table;
  const uint32_t wv = threadIdx.x >> 6, l = threadIdx.x & 63;
  if (wv == CONSUMERS)
    loader<0>(tab, n_stages, blockIdx.x, gridDim.x, sm, l);
  else if (wv == CONSUMERS + 1)
    loader<1>(tab, n_stages, blockIdx.x, gridDim.x, sm, l);
  else
    consumer(tab, n_stages, blockIdx.x, gridDim.x, sm, sync, wv, l);
}
