// Timeline probe of the K-split Q4_K decode matvec (n_in 4096) over the config-2 launches of
// 36 Qwen3-8B layers (q+k+v, o with ACCUM, gate+up; one HIP graph, dependent launches).
//
// A diagnostic build, not part of the library: the body of matvec_q4k_ks_body (matvec.hip)
// with per-wave wall-clock stamps (entry, activations and their sums, header decoded, first
// row, all rows, the workgroup barrier, the store), and variants of it that keep the same
// loads and grid:
//   V 0  the library's arithmetic (f32 FMAs on v_cvt_f32_ubyte quants)
//   V 2  the same products as v_fma_mix_f32 of f16 subnormal nibble pairs (fewer VALU)
//   V 9  the same loads, no arithmetic (XOR of the loaded words): the floor of the loads
//   V 8  V 9 without the activation loads
//   V 7  V 8 with each workgroup's rows read as one contiguous range
// Weights are random bytes with valid f16 d / dmin; every stamp index is checked on the host
// against the stamp buffer before any launch.
//
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       -o matvec_timeline skyla-kernel_amd/tools/matvec_timeline.hip
//   ./matvec_timeline V R_qkv R_o R_gateup NG_gateup STAMPS      (e.g. 0 4 4 4 1 1)
#include "../csrc/kernels/common.h"
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>
#include <string>
#include <cmath>

#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); exit(1);} } while (0)

struct MatvecPush2 { uint32_t o0, o1, x_off, y_off, n_in, n_out, ids_off, x_stride, y_stride; };
constexpr int NST = 8;
struct TL { unsigned long long *buf; uint32_t launch; uint32_t wg_base; };

#define STAMP(i) do { if (l == 0 && tl.buf) { tl.buf[((size_t)(tl.wg_base + bx_glob) * 8 + wv) * NST + (i)] = wall_clock64(); } } while (0)

template <int V>
SK_DEV float prod16(uint4 q, uint32_t mask, const float4 (&x)[4], float s) {
  if constexpr (V < 2) {
    return fma_bytes16(q, mask, x, s);
  } else {
    // f16 subnormal pairs: (b0, b2) and (b1, b3) of each word
    const uint32_t m = mask & 0x00ff00ffu;   // 0x000f000f or 0x00f000f0
    uint32_t ws[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint32_t a = ws[k] & m, c = (ws[k] >> 8) & m;
      const f16x2 ha = as_f16x2(a), hc = as_f16x2(c);
      const float *xv = (const float *)&x[k];
      s = __builtin_fmaf((float)ha[0], xv[0], s);
      s = __builtin_fmaf((float)hc[0], xv[1], s);
      s = __builtin_fmaf((float)ha[1], xv[2], s);
      s = __builtin_fmaf((float)hc[1], xv[3], s);
    }
    return s;
  }
}

template <int ACCUM, int RPL, int NG, int V>
__device__ void body(const uint4 *__restrict__ w, const float *x, float *y, const MatvecPush2 &p, uint32_t bx,
                     TL tl, uint32_t bx_glob) {
  constexpr int RG = 4 * RPL, OG = RG, OUT = OG * NG, CPL = RG / 8;
  __shared__ float4 hp[8][RG][2][4];
  __shared__ float part[8][RG * NG];
  const uint32_t tid = threadIdx.x, wv = tid >> 6, l = tid & 63;
  STAMP(0);
  const uint32_t ul = l & 15, slot = l >> 4;
  const uint32_t unit = wv * 16 + ul, sbl = ul >> 3, c = (unit >> 1) & 3;
  const uint32_t LO4 = opaque_mask(V >= 2 ? 0x000f000fu : 0x0f0f0f0fu), HI4 = opaque_mask(V >= 2 ? 0x00f000f0u : 0xf0f0f0f0u);
  const uint32_t out0 = bx * OUT;
  auto row_of = [&](uint32_t g, uint32_t s, uint32_t r) -> uint32_t {
    return min(out0 + g * OG + s * RPL + r, p.n_out - 1);
  };
  const uint32_t hh = (l * CPL) >> 2, hc0 = (l * CPL) & 3, h_rl = hh >> 1, h_sb = hh & 1;
  const uint32_t qo = p.o0, hho = p.o1;
  auto load_group = [&](uint32_t g, uint4 (&q)[RPL], uint4 &h) {
    h = w[hho + (size_t)row_of(g, h_rl / RPL, h_rl % RPL) * 16 + 2 * wv + h_sb];
#pragma unroll
    for (int r = 0; r < RPL; r++) q[r] = w[qo + (size_t)row_of(g, slot, r) * 128 + unit];
  };
  const uint32_t at = (unit >> 3) * 256 + c * 64 + (unit & 1) * 16;
  const float *xv = x + p.x_off;
  float4 xl[4], xh[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    if constexpr (V == 7 || V == 8) {
      xl[k] = make_float4(0.f, 0.f, 0.f, 0.f); xh[k] = xl[k];
    } else {
      xl[k] = *(const float4 *)(xv + at + 4 * k);
      xh[k] = *(const float4 *)(xv + at + 32 + 4 * k);
    }
  }
  if constexpr (V >= 1) __builtin_amdgcn_sched_barrier(0);
  uint4 qc[RPL], hc;
  if constexpr (V == 7) {  // the workgroup's rows as one contiguous range: instruction r covers 8 KB
    static_assert(RPL == 4, "V7 is written for 16 rows per workgroup");
    hc = make_uint4(0, 0, 0, 0);
    if (tid < 256) hc = w[hho + (size_t)out0 * 16 + tid];
#pragma unroll
    for (int r = 0; r < RPL; r++) qc[r] = w[qo + (size_t)out0 * 128 + r * 512 + tid];
  } else {
    load_group(0, qc, hc);
  }
  float yold = 0.0f;
  if constexpr (ACCUM)
    if (tid < (uint32_t)OUT && out0 + tid < p.n_out) yold = y[p.y_off + out0 + tid];
  if constexpr (V >= 1) __builtin_amdgcn_sched_barrier(0);
  const float sl = (sum4(xl[0]) + sum4(xl[1])) + (sum4(xl[2]) + sum4(xl[3]));
  const float sh = (sum4(xh[0]) + sum4(xh[1])) + (sum4(xh[2]) + sum4(xh[3]));
  if (V >= 1) { asm volatile("" :: "v"(sl), "v"(sh)); }
  STAMP(1);
  if constexpr (V >= 7) {
    uint32_t acc = __float_as_uint(sl) ^ __float_as_uint(sh) ^ __float_as_uint(yold);
#pragma unroll
    for (int g = 0; g < NG; g++) {
      uint4 qn[RPL], hn;
      if (g + 1 < NG) load_group(g + 1, qn, hn);
      acc ^= hc.x ^ hc.y ^ hc.z ^ hc.w;
#pragma unroll
      for (int r = 0; r < RPL; r++) acc ^= qc[r].x ^ qc[r].y ^ qc[r].z ^ qc[r].w;
      if (g + 1 < NG) {
#pragma unroll
        for (int r = 0; r < RPL; r++) qc[r] = qn[r];
        hc = hn;
      }
    }
    STAMP(4);
    if (ul == 0) part[wv][slot] = __uint_as_float(acc);
    __syncthreads();
    STAMP(5);
    if (tid < (uint32_t)OUT && out0 + tid < p.n_out) {
      uint32_t t = 0;
      for (int i = 0; i < 8; i++) t ^= __float_as_uint(part[i][tid % 4]);
      y[p.y_off + out0 + tid] = __uint_as_float(t);
    }
    STAMP(6);
    return;
  }
#pragma unroll
  for (int g = 0; g < NG; g++) {
    uint4 qn[RPL], hn;
    if (g + 1 < NG) load_group(g + 1, qn, hn);
    {
      const float d = f16_bits_to_f32(hc.x & 0xffffu), dmin = f16_bits_to_f32(hc.x >> 16);
      const float d16 = d * ((V >= 2) ? 16777216.0f / 16.0f * 0.0625f * 16.0f : 0.0625f);
      const float dl = (V >= 2) ? d * 16777216.0f : d;
      const uint32_t sw[2] = {hc.y & 0x3f3f3f3fu, (hc.w & 0x0f0f0f0fu) | ((hc.y >> 2) & 0x30303030u)};
      const uint32_t mw[2] = {hc.z & 0x3f3f3f3fu, ((hc.w >> 4) & 0x0f0f0f0fu) | ((hc.z >> 2) & 0x30303030u)};
#pragma unroll
      for (int i = 0; i < CPL; i++) {
        const uint32_t cc = hc0 + i;
        const uint32_t sv = (cc < 2 ? sw[0] : sw[1]) >> (16 * (cc & 1));
        const uint32_t mv = (cc < 2 ? mw[0] : mw[1]) >> (16 * (cc & 1));
        hp[wv][h_rl][h_sb][cc] = make_float4(dl * (float)(sv & 255u), d16 * (float)((sv >> 8) & 255u),
                                             dmin * (float)(mv & 255u), dmin * (float)((mv >> 8) & 255u));
      }
    }
    if (g == 0) STAMP(2);
#pragma unroll
    for (int r = 0; r < RPL; r++) {
      const float sa = prod16<V>(qc[r], LO4, xl, 0.0f);
      const float sb = prod16<V>(qc[r], HI4, xh, 0.0f);
      const float4 f = hp[wv][slot * RPL + r][sbl][c];
      float v = f.x * sa;
      v = __builtin_fmaf(f.y, sb, v);
      v = __builtin_fmaf(-f.z, sl, v);
      v = __builtin_fmaf(-f.w, sh, v);
      v = lane_sum<16>(v);
      if (ul == 0) part[wv][g * RG + slot * RPL + r] = v;
      if (g == 0 && r == 0) STAMP(3);
    }
    if (g + 1 < NG) {
#pragma unroll
      for (int r = 0; r < RPL; r++) qc[r] = qn[r];
      hc = hn;
    }
  }
  STAMP(4);
  __syncthreads();
  STAMP(5);
  if (tid < (uint32_t)OUT && out0 + tid < p.n_out) {
    const uint32_t g = tid / OG, o = tid % OG;
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) t += part[i][g * RG + o];
    const uint32_t yo = p.y_off + out0 + tid;
    if (ACCUM) y[yo] = yold + t; else y[yo] = t;
  }
  STAMP(6);
}

template <int ACCUM, int RPL, int NG, int V>
__global__ __launch_bounds__(512) void ks(const uint4 *w, const float *x, float *y, Segments<MatvecPush2> m, TL tl) {
  const uint32_t s = segment_of(m, blockIdx.x);
  body<ACCUM, RPL, NG, V>(w, x, y, segment_push(m, s), blockIdx.x - m.start[s], tl, blockIdx.x);
}

__global__ void fill(uint32_t *p, size_t n, uint32_t seed) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint32_t h = (uint32_t)i * 2654435761u ^ seed; h ^= h >> 15; h *= 2246822519u; h ^= h >> 13;
    p[i] = h;
  }
}
__global__ void fixhdr(uint4 *w, size_t first, size_t n) {  // d, dmin = 2^-8 (valid f16)
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) w[first + i].x = 0x1c001c00u;
}
__global__ void fillx(float *x, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    x[i] = ((int)((i * 2654435761u) >> 16 & 1023) - 512) / 256.0f;
}

struct Mat { uint32_t o0, o1, n_out; };


typedef void (*KFn)(const uint4 *, const float *, float *, Segments<MatvecPush2>, TL);
#include <map>
#include <tuple>
static std::map<std::tuple<int, int, int, int>, KFn> g_k;
#define REG1(A, R, G, VV) g_k[std::make_tuple(A, R, G, VV)] = ks<A, R, G, VV>;
#define REGV(A, R, G) REG1(A, R, G, 0) REG1(A, R, G, 2) REG1(A, R, G, 9) REG1(A, R, G, 8)
#define REGG(A, R) REGV(A, R, 1) REGV(A, R, 2)
static void reg() { REGG(0, 2) REGG(1, 2) REGG(0, 4) REGG(1, 4) REGG(0, 8) REGG(1, 8) REG1(0, 4, 1, 7) REG1(1, 4, 1, 7) }

int main(int argc, char **argv) {
  reg();
  const int V = argc > 1 ? atoi(argv[1]) : 0;
  int R[3] = {argc > 2 ? atoi(argv[2]) : 4, argc > 3 ? atoi(argv[3]) : 4, argc > 4 ? atoi(argv[4]) : 4};
  int G[3] = {1, 1, argc > 5 ? atoi(argv[5]) : 1};
  const int stamps = argc > 6 ? atoi(argv[6]) : 1;
  for (int k = 0; k < 3; k++)
    if (!g_k.count(std::make_tuple(0, R[k], G[k], V))) { fprintf(stderr, "no kernel for V=%d R=%d G=%d\n", V, R[k], G[k]); return 2; }
  const int NL = 36;
  const uint32_t N = 4096;
  const uint32_t rows[6] = {4096, 1024, 1024, 4096, 12288, 12288};
  std::vector<std::vector<Mat>> L(NL);
  size_t off = 0;
  for (int l = 0; l < NL; l++)
    for (int m = 0; m < 6; m++) {
      Mat mt; mt.n_out = rows[m];
      mt.o0 = (uint32_t)off; off += (size_t)rows[m] * 128;
      mt.o1 = (uint32_t)off; off += (size_t)rows[m] * 16;
      L[l].push_back(mt);
    }
  if (off >= (1ull << 32)) { fprintf(stderr, "offsets past 32 bits\n"); return 2; }
  uint4 *w; float *a; unsigned long long *tb = nullptr;
  CK(hipMalloc(&w, off * 16));
  hipLaunchKernelGGL(fill, dim3(4096), dim3(256), 0, 0, (uint32_t *)w, off * 4, 12345u);
  for (int l = 0; l < NL; l++) for (int m = 0; m < 6; m++)
    hipLaunchKernelGGL(fixhdr, dim3(256), dim3(256), 0, 0, w, (size_t)L[l][m].o1, (size_t)rows[m] * 16);
  const uint32_t o_n = 64, o_attn = o_n + 4096, o_x = o_attn + 4096, o_q = o_x + 4096, o_k = o_q + 4096, o_v = o_k + 1024,
                 o_g = o_v + 1024, o_u = o_g + 12288, o_end = o_u + 12288;
  CK(hipMalloc(&a, o_end * 4));
  hipLaunchKernelGGL(fillx, dim3(64), dim3(256), 0, 0, a, (size_t)o_end);
  auto push = [&](const Mat &m, uint32_t xo, uint32_t yo) { MatvecPush2 p{m.o0, m.o1, xo, yo, N, m.n_out, 0, 0, 0}; return p; };
  struct Launch { int kind, accum; Segments<MatvecPush2> sg; uint32_t grid; };
  std::vector<Launch> ls;
  for (int l = 0; l < NL; l++) {
    auto mk = [&](int kind, std::vector<MatvecPush2> ps, int accum) {
      const uint32_t per = 4 * R[kind] * G[kind];
      Launch la; la.kind = kind; la.accum = accum; la.sg.n = ps.size();
      uint32_t b = 0;
      for (int i = 0; i < 4; i++) la.sg.start[i] = 0xffffffffu;
      for (size_t i = 0; i < ps.size(); i++) { la.sg.start[i] = b; la.sg.p[i] = ps[i]; b += (ps[i].n_out + per - 1) / per; }
      la.sg.start[0] = 0;
      for (size_t i = ps.size(); i < 4; i++) la.sg.p[i] = ps[0];
      la.grid = b; ls.push_back(la);
    };
    mk(0, {push(L[l][0], o_n, o_q), push(L[l][1], o_n, o_k), push(L[l][2], o_n, o_v)}, 0);
    mk(1, {push(L[l][3], o_attn, o_x)}, 1);
    mk(2, {push(L[l][4], o_n, o_g), push(L[l][5], o_n, o_u)}, 0);
  }
  size_t n_wg_max = 0;
  for (auto &la : ls) n_wg_max = std::max(n_wg_max, (size_t)la.grid);
  const size_t tl_n = ls.size() * n_wg_max * 8 * NST;
  if (stamps) { CK(hipMalloc(&tb, tl_n * 8)); CK(hipMemset(tb, 0, tl_n * 8)); }
  for (size_t i = 0; i < ls.size(); i++) {
    const size_t last = ((i * n_wg_max + ls[i].grid - 1) * 8 + 7) * NST + NST - 1;
    if (ls[i].grid > n_wg_max || last >= tl_n) { fprintf(stderr, "launch %zu stamps past the buffer\n", i); return 3; }
  }
  CK(hipDeviceSynchronize());
  hipStream_t st; CK(hipStreamCreate(&st));
  int wcr = 0; CK(hipDeviceGetAttribute(&wcr, hipDeviceAttributeWallClockRate, 0));
  const double ns_per_tick = 1e6 / wcr;
  auto launch = [&](size_t i, hipStream_t s) {
    const Launch &la = ls[i];
    TL t{tb, (uint32_t)i, (uint32_t)(i * n_wg_max)};
    KFn f = g_k.at(std::make_tuple(la.accum, R[la.kind], G[la.kind], V));
    hipLaunchKernelGGL(f, dim3(la.grid), dim3(512), 0, s, w, a, a, la.sg, t);
  };
  hipGraph_t g; hipGraphExec_t ge;
  CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
  for (size_t i = 0; i < ls.size(); i++) launch(i, st);
  CK(hipStreamEndCapture(st, &g));
  CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
  for (int i = 0; i < 5; i++) CK(hipGraphLaunch(ge, st));
  CK(hipStreamSynchronize(st));
  std::vector<float> ts;
  for (int i = 0; i < 15; i++) {
    CK(hipEventRecord(e0, st)); CK(hipGraphLaunch(ge, st)); CK(hipEventRecord(e1, st)); CK(hipEventSynchronize(e1));
    float ms; CK(hipEventElapsedTime(&ms, e0, e1)); ts.push_back(ms);
  }
  std::sort(ts.begin(), ts.end());
  double bytes = 0;
  for (int m = 0; m < 6; m++) bytes += rows[m] * (double)(N / 256 * 144) + 4.0 * N + 4.0 * rows[m] + (m == 3 ? 4.0 * rows[m] : 0);
  bytes *= NL;
  printf("V=%d R=%d,%d,%d G=%d,%d,%d stamps=%d: graph %.4f ms (median of 15) %zu launches: %.3f us/launch, %.0f GB/s\n",
         V, R[0], R[1], R[2], G[0], G[1], G[2], stamps, ts[7], ls.size(), ts[7] * 1e3 / ls.size(), bytes / (ts[7] * 1e-3) / 1e9);
  // per-kind launch times: graphs of one kind only (36 launches with barriers)
  for (int k = 0; k < 3; k++) {
    hipGraph_t g2; hipGraphExec_t ge2;
    CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    for (size_t i = 0; i < ls.size(); i++) if (ls[i].kind == k) launch(i, st);
    CK(hipStreamEndCapture(st, &g2));
    CK(hipGraphInstantiate(&ge2, g2, nullptr, nullptr, 0));
    for (int i = 0; i < 3; i++) CK(hipGraphLaunch(ge2, st));
    std::vector<float> t2;
    for (int i = 0; i < 9; i++) {
      CK(hipEventRecord(e0, st)); CK(hipGraphLaunch(ge2, st)); CK(hipEventRecord(e1, st)); CK(hipEventSynchronize(e1));
      float ms; CK(hipEventElapsedTime(&ms, e0, e1)); t2.push_back(ms);
    }
    std::sort(t2.begin(), t2.end());
    const char *kn[3] = {"qkv", "o", "gate+up"};
    printf("  %-8s alone: %.3f us per launch\n", kn[k], t2[4] * 1e3 / NL);
    CK(hipGraphExecDestroy(ge2)); CK(hipGraphDestroy(g2));
  }
  if (!stamps) return 0;
  CK(hipGraphLaunch(ge, st));
  CK(hipStreamSynchronize(st));
  std::vector<unsigned long long> h(tl_n);
  CK(hipMemcpy(h.data(), tb, tl_n * 8, hipMemcpyDeviceToHost));
  const char *kind[3] = {"qkv", "o", "gate+up"};
  for (int k = 0; k < 3; k++) {
    double acc_span = 0, acc_p[NST][3] = {{0}};
    double acc_gap = 0; int ngap = 0;
    for (int l = 0; l < NL; l++) {
      size_t i = l * 3 + k;
      const Launch &la = ls[i];
      unsigned long long t0 = ~0ull, tend = 0;
      std::vector<std::vector<double>> ph(NST);
      for (uint32_t b = 0; b < la.grid; b++) for (int wv = 0; wv < 8; wv++) {
        const unsigned long long *s = &h[((i * n_wg_max + b) * 8 + wv) * NST];
        t0 = std::min(t0, s[0]); tend = std::max(tend, s[6]);
      }
      for (uint32_t b = 0; b < la.grid; b++) for (int wv = 0; wv < 8; wv++) {
        const unsigned long long *s = &h[((i * n_wg_max + b) * 8 + wv) * NST];
        for (int j = 0; j < 7; j++) if (s[j]) ph[j].push_back((double)(s[j] - t0) * ns_per_tick);
      }
      for (int j = 0; j < 7; j++) {
        if (ph[j].empty()) continue;
        std::sort(ph[j].begin(), ph[j].end());
        acc_p[j][0] += ph[j][ph[j].size() / 10]; acc_p[j][1] += ph[j][ph[j].size() / 2]; acc_p[j][2] += ph[j].back();
      }
      acc_span += (tend - t0) * ns_per_tick;
      if (i + 1 < ls.size()) {
        const Launch &ln = ls[i + 1];
        unsigned long long n0 = ~0ull;
        for (uint32_t b = 0; b < ln.grid; b++) for (int wv = 0; wv < 8; wv++) n0 = std::min(n0, h[(((i + 1) * n_wg_max + b) * 8 + wv) * NST]);
        acc_gap += ((double)n0 - (double)tend) * ns_per_tick; ngap++;
      }
    }
    printf("%-8s span %.0f ns, gap to next launch %.0f ns\n", kind[k], acc_span / NL, acc_gap / ngap);
    const char *pn[7] = {"entry", "x+sums", "hdr", "row0", "rows", "barrier", "store"};
    for (int j = 0; j < 7; j++) printf("   %-8s p10 %6.0f  p50 %6.0f  max %6.0f ns\n", pn[j], acc_p[j][0] / NL, acc_p[j][1] / NL, acc_p[j][2] / NL);
  }
  return 0;
}
