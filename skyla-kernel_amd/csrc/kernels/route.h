// moe_route's selection (moe_route.comp:23-75), shared by moe.hip (moe_route) and
// matvec.hip (the experts' gate/up form that routes for itself).
#pragma once

#include "common.h"

struct RoutePush { uint32_t logits_off, ids_off, weights_off, n_expert, n_used; };

// Monotone u32 key of a float with -0 folded onto +0 (so equal values tie exactly as the
// float comparisons of moe_route.comp:36-52 do).
SK_DEV uint32_t order_key(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v + 0.0f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

SK_DEV float key_value(uint32_t k) {
  const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __builtin_bit_cast(float, b);
}

template <int CTRL>
SK_DEV uint32_t dpp_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// moe_route (moe_route.comp:23-75): per token, n_used rounds of "largest logit, lowest
// index on ties", then weights exp(v_k - v_0) / sum.  One wave per token: expert
// e = lane + 64 j is held in key[j] (n_expert <= 256), a round is a lane maximum, a wave
// maximum (DPP within rows of 16, then two shuffles) and a ballot for the lowest expert
// holding it.  Lane k keeps round k's choice; the exponentials are computed in parallel
// and summed in round order, as the reference does.
// The routing weight of lane t's choice `chosen` (lane k holds round k's logit): exp(v_k - v_0)
// over the sum of the n_used exponentials, added in round order (moe_route.comp:66-73).
SK_DEV float route_weight(float chosen, uint32_t n_used) {
  const float largest = __shfl(chosen, 0, 64);
  const float e = expf(chosen - largest);
  float total = 0.0f;
  for (uint32_t k = 0; k < n_used; k++) total += __shfl(e, (int)k, 64);
  return e / total;
}

// This is the selection for token `tok` on one wave (lane t), writing ids[ids_off + ..] and
// aw[weights_off + ..].
SK_DEV void route_token(const float *a, float *aw, uint32_t *ids, const RoutePush &p, uint32_t tok,
                        uint32_t t) {
  const uint32_t n_used = min(p.n_used, 16u);
  const uint32_t n_expert = min(p.n_expert, 256u);
  const uint32_t logits_off = p.logits_off + tok * p.n_expert;
  // 0 marks "taken or absent"; a real key is >= 1 (only one NaN pattern maps to 0)
  uint32_t key[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t e = t + 64 * j;
    float v = 0.0f;
    if (e < n_expert)
      v = a[logits_off + e];
    key[j] = e < n_expert ? max(order_key(v), 1u) : 0u;
  }
  float chosen = 0.0f;
  uint32_t chosen_idx = 0;
  for (uint32_t k = 0; k < n_used; k++) {
    uint32_t m = max(max(key[0], key[1]), max(key[2], key[3]));
    m = max(m, dpp_u<0xb1>(m));   // quad_perm [1,0,3,2]
    m = max(m, dpp_u<0x4e>(m));   // quad_perm [2,3,0,1]
    m = max(m, dpp_u<0x141>(m));  // row_half_mirror
    m = max(m, dpp_u<0x140>(m));  // row_mirror
    m = max(m, (uint32_t)__shfl_xor((int)m, 16, 64));
    m = max(m, (uint32_t)__shfl_xor((int)m, 32, 64));
    // lowest expert index holding m: the smallest j with a holder, then the lowest lane
    uint32_t idx = 0;
    bool found = false;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint64_t holders = __ballot(key[j] == m);
      if (!found && holders != 0) {
        idx = (uint32_t)__builtin_ctzll(holders) + 64 * j;
        found = true;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (idx == t + 64 * j) key[j] = 0;
    if (t == k) {
      chosen = key_value(m);
      chosen_idx = idx;
    }
  }
  const float wt = route_weight(chosen, n_used);
  if (t < n_used) {
    ids[p.ids_off + tok * p.n_used + t] = chosen_idx;
    aw[p.weights_off + tok * p.n_used + t] = wt;
  }
}

// The same selection by a workgroup of 256 threads, for a kernel whose every workgroup
// routes for itself before it can load anything.  Expert e's place is the number of experts
// before it in the order "larger key first, lower index on ties" (all (key, index) pairs are
// distinct, so the places are 0, 1, ..), and the expert in place k is round k's choice in
// route_token.  Each (key, ~index) pair is one 64-bit word in LDS; thread t counts the words
// above expert t % 128's over half of the experts (n_expert <= 128) or expert t's over all of
// them, with no serial rounds.  Leaves sid[k] = the expert in place k and sval[k] = its logit
// (as route_token's rounds read it back from the key) for k < n_used, behind a barrier.
// Needs n_used <= n_expert (the runtime's configuration check).
SK_DEV void route_ranked(const float *a, const RoutePush &p, uint32_t tok, uint32_t t, uint32_t *sid,
                         float *sval) {
  __shared__ uint64_t kk[256];
  __shared__ uint32_t half[256];
  const uint32_t n_used = min(p.n_used, 16u);
  const uint32_t n_expert = min(p.n_expert, 256u);
  uint32_t key = 0;
  if (t < n_expert) key = max(order_key(a[p.logits_off + tok * p.n_expert + t]), 1u);
  kk[t] = ((uint64_t)key << 32) | (uint32_t)~t;
  __syncthreads();
  const bool halves = n_expert <= 128;  // wave-uniform: waves 0, 1 take the first half
  const uint32_t e = halves ? (t & 127) : t;
  const uint32_t len = halves ? (n_expert + 1) / 2 : n_expert;
  const uint32_t f0 = halves ? (t >> 7) * len : 0, f1 = min(f0 + len, n_expert);
  const uint64_t mine = kk[e];
  uint32_t before = 0;
#pragma unroll 8
  for (uint32_t f = f0; f < f1; f++) before += kk[f] > mine ? 1u : 0u;
  half[t] = before;
  __syncthreads();
  if (t < n_expert) {  // with halves, t < 128: thread t + 128 counted the second half
    const uint32_t place = before + (halves ? half[t + 128] : 0u);
    if (place < n_used) {
      sid[place] = t;
      sval[place] = key_value(key);
    }
  }
  __syncthreads();
}
