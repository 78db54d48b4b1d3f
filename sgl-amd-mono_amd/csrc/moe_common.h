// Routing shared by the MoE launches: sigmoid + bias top-k with lowest-id ties, the
// slot tables (slot 0 the shared expert) and the distinct-expert list every CTA
// derives identically from them.
#pragma once

#include "mono_device.h"

namespace mono {

constexpr int MOE_MAXR = 16;   // rows a MoE launch takes
constexpr int MOE_NEXP = 256;  // routed experts
constexpr int MOE_TOPK = 8;
constexpr int MOE_SLOTS = MOE_TOPK + 1;
constexpr int MOE_SHARED = 256;  // the shared expert's id
constexpr int MOE_NDIST = MOE_NEXP + 1;
constexpr int MOE_MAXGROUP = 16;  // expert groups of group-limited routing

// a launch's group-limited routing arguments: n_group 0 or 1 (none), or 2..MOE_MAXGROUP
// groups dividing the 256 experts, of which topk_group stay, holding at least 8 experts
__host__ __device__ inline bool route_groups_ok(int n_group, int topk_group) {
  if (n_group <= 1) return n_group >= 0;
  return n_group <= MOE_MAXGROUP && MOE_NEXP % n_group == 0 && topk_group >= 1 &&
         topk_group <= n_group && topk_group * (MOE_NEXP / n_group) >= MOE_TOPK;
}

// LDS routing state of one CTA
struct RouteLds {
  int32_t id[MOE_MAXR][MOE_SLOTS];  // slot 0: shared, then picks in selection order
  float w[MOE_MAXR][MOE_SLOTS];     // route weights (slot 0: 1)
  uint32_t mask[MOE_NDIST];         // per expert id: bit t = row t routed to it
  int32_t uexp[MOE_NDIST];          // distinct experts: u = 0 the shared, then ascending
  uint32_t umask[MOE_NDIST];
  int32_t uslot[MOE_NDIST];         // first (expert, row) slot of u; rows of u in order
  int32_t slot_ut[MOE_MAXR * MOE_SLOTS];  // slot -> (u << 8) | row
  int32_t nd;
};

// The top-k of one row, called by one whole wave. Lane l holds the scores of experts
// l + 64 i (i < 4) in `sc` and the matching biases in `bs`.
// Order: radix key of f32(score + bias) descending, then lower expert id
// (sgl_amd_mono/glm53/gfx950/kernel.py:1575-1629). Each lane sorts its four keys (ties
// to the lower slot, i.e. its lower id); a round takes the wave maximum of the lanes'
// heads (a DPP / permlane butterfly), then the lowest id holding it, and that lane pops
// its head. Writes slots 1..8 of row t into `rl` and sets the row's bit in rl.mask;
// weights are raw / (sum of the 8 raw, in pick order) * route_scale.
//
// Group-limited routing (n_group > 1, DeepSeek-V3's noaux_tc): the 256 experts form
// n_group groups of consecutive ids; a group's score is the sum of its two largest
// (score + bias) in f32 (the larger first); the topk_group groups of the largest scores
// (ties to the lower group) stay and every expert of another group drops out (key 0,
// below every real key) before the top-8. The caller checks 256 % n_group == 0,
// n_group <= MOE_MAXGROUP and topk_group * 256 / n_group >= 8.
__device__ inline void route_row(RouteLds& rl, int t, const float (&sc)[4], const float (&bs)[4],
                                 float route_scale, float* scores_out, int32_t* ids_out,
                                 float* weights_out, int n_group = 1, int topk_group = 1) {
  const int l = lane_id();
  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) key[i] = radix_key(sc[i] + bs[i]);
  if (n_group > 1) {
    const int gs = MOE_NEXP / n_group;  // experts a group
    float gsc = -INFINITY;              // lane g < n_group: group g's score
#pragma unroll 1
    for (int g = 0; g < n_group; ++g) {
      // the lane's two largest of group g, then the wave's: m1 the largest; m2 the
      // largest of the rest (m1 again when two lanes hold it)
      float a1 = -INFINITY, a2 = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = (l + 64 * i) / gs == g ? sc[i] + bs[i] : -INFINITY;
        if (v > a1) {
          a2 = a1;
          a1 = v;
        } else if (v > a2) {
          a2 = v;
        }
      }
      const float m1 = wave_max(a1);
      const uint64_t holders = __ballot(a1 == m1);
      const bool single = __popcll(holders) == 1;
      const bool mine = single && l == __ffsll((long long)holders) - 1;
      const float m2 = single ? wave_max(mine ? a2 : a1) : m1;
      if (l == g) gsc = m1 + m2;
    }
    // the topk_group best groups, ties to the lower group
    uint32_t live = 0;  // bit g: group g kept
#pragma unroll 1
    for (int k = 0; k < topk_group; ++k) {
      const bool cand = l < n_group && !((live >> l) & 1u);
      const float m = wave_max(cand ? gsc : -INFINITY);
      live |= 1u << (__ffsll((long long)__ballot(cand && gsc == m)) - 1);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (!((live >> ((l + 64 * i) / gs)) & 1u)) key[i] = 0;
  }
  // the lane's four candidates sorted by (key desc, slot asc): the next pick is always a
  // lane's head. Five compare-exchanges (a sorting network; the order is total, so
  // equal keys keep the lower slot first).
  uint32_t k[4];
  int s[4];
  float rw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k[i] = key[i];
    s[i] = i;
    rw[i] = sc[i];
  }
  auto cx = [&](int a, int b) {
    const bool sw = k[b] > k[a] || (k[b] == k[a] && s[b] < s[a]);
    const uint32_t ka = k[a], kb = k[b];
    const int sa = s[a], sb = s[b];
    const float ra = rw[a], rb = rw[b];
    k[a] = sw ? kb : ka;
    k[b] = sw ? ka : kb;
    s[a] = sw ? sb : sa;
    s[b] = sw ? sa : sb;
    rw[a] = sw ? rb : ra;
    rw[b] = sw ? ra : rb;
  };
  cx(0, 1);
  cx(2, 3);
  cx(0, 2);
  cx(1, 3);
  cx(1, 2);
  // A round takes the wave maximum of the heads; the pick is the lowest id holding it
  // (a single lane almost always; on a tie between lanes, the lowest slot * 64 + lane).
  // The owner pops its head. Rounds in a loop, not unrolled: this runs once a launch on
  // a few CTAs, so its code is fetched cold. Lane r keeps pick r; the sum of the raw
  // scores runs in pick order.
  float tot = 0.f, raw = 0.f;
  int e = 0;
#pragma unroll 1
  for (int r = 0; r < MOE_TOPK; ++r) {
    const uint32_t m = wave_max_u32(k[0]);
    const uint64_t held = __ballot(k[0] == m);
    int owner = __ffsll((long long)held) - 1;
    if (__popcll(held) != 1)
      owner = (int)(wave_min_u32(k[0] == m ? (uint32_t)(s[0] * 64 + l) : 0xFFFFFFFFu) & 63u);
    const float pr = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(rw[0]), owner));
    const int id = owner + 64 * __builtin_amdgcn_readlane(s[0], owner);
    tot += pr;
    if (l == r) {
      raw = pr;
      e = id;
    }
    const bool pop = l == owner;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      k[i] = pop ? k[i + 1] : k[i];
      s[i] = pop ? s[i + 1] : s[i];
      rw[i] = pop ? rw[i + 1] : rw[i];
    }
    k[3] = pop ? 0u : k[3];
    s[3] = pop ? 4 : s[3];
  }
  if (l < MOE_TOPK) {
    const float w = raw / tot * route_scale;
    rl.id[t][1 + l] = e;
    rl.w[t][1 + l] = w;
    atomicOr(&rl.mask[e], 1u << t);
    if (ids_out) ids_out[t * MOE_SLOTS + 1 + l] = e;
    if (weights_out) weights_out[t * MOE_SLOTS + 1 + l] = w;
  }
  if (l == 0) {
    rl.id[t][0] = MOE_SHARED;
    rl.w[t][0] = 1.f;
    if (ids_out) ids_out[t * MOE_SLOTS] = MOE_SHARED;
    if (weights_out) weights_out[t * MOE_SLOTS] = 1.f;
  }
  if (scores_out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) scores_out[t * MOE_NEXP + l + 64 * i] = sc[i];
  }
}

// exclusive prefix sum over the wave's lanes of a small count v < 2^BITS: one ballot
// per bit and a masked popcount (v_mbcnt), no cross-lane data movement
template <int BITS>
__device__ inline int wave_prefix(int v, int& total) {
  int pre = 0;
  total = 0;
#pragma unroll
  for (int k = 0; k < BITS; ++k) {
    const uint64_t bal = __ballot((v >> k) & 1);
    pre += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                         __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u))
           << k;
    total += __popcll(bal) << k;
  }
  return pre;
}

// Compact rl.mask into the distinct list (one whole wave): u = 0 the shared expert,
// then routed ids ascending, with each one's row mask. The up/gate stage needs only this.
__device__ inline void build_experts(RouteLds& rl, int rows) {
  const int l = lane_id();
  uint32_t m[4];
  int cnt = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    m[i] = rl.mask[4 * l + i];
    cnt += m[i] != 0;
  }
  int nroute = 0;
  int pos = 1 + wave_prefix<3>(cnt, nroute);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (m[i]) {
      rl.uexp[pos] = 4 * l + i;
      rl.umask[pos] = m[i];
      ++pos;
    }
  if (l == 0) {
    rl.nd = 1 + nroute;
    rl.uexp[0] = MOE_SHARED;
    rl.umask[0] = rows >= 32 ? 0xFFFFFFFFu : ((1u << rows) - 1u);
  }
}

// The (expert, row) slots of the distinct list built by build_experts (one whole wave;
// the list visible to it): uslot[u], the first slot of u (its rows in order), and
// slot_ut, slot -> (u << 8) | row. The mid quant and down stages need these.
__device__ inline void build_slots(RouteLds& rl, int rows) {
  const int l = lane_id();
  const int nd = rl.nd;
  const uint32_t shared_mask = rows >= 32 ? 0xFFFFFFFFu : ((1u << rows) - 1u);
  // lane l takes distinct experts u = 1 + 4 l .. 1 + 4 l + 3 (routed ones, in u order)
  uint32_t m[4];
  int c2 = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = 1 + 4 * l + i;
    m[i] = u < nd ? rl.umask[u] : 0u;
    c2 += __popc(m[i]);
  }
  int nslot = 0;
  int s = __popc(shared_mask) + wave_prefix<7>(c2, nslot);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int u = 1 + 4 * l + i;
    if (u < nd) {
      rl.uslot[u] = s;
      for (uint32_t mm = m[i]; mm; mm &= mm - 1) rl.slot_ut[s++] = (u << 8) | (__ffs(mm) - 1);
    }
  }
  if (l == 0) {
    rl.uslot[0] = 0;
    int s0 = 0;
    for (uint32_t mm = shared_mask; mm; mm &= mm - 1) rl.slot_ut[s0++] = __ffs(mm) - 1;
  }
}

// both, in order (the lists of build_experts written before build_slots reads them: one
// wave's LDS accesses complete in order)
__device__ inline void build_distinct(RouteLds& rl, int rows) {
  build_experts(rl, rows);
  __builtin_amdgcn_wave_barrier();
  build_slots(rl, rows);
}

// the slot of (u, row t), or -1 when row t is not routed to u
__device__ inline int slot_of(const RouteLds& rl, int u, uint32_t mask, int t) {
  return ((mask >> t) & 1u) ? rl.uslot[u] + __popc(mask & ((1u << t) - 1u)) : -1;
}

// route weight of row t for expert e (0 when e is not among its slots)
__device__ inline float route_weight(const RouteLds& rl, int t, int e) {
  float w = 0.f;
#pragma unroll
  for (int s = 0; s < MOE_SLOTS; ++s)
    if (rl.id[t][s] == e) w = rl.w[t][s];
  return w;
}

}  // namespace mono
