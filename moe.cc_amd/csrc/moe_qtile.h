// moe_qtile.h - quantized row-tile machinery shared by the GEMV and the MoE
// kernels: packed activation tables and exact integer row dots.
//
// Arithmetic contract (kernels.c:51-74, 96-128):
//   a_k = (int32)(x_k * 127.0f)  (Q8)   or  (int32)(x_k * 7.0f)  (Q4)
//   dot = sum_k a_k * w_k   in wrapping int32 (order-free, exact)
//
// Packed activation table ("act table") of one activation row, built once
// by pack_act_row and then read by every wave that needs the row:
//   header (16 B): nl (limbs needed: 1, 2 or 4), asum (sum_k a_k, wrapping)
//   4 limb planes of K bytes each (a = sum_l b_l 256^l, b_l signed int8):
//     Q8: plane dword d = limb of a[4d .. 4d+3]
//     Q4: plane dword d        (d < K/8)  = limb of a[8d], a[8d+2], a[8d+4], a[8d+6]
//         plane dword K/8 + d            = limb of a[8d+1], a[8d+3], a[8d+5], a[8d+7]
// so that one weight dword meets its activations in one (Q8) or two (Q4,
// even/odd nibbles) v_dot4_i32_i8 per limb.  Q4 weights enter as unsigned
// nibbles u = w + 8 and the offset is removed once per row: sum a*w =
// sum a*u - 8*asum.
#pragma once
#include <type_traits>

#include "moe_device.h"

namespace moe {

constexpr int kTileBlock = 256;
constexpr int kTileWaves = kTileBlock / kWave;

__host__ __device__ constexpr size_t act_table_bytes(int K) {
  return 16 + 4 * (((size_t)K + 15) / 16) * 16;
}
__device__ __forceinline__ int act_nl(const uint8_t* tab) {
  return *reinterpret_cast<const int*>(tab);
}
__device__ __forceinline__ uint32_t act_asum(const uint8_t* tab) {
  return *reinterpret_cast<const uint32_t*>(tab + 4);
}
__device__ __forceinline__ const uint32_t* act_plane(const uint8_t* tab, int K, int l) {
  return reinterpret_cast<const uint32_t*>(tab + 16 + (size_t)l * (((size_t)K + 15) / 16) * 16);
}

// Block-wide max of nl and sum of part into scratch[0] / scratch[1] (LDS,
// set to {1, 0} by the caller before a barrier): each wave reduces across
// its lanes first, then one LDS atomic pair per wave (hundreds of atomics on
// one address serialise: ~3 us for a 256-thread block, measured).  Whole
// waves only.
__device__ __forceinline__ void block_max_sum(int nl, uint32_t part, int* scratch) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const int o = __shfl_xor(nl, off, kWave);
    nl = o > nl ? o : nl;
    part += (uint32_t)__shfl_xor((int)part, off, kWave);
  }
  if (threadIdx.x % kWave == 0) {
    atomicMax(&scratch[0], nl);
    atomicAdd(reinterpret_cast<unsigned*>(&scratch[1]), part);
  }
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Unit u (columns 16u .. 16u + 15) of an x *unit* table (the expert-major
// path's layout: the act table's header and plane offsets, each limb plane
// a sequence of 16-byte units, Q8 in column order, Q4 the 8 even columns
// then the 8 odd ones): a = trunc(x * 7 or 127) (kernels.c:115 / :66) into
// the four planes; the limb count and the wrapping sum fold into nl / part.
template <bool Q4>
__device__ __forceinline__ void pack_unit16(const float (&x)[16], uint8_t* tab, int K, int u, int& nl,
                                            uint32_t& part) {
  const float mult = Q4 ? 7.0f : 127.0f;
  uint32_t b[16][4];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int32_t a = f2i_trunc_x86(x[i] * mult);
    const int n = limbs_needed(a);
    nl = n > nl ? n : nl;
    part += (uint32_t)a;
    split_limbs(a, b[i]);
  }
#pragma unroll
  for (int l = 0; l < 4; ++l) {
    u32x4 o;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      // Q4: dwords 0-1 the even columns, 2-3 the odd ones
      const int c0 = Q4 ? (d < 2 ? 8 * d : 8 * (d - 2) + 1) : 4 * d;
      const int st = Q4 ? 2 : 1;
      o[d] = pack4(b[c0][l], b[c0 + st][l], b[c0 + 2 * st][l], b[c0 + 3 * st][l]);
    }
    *reinterpret_cast<u32x4*>(const_cast<uint32_t*>(act_plane(tab, K, l)) + 4 * u) = o;
  }
}

// Packs one activation row into its table.  Called by a whole block (whole
// waves); contains barriers.  `scratch` is 2 ints of LDS.
template <bool Q4>
__device__ void pack_act_row(const float* __restrict__ x, int K, uint8_t* __restrict__ tab,
                             int* scratch) {
  const float mult = Q4 ? 7.0f : 127.0f;
  const size_t plane = (((size_t)K + 15) / 16) * 16;
  uint32_t* p0 = reinterpret_cast<uint32_t*>(tab + 16);
  if (threadIdx.x == 0) { scratch[0] = 1; scratch[1] = 0; }
  __syncthreads();
  int nl = 1;
  uint32_t part = 0;
  const int nd = Q4 ? (K + 7) / 8 : (K + 3) / 4;
  for (int d = threadIdx.x; d < nd; d += blockDim.x) {
    constexpr int V = Q4 ? 8 : 4;
    uint32_t b[V][4];
#pragma unroll
    for (int i = 0; i < V; ++i) {
      const int k = V * d + i;
      const int32_t v = k < K ? f2i_trunc_x86(x[k] * mult) : 0;
      const int n = limbs_needed(v);
      nl = n > nl ? n : nl;
      part += (uint32_t)v;
      split_limbs(v, b[i]);
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      uint32_t* pl = p0 + (size_t)l * (plane / 4);
      if constexpr (!Q4) {
        pl[d] = pack4(b[0][l], b[1][l], b[2][l], b[3][l]);
      } else {
        const int KW = (K + 7) / 8;
        pl[d] = pack4(b[0][l], b[2][l], b[4][l], b[6][l]);
        pl[KW + d] = pack4(b[1][l], b[3][l], b[5][l], b[7][l]);
      }
    }
  }
  block_max_sum(nl, part, scratch);
  __syncthreads();
  if (threadIdx.x == 0) {
    reinterpret_cast<int*>(tab)[0] = scratch[0];
    reinterpret_cast<uint32_t*>(tab)[1] = (uint32_t)scratch[1];
  }
}

// ---- tagged words: hand-overs between the blocks of one launch ----
//
// A 64-bit word {tag, value} stored and loaded with relaxed agent-scope
// atomics: a load sees the stores to its own address in order (per-location
// coherence, across the XCDs' L2s), so a reader that finds the current
// launch's tag has that launch's value -- no fence, no flag, no release
// (a device-scope release is an L2 write-back per block on gfx950).
__device__ __forceinline__ uint64_t tag_word(uint32_t tag, uint32_t v) {
  return ((uint64_t)tag << 32) | v;
}
__device__ __forceinline__ void tag_put(uint64_t* p, uint32_t tag, uint32_t v) {
  __hip_atomic_store(p, tag_word(tag, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The value at p once it carries `tag`; past `deadline` (wall clock) it
// stops waiting and sets `late` (the caller then poisons its results), so
// every wait ends.
__device__ __forceinline__ uint32_t tag_wait(const uint64_t* p, uint32_t tag, long long deadline,
                                             bool& late) {
  uint64_t w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while ((uint32_t)(w >> 32) != tag) {
    if (late || wall_clock64() > deadline) {
      late = true;
      break;
    }
    __builtin_amdgcn_s_sleep(2);
    w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  return (uint32_t)w;
}

// N tagged words at once (addr(i) gives word i's address): every load
// issued first, then only the stale words polled again, so the wait costs
// one round trip when the words are there.  Same deadline rule as tag_wait.
template <int N, int SLEEP = 2, class Addr>
__device__ __forceinline__ void tag_wait_all(Addr addr, uint32_t (&v)[N], uint32_t tag,
                                             long long deadline, bool& late) {
  uint64_t w[N];
#pragma unroll
  for (int i = 0; i < N; ++i) w[i] = __hip_atomic_load(addr(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) ok = ok && (uint32_t)(w[i] >> 32) == tag;
    if (ok || late) break;
    if (wall_clock64() > deadline) {
      late = true;
      break;
    }
    __builtin_amdgcn_s_sleep(SLEEP);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if ((uint32_t)(w[i] >> 32) != tag)
        w[i] = __hip_atomic_load(addr(i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = (uint32_t)w[i];
}

// Packs columns [c0, c1) of one activation row (x points at column 0) into
// the table's planes; c0 is a multiple of 8.  Returns this thread's limb
// count and activation sum over the columns it packed; threads of a team
// (tid in [0, nthr)) split the work.  ttab (optional): every plane dword
// also as a tagged word, plane l's dword i at ttab[l * plane dwords + i].
template <bool Q4>
__device__ void pack_act_cols(const float* x, int K, int c0, int c1, uint8_t* tab, int tid,
                              int nthr, int& nl_out, uint32_t& sum_out,
                              uint64_t* ttab = nullptr, uint32_t tag = 0) {
  const float mult = Q4 ? 7.0f : 127.0f;
  constexpr int V = Q4 ? 8 : 4;
  const size_t plane = (((size_t)K + 15) / 16) * 16;
  uint32_t* p0 = reinterpret_cast<uint32_t*>(tab + 16);
  const int KW = (K + 7) / 8;
  int nl = 1;
  uint32_t part = 0;
  const int nv = (c1 - c0 + V - 1) / V;
  for (int i = tid; i < nv; i += nthr) {
    const int d = c0 / V + i;
    uint32_t b[V][4];
#pragma unroll
    for (int v = 0; v < V; ++v) {
      const int k = V * d + v;
      const int32_t a = k < c1 ? f2i_trunc_x86(x[k] * mult) : 0;
      const int n = limbs_needed(a);
      nl = n > nl ? n : nl;
      part += (uint32_t)a;
      split_limbs(a, b[v]);
    }
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      uint32_t* pl = p0 + (size_t)l * (plane / 4);
      uint64_t* tl = ttab ? ttab + (size_t)l * (plane / 4) : nullptr;
      if constexpr (!Q4) {
        const uint32_t v = pack4(b[0][l], b[1][l], b[2][l], b[3][l]);
        pl[d] = v;
        if (tl) tag_put(tl + d, tag, v);
      } else {
        const uint32_t ve = pack4(b[0][l], b[2][l], b[4][l], b[6][l]);
        const uint32_t vo = pack4(b[1][l], b[3][l], b[5][l], b[7][l]);
        pl[d] = ve;
        pl[KW + d] = vo;
        if (tl) {
          tag_put(tl + d, tag, ve);
          tag_put(tl + KW + d, tag, vo);
        }
      }
    }
  }
  nl_out = nl;
  sum_out = part;
}

// ---- cross-lane integer sums with DPP ----
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, true);
}

// Sum over groups of W consecutive lanes (W = 4, 8, 16, 32, 64).  For W <= 16
// every lane of the group gets the total; for W = 32 / 64 lane 0 of the group
// is guaranteed to have it.
template <int W>
__device__ __forceinline__ uint32_t group_sum_dpp(uint32_t v) {
  v += dpp_u32<0xB1>(v);                 // quad_perm [1,0,3,2]
  v += dpp_u32<0x4E>(v);                 // quad_perm [2,3,0,1]
  if (W >= 8) v += dpp_u32<0x141>(v);    // row_half_mirror
  if (W >= 16) v += dpp_u32<0x140>(v);   // row_mirror
  if (W >= 32) v += (uint32_t)__shfl_xor((int)v, 16, kWave);
  if (W >= 64) v += (uint32_t)__shfl_xor((int)v, 32, kWave);
  return v;
}

// Geometry of one tiled configuration: a row of ROW_BYTES = LPR*P*16 bytes is
// read by LPR consecutive lanes, each with P dwordx4 loads at byte offsets
// (p*LPR + r)*16; a wave covers WR = 64/LPR rows at once.
template <int P_, int LPR_>
struct TileGeom {
  static constexpr int P = P_, LPR = LPR_;
  static constexpr int WR = kWave / LPR;
  static constexpr int DW = P * 4;                 // weight dwords per lane per row
  static constexpr int ROW_BYTES = LPR * P * 16;
};


// Weight rows are streamed once per launch: nontemporal loads keep them from
// displacing reused data in the caches (measured ~+15% streaming bandwidth).
// NT = false: ordinary loads, for launches in which several blocks read the
// same rows (the few-token expert kernels: tokens routed to one expert).
template <class G, bool NT = true>
__device__ __forceinline__ void load_row_regs(const uint8_t* row, uint32_t (&w)[G::DW]) {
  const int r = (threadIdx.x % kWave) % G::LPR;
#pragma unroll
  for (int p = 0; p < G::P; ++p) {
    const u32x4* src = reinterpret_cast<const u32x4*>(row + (size_t)(p * G::LPR + r) * 16);
    const u32x4 v = NT ? __builtin_nontemporal_load(src) : *src;
    w[4 * p + 0] = v.x; w[4 * p + 1] = v.y; w[4 * p + 2] = v.z; w[4 * p + 3] = v.w;
  }
}

// This lane's activation dwords for its weight chunk: Q8 -> a[l][i] (i <
// DW); Q4 -> even dwords in a[l][i], odd in a[l][DW + i].
template <bool Q4, class G, int NL>
struct ActRegs {
  uint32_t a[NL][Q4 ? 2 * G::DW : G::DW];
};

template <bool Q4, class G, int NL>
__device__ __forceinline__ void load_act_regs(const uint8_t* tab, int K, ActRegs<Q4, G, NL>& ar) {
  const int r = (threadIdx.x % kWave) % G::LPR;
#pragma unroll
  for (int l = 0; l < NL; ++l) {
    const uint32_t* pl = act_plane(tab, K, l);
#pragma unroll
    for (int p = 0; p < G::P; ++p) {
      const int d = (p * G::LPR + r) * 4;   // first weight dword of the chunk
      const uint4 e = *reinterpret_cast<const uint4*>(pl + d);
      ar.a[l][4 * p + 0] = e.x; ar.a[l][4 * p + 1] = e.y;
      ar.a[l][4 * p + 2] = e.z; ar.a[l][4 * p + 3] = e.w;
      if constexpr (Q4) {
        const uint4 o = *reinterpret_cast<const uint4*>(pl + (K + 7) / 8 + d);
        ar.a[l][G::DW + 4 * p + 0] = o.x; ar.a[l][G::DW + 4 * p + 1] = o.y;
        ar.a[l][G::DW + 4 * p + 2] = o.z; ar.a[l][G::DW + 4 * p + 3] = o.w;
      }
    }
  }
}

// This lane's partial dot of one weight row chunk with one activation row.
template <bool Q4, class G, int NL>
__device__ __forceinline__ uint32_t lane_dot(const uint32_t (&w)[G::DW],
                                             const ActRegs<Q4, G, NL>& ar) {
  int32_t acc[NL];
#pragma unroll
  for (int l = 0; l < NL; ++l) acc[l] = 0;
#pragma unroll
  for (int i = 0; i < G::DW; ++i) {
    if constexpr (!Q4) {
#pragma unroll
      for (int l = 0; l < NL; ++l) acc[l] = dot4(w[i], ar.a[l][i], acc[l]);
    } else {
      const uint32_t lo = w[i] & 0x0F0F0F0Fu;
      const uint32_t hi = (w[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int l = 0; l < NL; ++l) {
        acc[l] = dot4(lo, ar.a[l][i], acc[l]);
        acc[l] = dot4(hi, ar.a[l][G::DW + i], acc[l]);
      }
    }
  }
  return combine_limbs<NL>(acc);
}

// Streams rows [r0, r1) of NM matrices (W[mat], row stride rs) against MTI
// packed activation tables; each wave walks row groups gi = wave, wave+4, ...
// with the loads of the next group issued before the current one is reduced.
// For each valid row, lane 0 of its lane group calls
//     epi(row, tot)   with tot[mat][t] = exact int32 dot (Q4 offset removed).
// Row groups of loads in flight per wave.  Measured on MI355X: two beats
// three or four (registers limit occupancy).  Q4 with 2-limb activations
// (|x| > 18.1, rare) uses one, so that branch fits the 1-limb register
// budget the kernel is allocated for.
template <bool Q4, int NL>
constexpr int pf_for() { return (Q4 && NL > 1) ? 1 : 2; }

// The rows are shared by a team of nwv waves; this wave is number wv.
// asum_in (optional, per token slot) replaces the tables' header sums.
// The epilogue's per-row data (its scales) is fetched with the row's
// weights: epi.pre(row) at load time, epi(row, tot, pre) at the end, so the
// scale load's latency hides behind the weight stream.
template <bool Q4, class G, int NL, int MTI, int NM, bool NT = true, class Epi>
__device__ __forceinline__ void stream_rows(const uint8_t* const* W, long long rs, int K,
                                            const uint8_t* const* tab, int r0, int r1,
                                            Epi& epi, int wv, int nwv,
                                            const uint32_t* asum_in = nullptr) {
  ActRegs<Q4, G, NL> ar[MTI];
  uint32_t asum[MTI];
  const int lane = threadIdx.x % kWave, wave = wv;
  const int g = lane / G::LPR, r = lane % G::LPR;
  const int ngroups = (r1 - r0 + G::WR - 1) / G::WR;
  using Pre = typename Epi::Pre;
  auto load = [&](int gi, uint32_t (&w)[NM][G::DW], Pre& pd) {
    const int row = r0 + gi * G::WR + g;
    pd = epi.pre(row < r1 ? row : r0);
#pragma unroll
    for (int mat = 0; mat < NM; ++mat) {
      if (row < r1) {
        load_row_regs<G, NT>(W[mat] + (size_t)row * (size_t)rs, w[mat]);
      } else {
#pragma unroll
        for (int i = 0; i < G::DW; ++i) w[mat][i] = 0;
      }
    }
  };
  auto finish = [&](int gi, const uint32_t (&w)[NM][G::DW], const Pre& pd) {
    const int row = r0 + gi * G::WR + g;
    uint32_t tot[NM][MTI];
#pragma unroll
    for (int mat = 0; mat < NM; ++mat)
#pragma unroll
      for (int t = 0; t < MTI; ++t) {
        const uint32_t v = group_sum_dpp<G::LPR>(lane_dot<Q4, G, NL>(w[mat], ar[t]));
        tot[mat][t] = Q4 ? v - 8u * asum[t] : v;
      }
    if (r == 0 && row < r1) epi(row, tot, pd);
  };

  // PF row groups of loads in flight: group gi is reduced while the loads of
  // the next PF-1 groups of this wave are outstanding
  constexpr int PF = pf_for<Q4, NL>();
  uint32_t wr[PF][NM][G::DW];
  Pre pre[PF];
#pragma unroll
  for (int i = 0; i < PF; ++i)
    if (wave + i * nwv < ngroups) load(wave + i * nwv, wr[i], pre[i]);  // weights first
#pragma unroll
  for (int t = 0; t < MTI; ++t) {
    load_act_regs<Q4, G, NL>(tab[t], K, ar[t]);
    asum[t] = Q4 ? (asum_in ? asum_in[t] : act_asum(tab[t])) : 0u;
  }
  for (int base = 0;; base += PF) {
    bool done = false;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int gi = wave + (base + i) * nwv;
      if (gi >= ngroups) { done = true; break; }
      finish(gi, wr[i], pre[i]);
      const int gn = gi + PF * nwv;
      if (gn < ngroups) load(gn, wr[i], pre[i]);
    }
    if (done) break;
  }
}

// Token slots per weight pass so that activation registers stay within a
// budget (96 dwords for one matrix, 64 for two); 0 = does not fit.
// Activations needing 4 limbs (|x| > 257 for Q8), or more than one for Q4
// (|x| > 18.3, rare after RMSNorm), take the exact fp32 fallback, which keeps
// the tiled kernels' registers (and so their occupancy) at the one-limb
// budget for Q4 and the two-limb one for Q8 (|x| > 1.008 is common there).
template <bool Q4, class G, int NL, int NM>
constexpr int mti_for() {
  if (NL > 2 || (Q4 && NL > 1)) return 0;
  constexpr int per = NL * G::DW * (Q4 ? 2 : 1);
  constexpr int n = (NM == 1 ? 64 : 48) / per;
  return n >= 4 ? 4 : (n >= 2 ? 2 : (n >= 1 ? 1 : 0));
}

// Exact fallback on fp32 activations: one wave per row, wrapping int32
// multiply-add with the reference's byte addressing (row start n*rs, byte
// k/2 for Q4, odd-K guard).  Calls epi(row, tot) like stream_rows with one
// token slot.
template <bool Q4, int NM, class Epi>
__device__ void generic_rows_fp32(const uint8_t* const* W, long long rs, int K, const float* x,
                                  int r0, int r1, Epi& epi, int wv, int nwv) {
  const int lane = threadIdx.x % kWave;
  for (int row = r0 + wv; row < r1; row += nwv) {
    uint32_t tot[NM][1];
#pragma unroll
    for (int mat = 0; mat < NM; ++mat) {
      const uint8_t* wr = W[mat] + (size_t)row * (size_t)rs;
      uint32_t acc = 0;
      if constexpr (!Q4) {
        for (int k = lane; k < K; k += kWave)
          acc += (uint32_t)f2i_trunc_x86(x[k] * 127.0f) * (uint32_t)(int32_t)(int8_t)wr[k];
      } else {
        for (int j = lane; 2 * j < K; j += kWave) {
          const uint32_t byte = wr[j];
          const int k = 2 * j;
          acc += (uint32_t)f2i_trunc_x86(x[k] * 7.0f) * (uint32_t)((int32_t)(byte & 0x0Fu) - 8);
          if (k + 1 < K)
            acc += (uint32_t)f2i_trunc_x86(x[k + 1] * 7.0f) *
                   (uint32_t)((int32_t)((byte >> 4) & 0x0Fu) - 8);
        }
      }
      tot[mat][0] = group_sum_dpp<kWave>(acc);
    }
    if (lane == 0) epi(row, tot);
  }
}

// All tokens of a block against rows [r0, r1): picks the limb count from the
// tables' headers (uniform), then walks token chunks of the largest size that
// fits in registers.  make_epi(t0) returns the epilogue for token slots
// t0 .. t0+MTI-1 (an object with a templated operator()(row, tot)).
// xs[t] are the fp32 activation rows, used only by the exact fallback.
// nl_in > 0: the limb count of all tokens, and asum_in (per token, may be
// null) their activation sums, given instead of read from the headers.
template <bool Q4, class G, int NM, int MT, bool NT = true, class MakeEpi>
__device__ void stream_tokens(const uint8_t* const* W, long long rs, int K,
                              const uint8_t* const* tabs, const float* const* xs, int ntok, int r0,
                              int r1, MakeEpi& make_epi, int wv, int nwv, int nl_in = 0,
                              const uint32_t* asum_in = nullptr) {
  int nl = nl_in;
  if (nl <= 0) {
    nl = 1;
    for (int t = 0; t < ntok; ++t) {
      const int v = act_nl(tabs[t]);
      nl = v > nl ? v : nl;
    }
  }
  auto run = [&](auto nl_tag) {
    constexpr int NL = decltype(nl_tag)::value;
    constexpr int M0 = mti_for<Q4, G, NL, NM>();
    if constexpr (M0 == 0) {
      for (int t = 0; t < ntok; ++t) {
        auto epi = make_epi.template at<1>(t);
        generic_rows_fp32<Q4, NM>(W, rs, K, xs[t], r0, r1, epi, wv, nwv);
      }
    } else {
      constexpr int MTI = M0 < MT ? M0 : MT;
      for (int t0 = 0; t0 < ntok; t0 += MTI) {
        const uint8_t* tb[MTI];
#pragma unroll
        for (int t = 0; t < MTI; ++t) tb[t] = tabs[t0 + t < ntok ? t0 + t : ntok - 1];
        uint32_t as[MTI];
#pragma unroll
        for (int t = 0; t < MTI; ++t) as[t] = asum_in ? asum_in[t0 + t < ntok ? t0 + t : ntok - 1] : 0u;
        auto epi = make_epi.template at<MTI>(t0);
        stream_rows<Q4, G, NL, MTI, NM, NT>(W, rs, K, tb, r0, r1, epi, wv, nwv,
                                            asum_in ? as : nullptr);
      }
    }
  };
  if (nl == 1)
    run(std::integral_constant<int, 1>());
  else if (nl == 2)
    run(std::integral_constant<int, 2>());
  else
    run(std::integral_constant<int, 4>());
}

// Whole-block team: every wave of the block shares the rows.
template <bool Q4, class G, int NM, int MT, bool NT = true, class MakeEpi>
__device__ __forceinline__ void stream_tokens(const uint8_t* const* W, long long rs, int K,
                                              const uint8_t* const* tabs, const float* const* xs,
                                              int ntok, int r0, int r1, MakeEpi& make_epi,
                                              int nl_in = 0, const uint32_t* asum_in = nullptr) {
  stream_tokens<Q4, G, NM, MT, NT>(W, rs, K, tabs, xs, ntok, r0, r1, make_epi,
                               (int)(threadIdx.x / kWave), (int)(blockDim.x / kWave), nl_in,
                               asum_in);
}

// One wave alone streams rows [r0, r1) for one activation row whose limb
// count nl and activation sum asum are given (the table's header is not read).
template <bool Q4, class G, int NM, bool NT = true, class MakeEpi>
__device__ __forceinline__ void stream_row_wave(const uint8_t* const* W, long long rs, int K,
                                                const uint8_t* tab, const float* x, int r0,
                                                int r1, MakeEpi& make_epi, int nl,
                                                uint32_t asum) {
  const uint8_t* tabs[1] = {tab};
  const uint32_t as[1] = {asum};
  auto run = [&](auto nl_tag) {
    constexpr int NL = decltype(nl_tag)::value;
    if constexpr (mti_for<Q4, G, NL, NM>() == 0) {
      auto epi = make_epi.template at<1>(0);
      generic_rows_fp32<Q4, NM>(W, rs, K, x, r0, r1, epi, 0, 1);
    } else {
      auto epi = make_epi.template at<1>(0);
      stream_rows<Q4, G, NL, 1, NM, NT>(W, rs, K, tabs, r0, r1, epi, 0, 1, as);
    }
  };
  if (nl <= 1)
    run(std::integral_constant<int, 1>());
  else if (nl == 2)
    run(std::integral_constant<int, 2>());
  else
    run(std::integral_constant<int, 4>());
}

template <bool Q4, int NM, class Epi>
__device__ __forceinline__ void generic_rows_fp32(const uint8_t* const* W, long long rs, int K,
                                                  const float* x, int r0, int r1, Epi& epi) {
  generic_rows_fp32<Q4, NM>(W, rs, K, x, r0, r1, epi, (int)(threadIdx.x / kWave),
                            (int)(blockDim.x / kWave));
}

template <bool Q4, int NM, class Epi>
__device__ __forceinline__ void generic_rows_fp32_wave(const uint8_t* const* W, long long rs,
                                                       int K, const float* x, int r0, int r1,
                                                       Epi& epi) {
  generic_rows_fp32<Q4, NM>(W, rs, K, x, r0, r1, epi, 0, 1);
}

}  // namespace moe
