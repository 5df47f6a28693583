// expert_gemm.hip - the expert products of the many-token MoE block as
// grouped integer GEMMs on v_mfma_i32_32x32x32_i8 (gfx950), bit-identical to
// the per-(token, rank) GEMVs of test_model_trace.c:496-503.
//
// A block takes one task -- up to NP (token, rank) pairs routed to one
// expert, listed by group_kernel -- and one tile of rows.  Its waves form RG
// row groups x PG pair groups; a wave holds 64 weight rows (gate/up: 32
// gate and the same 32 up rows, so a lane holds g and u of one (row, pair)
// for the SwiGLU epilogue (:496-501); down: two 32-row tiles) and NTW pair
// tiles of 32 (tile t of pair group pg is the task's tile t * PG + pg).
// Tiles past the task's pairs skip their MFMAs and epilogue.
// K runs outermost in stages of 64 weight bytes per row (128 Q4 columns or
// 64 Q8 columns).  Both operands go straight from memory into a D-stage
// LDS ring with global_load_lds_dwordx4 (D - 1 stages ahead, no
// registers): the block's weight rows and the pairs' activation units (16
// bytes of one limb plane), which all waves share.  Both are XOR-swizzled
// so that the MFMA operand reads are free of bank conflicts.  One barrier
// per stage; the wait before it counts this wave's loads.
// Every unpacked weight operand feeds the wave's NTW pair tiles, and each
// weight byte leaves memory once per task.
//
// The integer dots are exact in any order.  A quantized activation a is
// split into int8 limbs a = sum_l b_l 256^l; a task whose activations need
// one limb runs one pass, otherwise the limbs run one after another and
// fold into a wrapping uint32 total (sum_l dot_l << 8l).  Q4 weights enter
// as unsigned nibbles u = w + 8 and sum a*w = sum a*u - 8*sum a is applied
// once per output.  The fp32 epilogues are the reference's operations in
// the reference's order.
//
// MFMA layout (checked on gfx950): A lane l = row l % 32 with 16 bytes of
// k-group l / 32; B lane l = column l % 32 with the same k-group; result
// register i of lane l = row 8*(i/4) + 4*(l/32) + i%4, column l % 32.  The
// columns a slot (lane half h, step s) stands for are this file's choice,
// made identically for both operands: 16-column unit u = h*S + s of the
// stage (S steps per stage), so a lane's weight bytes of one stage are the
// 32 contiguous bytes 32h .. 32h + 31 of the row's 64-byte stage chunk.
//
// Unit tables (this path's activation tables): the header and plane
// offsets of moe_qtile.h's act tables, but each limb plane is a sequence of
// 16-byte units, unit u = columns 16u .. 16u + 15: Q8 in column order, Q4
// the 8 even columns then the 8 odd ones (the order a packed weight dword's
// low nibbles, then high nibbles, take).  The router blocks write the x
// tables (pack_unit16, moe_grouped.hip), the gate/up epilogue the h tables.
#include <utility>

#include "moe_device.h"
#include "moe_internal.h"
#include "moe_layer.h"
#include "moe_lib.h"
#include "moe_qtile.h"

namespace moe {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned int v16u __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kEgWaves = 4;   // waves per block unless a shape says otherwise (the 256-pair shape: 8)

__device__ __forceinline__ v16i mfma32(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

template <bool Q4>
struct EgStage {
  static constexpr int S = Q4 ? 4 : 2;           // 32-column MFMA steps per stage
  static constexpr int COLS = 32 * S;            // columns per stage
  static constexpr int UNITS = 2 * S;            // 16-byte units per pair row
  static constexpr int ROWB = UNITS * 16;        // LDS bytes per pair row
  static constexpr int RPI = 1024 / ROWB;        // pair rows per LDS load instruction
};

// Slot of unit u in pair row r of an LDS stage: u ^ swz(r).  Q4 rows are 128
// bytes (one pass over the banks), Q8 rows 64: eight consecutive rows' reads
// of one unit then cover eight distinct 16-byte bank groups.
template <bool Q4>
__device__ __forceinline__ int swz(int r) {
  return Q4 ? (r & 7) : ((r >> 1) & 3);
}

// 32 weight bytes of one row for one stage: bytes 32h .. 32h + 31 of the
// row's 64-byte chunk.
struct WFrag32 {
  u32x4 w[2];
};

// A operand of step s: Q4 packed bytes 8s .. 8s + 7 of the fragment as
// [low nibbles of dwords 2s, 2s+1][high nibbles of the same]; Q8 bytes
// 16s .. 16s + 15.
template <bool Q4>
__device__ __forceinline__ v4i a_op(const WFrag32& f, int s) {
  v4i r;
  if constexpr (Q4) {
    const u32x4 w = f.w[s >> 1];
    const uint32_t w0 = (s & 1) ? w[2] : w[0];
    const uint32_t w1 = (s & 1) ? w[3] : w[1];
    constexpr uint32_t M = 0x0F0F0F0Fu;
    r[0] = (int)(w0 & M);
    r[1] = (int)(w1 & M);
    r[2] = (int)((w0 >> 4) & M);
    r[3] = (int)((w1 >> 4) & M);
  } else {
    const u32x4 w = f.w[s];
    r[0] = (int)w[0]; r[1] = (int)w[1]; r[2] = (int)w[2]; r[3] = (int)w[3];
  }
  return r;
}

// ---------------------------------------------------------------- passes

// The task's pairs, prefetched into LDS: pair id, activation table, the
// table's activation sum, and the epilogue's per-pair reductions.
struct EgPairs {
  int pair[kEgPairs];
  const uint8_t* tab[kEgPairs];
  uint32_t asum[kEgPairs];
  int red_nl[kEgPairs];
  unsigned red_sum[kEgPairs];
  int nl;
  int rot;   // the task index: stage rot % stages comes first
};

// Block shape: RG row groups x PG = NW / RG pair groups of NW waves.  Wave
// w is row group w % RG (64 weight rows: gate rows 0-31 and up rows 32-63
// of its 32 h-rows for gate/up, two 32-row tiles for down) and pair group w
// / RG (NTW tiles of 32 pairs).  A pass covers NP = 32 * NTW * PG pairs; D
// stages in the LDS ring.  LDS layout of one stage (pair row r = the pass's
// pair r):
//   W  64 * RG weight rows x 64 bytes, 16-byte chunk c of row r in slot
//      c ^ wswz(r);
//   B  NP pair rows x ROWB bytes, unit u of pair row r in slot u ^ swz(r).
__device__ __forceinline__ int wswz(int r) { return (r >> 1) & 3; }

template <bool Q4, int RG, int NTW, int D, int NW = kEgWaves>
struct EgCfg {
  static constexpr int W = NW;                                   // waves per block
  static constexpr int PG = NW / RG;
  static constexpr int NP = 32 * NTW * PG;
  static constexpr int W_BYTES = 64 * RG * 64;
  static constexpr int B_BYTES = NP * EgStage<Q4>::ROWB;
  static constexpr int STAGE = W_BYTES + B_BYTES;
  static constexpr int NIW = W_BYTES / 1024;                     // W load instructions (4 * RG)
  static constexpr int NIB = B_BYTES / 1024;                     // B load instructions
  static constexpr int PERW = NIW / NW;                          // per wave
  static constexpr int PERB = (NIB + NW - 1) / NW;               // per wave
  static constexpr int Q = PERW + PERB;                          // loads per wave per stage
  static constexpr size_t BYTES = (size_t)D * STAGE;
  static_assert(NW % RG == 0 && NIW % NW == 0, "block shape");
  static_assert(NP <= kEgPairs, "pairs of a pass");
};

// One 16-byte-per-lane global -> LDS load: lane i's 16 bytes from src land at
// LDS address lds + 16 i.  Issued from inline asm so that the compiler's
// wait-count bookkeeping, which does not place these loads correctly among
// the register loads, never sees them: every wait for them is explicit
// (stage_sync), and the compiler's own vmcnt waits only grow stricter.
// M0 is reserved to the compiler, which uses it in these kernels for nothing
// else (checked in the generated code), so setting it here is safe.
__device__ __forceinline__ void lds_load16(const void* src, uint8_t* lds) {
  const uint32_t la = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(la)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// Sixteen zero bytes: the B source of an h-table unit whose segment's values
// needed fewer limbs than the pass's limb (the gate/up epilogue writes only
// the planes a segment needs).
__device__ __align__(16) const uint8_t kEgZero[16] = {};

// This lane's load sources of a pass, at column 0: its weight chunks (LDS
// row 16 * ins + lane / 4, slot lane % 4, for the wave's instructions ins =
// wave + 4k) and its B units (limb plane l of pair row ins * RPI + lane /
// UNITS, slot lane % UNITS).  wrow(r) is the weight row behind LDS row r.
template <bool Q4, class C>
struct EgSrc {
  const uint8_t* w[C::PERW];
  const uint8_t* b[C::PERB];
  int nb;                   // B loads this wave issues per stage (its instructions holding a live pair row)
  uint32_t segs[C::PERB];   // SEGM passes: segments whose plane holds this B row's limb
  int col[C::PERB];         // column of this lane's B unit within a stage
};

template <bool Q4, class C, class WRow>
__device__ __forceinline__ void eg_sources(EgSrc<Q4, C>& src, WRow&& wrow, const EgPairs& sp,
                                           int pbase, int n, int K, int l, const uint32_t* segmask) {
  using SG = EgStage<Q4>;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
#pragma unroll
  for (int k = 0; k < C::PERW; ++k) {
    const int r = 16 * (wave + C::W * k) + lane / 4;
    src.w[k] = wrow(r) + 16 * ((lane % 4) ^ wswz(r));
  }
#pragma unroll
  for (int k = 0; k < C::PERB; ++k) {
    const int ins = (wave + C::W * k) % C::NIB;
    const int row = ins * SG::RPI + lane / SG::UNITS;
    const int unit = (lane % SG::UNITS) ^ swz<Q4>(row);
    const int q = min(pbase + row, n - 1);
    src.b[k] = reinterpret_cast<const uint8_t*>(act_plane(sp.tab[q], K, l)) + unit * 16;
    src.segs[k] = segmask && l > 0 ? segmask[(l - 1) * kEgPairs + q] : ~0u;
    src.col[k] = unit * 16;
  }
  // B instructions past the pass's pairs are not issued (shapes of more
  // than 128 pairs, where a pass is often half full; the smaller shapes
  // measured faster with every wave issuing PERB): instruction ins holds
  // pair rows ins * RPI ..; this wave issues ins = wave + W k
  if constexpr (C::NP > 128) {
    const int live = min(n - pbase, C::NP);
    const int nins = (live + SG::RPI - 1) / SG::RPI;
    src.nb = __builtin_amdgcn_readfirstlane(min(max((nins - wave + C::W - 1) / C::W, 0), C::PERB));
  } else {
    src.nb = C::PERB;
  }
}

// Loads stage st into buffer buf: this wave's PERW weight loads and src.nb
// B loads (a wave past the last B instruction repeats one another wave
// issued: the same bytes to the same place).  Pair rows past the pass's
// pairs inside an issued instruction repeat its last pair; the LDS rows of
// instructions not issued keep stale bytes, which only tiles' rows past the
// pairs read (their results are dropped).  SEGM: a B unit in a segment of
// BRS columns outside src.segs loads kEgZero.
template <bool Q4, class C, bool SEGM, int BRS>
__device__ __forceinline__ void stage_load(const EgSrc<Q4, C>& src, int st, size_t woff, uint8_t* buf) {
  using SG = EgStage<Q4>;
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int k = 0; k < C::PERW; ++k)
    lds_load16(src.w[k] + woff + (size_t)st * 64, buf + (wave + C::W * k) * 1024);
#pragma unroll
  for (int k = 0; k < C::PERB; ++k) {
    if (C::NP > 128 && k >= src.nb) break;
    const int ins = (wave + C::W * k) % C::NIB;
    const uint8_t* b = src.b[k] + (size_t)st * SG::UNITS * 16;
    if constexpr (SEGM) {
      const int seg = (st * SG::COLS + src.col[k]) / BRS;
      b = (src.segs[k] >> seg) & 1u ? b : kEgZero;
    }
    lds_load16(b, buf + C::W_BYTES + ins * 1024);
  }
}

// Waits for this wave's loads of the stage about to be read (N later loads
// may stay in flight) and its LDS reads, then joins the block: after it the
// whole stage is in LDS and every wave is done with the buffer that the
// next loads overwrite.
template <int N>
__device__ __forceinline__ void stage_sync() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// stage_sync with N = (D - 2) q, q this wave's loads per stage (uniform).
template <int D, int QMAX>
__device__ __forceinline__ void stage_sync_q(int q) {
  if constexpr (QMAX > 0) {
    if (q < QMAX) {
      stage_sync_q<D, QMAX - 1>(q);
      return;
    }
  }
  stage_sync<(D - 2) * QMAX>();
}

// This wave's 32 weight bytes of its row-group row 32m + lane % 32 (bytes
// 32h .. 32h + 31 of the stage chunk: chunks 2h and 2h + 1).
template <int RG>
__device__ __forceinline__ WFrag32 w_frag(const uint8_t* wbuf, int m) {
  const int lane = threadIdx.x % kWave, rg = (threadIdx.x / kWave) % RG, j = lane % 32, h = lane / 32;
  const int r = 64 * rg + 32 * m + j;
  const uint8_t* row = wbuf + r * 64;
  WFrag32 f;
  f.w[0] = *reinterpret_cast<const u32x4*>(row + 16 * ((2 * h) ^ wswz(r)));
  f.w[1] = *reinterpret_cast<const u32x4*>(row + 16 * ((2 * h + 1) ^ wswz(r)));
  return f;
}

// One step of the stage ring: wait for the stage in buffer cbuf, issue the
// loads of K stage lst (weights woff bytes further) into buffer lbuf, then
// the MFMAs of buffer cbuf: acc[m][t] for this wave's live pair tiles t <
// NL.
template <bool Q4, int RG, int NTW, int D, int NW, int NL, bool SEGM>
__device__ __forceinline__ void eg_stage(const EgSrc<Q4, EgCfg<Q4, RG, NTW, D, NW>>& src, int lst,
                                         size_t woff, int lbuf, int cbuf, uint8_t* lds,
                                         v16i (&acc)[2][NTW]) {
  using SG = EgStage<Q4>;
  using C = EgCfg<Q4, RG, NTW, D, NW>;
  const int lane = threadIdx.x % kWave, pg = (threadIdx.x / kWave) / RG, j = lane % 32, h = lane / 32;
  if constexpr (C::NP > 128)
    stage_sync_q<D, C::Q>(C::PERW + src.nb);
  else
    stage_sync<(D - 2) * C::Q>();
  stage_load<Q4, C, SEGM, 32 * RG>(src, lst, woff, lds + lbuf * C::STAGE);
  const uint8_t* buf = lds + cbuf * C::STAGE;
  const WFrag32 f0 = w_frag<RG>(buf, 0), f1 = w_frag<RG>(buf, 1);
  const uint8_t* B = buf + C::W_BYTES + (32 * pg + j) * SG::ROWB;
  const int sw = swz<Q4>(j);   // = swz(32 tile + j) for every tile
  if constexpr (NL <= 2) {
    // every B fragment of the stage requested before the first MFMA, so
    // that the reads' latencies overlap (the registers fit up to 2 tiles)
    v4i bf[SG::S][NL > 0 ? NL : 1];
#pragma unroll
    for (int s = 0; s < SG::S; ++s)
#pragma unroll
      for (int t = 0; t < NL; ++t)
        bf[s][t] = *reinterpret_cast<const v4i*>(B + 32 * C::PG * t * SG::ROWB + ((h * SG::S + s) ^ sw) * 16);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < SG::S; ++s) {
      const v4i a0 = a_op<Q4>(f0, s);
      const v4i a1 = a_op<Q4>(f1, s);
#pragma unroll
      for (int t = 0; t < NL; ++t) {
        acc[0][t] = mfma32(a0, bf[s][t], acc[0][t]);
        acc[1][t] = mfma32(a1, bf[s][t], acc[1][t]);
      }
    }
  } else {
#pragma unroll
    for (int s = 0; s < SG::S; ++s) {
      const v4i a0 = a_op<Q4>(f0, s);
      const v4i a1 = a_op<Q4>(f1, s);
      const int slot = (h * SG::S + s) ^ sw;
#pragma unroll
      for (int t = 0; t < NL; ++t) {
        const v4i b = *reinterpret_cast<const v4i*>(B + 32 * C::PG * t * SG::ROWB + slot * 16);
        acc[0][t] = mfma32(a0, b, acc[0][t]);
        acc[1][t] = mfma32(a1, b, acc[1][t]);
      }
    }
  }
}

// The stage loop of a wave with NL live tiles; NL is chosen once per pass
// (live_tiles), so that the MFMA sequence of a stage has no branches.
template <bool Q4, int RG, int NTW, int D, int NW, int NL, bool SEGM>
__device__ __forceinline__ void eg_loop(const EgSrc<Q4, EgCfg<Q4, RG, NTW, D, NW>>& src, int nst, int rot,
                                        int ntl, uint8_t* lds, v16i (&acc)[2][NTW]) {
  if constexpr (NL > 0) {
    if (ntl < NL) {
      eg_loop<Q4, RG, NTW, D, NW, NL - 1, SEGM>(src, nst, rot, ntl, lds, acc);
      return;
    }
  }
  for (int st = 0; st < nst; ++st)
    eg_stage<Q4, RG, NTW, D, NW, NL, SEGM>(src, (min(st + D - 1, nst - 1) + rot) % nst, 0,
                                           (st + D - 1) % D, st % D, lds, acc);
}

// The ring run on across R consecutive row tiles (weights wstep bytes
// apart): step g is K stage g % nst of row tile g / nst, so the first loads
// of a tile are issued during the last stages of the one before.  After a
// tile's last stage epi(r, acc) takes its dots (epi must leave the ring
// alone) and the accumulators restart.  One limb (no segment masks).
template <bool Q4, int RG, int NTW, int D, int NW, int NL, class Epi>
__device__ __forceinline__ void eg_loop_rows(const EgSrc<Q4, EgCfg<Q4, RG, NTW, D, NW>>& src, int nst,
                                             int rot, int R, size_t wstep, int ntl, uint8_t* lds, Epi& epi) {
  if constexpr (NL > 0) {
    if (ntl < NL) {
      eg_loop_rows<Q4, RG, NTW, D, NW, NL - 1>(src, nst, rot, R, wstep, ntl, lds, epi);
      return;
    }
  }
  using C = EgCfg<Q4, RG, NTW, D, NW>;
  v16i acc[2][NTW];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int t = 0; t < NTW; ++t) acc[m][t] = v16i{};
  const int total = nst * R;
  for (int p = 0; p < D - 1; ++p) {
    const int gl = min(p, total - 1);
    stage_load<Q4, C, false, 32 * RG>(src, (gl % nst + rot) % nst, (size_t)(gl / nst) * wstep,
                                      lds + p * C::STAGE);
  }
  for (int g = 0; g < total; ++g) {
    const int gl = min(g + D - 1, total - 1);
    eg_stage<Q4, RG, NTW, D, NW, NL, false>(src, (gl % nst + rot) % nst, (size_t)(gl / nst) * wstep,
                                            (g + D - 1) % D, g % D, lds, acc);
    if (g % nst == nst - 1) {
      epi(g / nst, acc);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int t = 0; t < NTW; ++t) acc[m][t] = v16i{};
    }
  }
  stage_sync<0>();
}

// Live pair tiles of this wave in a pass over pairs pbase .. n - 1: tiles t
// with 32 (t PG + pg) < n - pbase.  The same for every lane of the wave.
template <int PG, int NTW>
__device__ __forceinline__ int live_tiles(int pbase, int n, int pg) {
  const int live = n - pbase;   // >= 1
  const int tiles = (live + 31) / 32;
  const int t = (tiles - pg + PG - 1) / PG;
  return __builtin_amdgcn_readfirstlane(min(max(t, 0), NTW));
}

// acc[m][t] = sum over all K columns of W_m[lane's row] x limb l of pair
// pbase + 32 (NTW pg + t) + (lane % 32).  Every thread of the block calls
// this.  On return every load of the pass has landed and every wave is done
// with the LDS ring.
template <bool Q4, int RG, int NTW, int D, int NW, bool SEGM, class WRow>
__device__ __forceinline__ void eg_pass(WRow&& wrow, int K, const EgPairs& sp, int pbase, int n,
                                        int l, const uint32_t* segmask, uint8_t* lds, v16i (&acc)[2][NTW]) {
  using SG = EgStage<Q4>;
  using C = EgCfg<Q4, RG, NTW, D, NW>;
  const int nst = K / SG::COLS;
  const int ntl = live_tiles<C::PG, NTW>(pbase, n, (threadIdx.x / kWave) / RG);
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int t = 0; t < NTW; ++t) acc[m][t] = v16i{};
  EgSrc<Q4, C> src;
  eg_sources<Q4, C>(src, wrow, sp, pbase, n, K, l, segmask);
  // the stages run in a rotated order, one per task (the dots are exact in
  // any order): concurrent tasks read different column slices of their
  // rows, while the row blocks of one task (one XCD, dispatched together)
  // read the same activation units at about the same time, from its L2
  // (by block instead: gate/up fetched 280 MB against 256 at T = 2048)
  const int rot = sp.rot % nst;
#pragma unroll
  for (int p = 0; p < D - 1; ++p)
    stage_load<Q4, C, SEGM, 32 * RG>(src, (min(p, nst - 1) + rot) % nst, 0, lds + p * C::STAGE);
  eg_loop<Q4, RG, NTW, D, NW, NTW, SEGM>(src, nst, rot, ntl, lds, acc);
  // the clamped loads past the last stage land before the ring is reused
  stage_sync<0>();
}

// Dots of a pass over all limbs: one pass (nl == 1) or limb passes folded
// into wrapping uint32 totals.  segmask (down: [3][kEgPairs] in LDS, else
// null): bit s of segmask[l - 1][pair] says segment s of the pair's h
// table holds limb plane l.
template <bool Q4, int RG, int NTW, int D, int NW, class WRow>
__device__ __forceinline__ void eg_dots(WRow&& wrow, int K, const EgPairs& sp, int pbase, int n,
                                        int nl, const uint32_t* segmask, uint8_t* lds,
                                        v16u (&dots)[2][NTW]) {
  v16i acc[2][NTW];
  eg_pass<Q4, RG, NTW, D, NW, false>(wrow, K, sp, pbase, n, 0, nullptr, lds, acc);
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int t = 0; t < NTW; ++t) dots[m][t] = __builtin_bit_cast(v16u, acc[m][t]);
  for (int l = 1; l < nl; ++l) {
    if (segmask)
      eg_pass<Q4, RG, NTW, D, NW, true>(wrow, K, sp, pbase, n, l, segmask, lds, acc);
    else
      eg_pass<Q4, RG, NTW, D, NW, false>(wrow, K, sp, pbase, n, l, nullptr, lds, acc);
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int t = 0; t < NTW; ++t) dots[m][t] += __builtin_bit_cast(v16u, acc[m][t]) << (8u * l);
  }
}

// One-limb dots of R consecutive row tiles (weights wstep bytes apart) over
// all n pairs of the task, epi(r, acc) after each tile (eg_loop_rows).
template <bool Q4, int RG, int NTW, int D, int NW, class WRow, class Epi>
__device__ __forceinline__ void eg_rows(WRow&& wrow, int K, const EgPairs& sp, int n, int R, size_t wstep,
                                        uint8_t* lds, Epi&& epi) {
  using SG = EgStage<Q4>;
  using C = EgCfg<Q4, RG, NTW, D, NW>;
  const int nst = K / SG::COLS;
  const int ntl = live_tiles<C::PG, NTW>(0, n, (threadIdx.x / kWave) / RG);
  EgSrc<Q4, C> src;
  eg_sources<Q4, C>(src, wrow, sp, 0, n, K, 0, nullptr);
  const int rot = sp.rot % nst;
  eg_loop_rows<Q4, RG, NTW, D, NW, NTW>(src, nst, rot, R, wstep, ntl, lds, epi);
}

// Where row r of an activation unit table sits in its limb plane.
template <bool Q4>
__device__ __forceinline__ int unit_byte(int r) {
  if constexpr (!Q4) return r;
  const int i = r % 16;
  return (r - i) + ((i & 1) ? 8 + i / 2 : i / 2);
}

struct EgArgs {
  const uint8_t* w0; const uint8_t* w1;   // gate and up (gate/up) or down (w1 unused)
  const float* s0; const float* s1;       // their row scales [E][rows]
  long long rb;                           // weight row bytes
  int rows;                               // rows per expert (d_ff or D)
  int K;                                  // logical columns (D or d_ff)
  int topk;
  const int* perm;                        // pair ids grouped by expert
  const int2* tasks;                      // {expert | pairs << 16, first pair}, x < 0 past the end
  int ntask;                              // entries of tasks
  const uint8_t* tab;                     // x tables [T] (gate/up) or h tables [pairs] (down)
  size_t tab_bytes;
  uint8_t* htab; size_t htab_bytes;       // gate/up: h tables out
  uint32_t* hpart; int nseg;              // per-segment h headers: written by gate/up, read by down
  float* y;                               // down: [pairs][D]
  int16_t* y16;                           // down, Q4: [pairs][D] dots that fit int16, else -32768 and y
  int rtpb;                               // down: row tiles per block (rows % tile == 0 when > 1)
};

// Block -> (task, row tile), so that the row tiles of a task run on one XCD
// (blocks are dealt to the 8 XCDs in turn) and share its L2.  The grid is
// nrt * ceil8(ntask) blocks.  Returns false past the last task.
__device__ __forceinline__ bool eg_block(int ntask, int nrt, int* task, int* rt) {
  const int lin = blockIdx.x, xcd = lin % 8, k = lin / 8;
  *task = (k / nrt) * 8 + xcd;
  *rt = k % nrt;
  return *task < ntask;
}

// ---------------------------------------------------------------- gate/up

// SwiGLU epilogue of one pass (:496-501): lane (j, h) of wave (rg, pg) holds,
// for pair pbase + 32 (t PG + pg) + j, gate and up dots of rows rb + 32 rg +
// 8q + 4h + r.  h = (g / (1 + expf(-g))) * u is quantized for down.  The
// block's h rows of one pair are BR consecutive bytes of each limb plane of
// its h table (rb % 16 == 0), so they are assembled in LDS (stg, the free
// ring of RING bytes) and written 16 bytes a lane, and only the limb planes this
// segment needs: limb counts and activation sums per pair go to red_nl /
// red_sum (then to hpart), and down reads zeros for a plane past a
// segment's count.  `flag` (LDS, 0 on entry) marks a block whose values
// need more than one limb; it is 0 again on return.
template <bool Q4, int RG, int PG, int NTW, size_t RING>
__device__ __forceinline__ void gate_up_epi(const EgArgs& a, EgPairs& sp, v16u (&dots)[2][NTW],
                                            int pbase, int n, int rb, const float* sg,
                                            const float* su, const uint64_t* exp_tab, uint8_t* stg,
                                            int* flag) {
  constexpr int BR = 32 * RG;          // h rows of the block
  constexpr int SROW = BR + 4;         // staging row of a pair (odd dword count: no bank conflicts)
  constexpr int NPP = 32 * PG * NTW;   // pairs of the pass
  constexpr int PLANE = NPP * SROW;
  constexpr int NTH = 64 * RG * PG;
  constexpr int PR = RING / PLANE < 4 ? RING / PLANE : 4;   // staged planes per round
  static_assert(PR >= 1, "one staged plane fits in the LDS ring");
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, j = lane % 32, h = lane / 32;
  const int rg = wave % RG, pg = wave / RG;
  const float div = Q4 ? 7.0f : 127.0f;
  const int ntl = live_tiles<PG, NTW>(pbase, n, pg);
  // 1. h values (in place of the gate dots), limb counts and sums per pair
  int multi = 0;
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    if (t >= ntl) break;
    const int i = pbase + 32 * (PG * t + pg) + j;
    const uint32_t xs = sp.asum[min(i, n - 1)];
    // the rows' value range (limbs_needed is monotone in |value|; a row
    // past the matrix counts as 0) and wrapping sum
    int32_t lo = 0, hi = 0;
    uint32_t hs = 0;
    const int rows_left = a.rows - rb - 32 * rg - 4 * h;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int lr = 32 * rg + 8 * q + 4 * h;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint32_t dg = dots[0][t][4 * q + r], du = dots[1][t][4 * q + r];
        if (Q4) { dg -= 8u * xs; du -= 8u * xs; }
        const float gv = qdot_epilogue(dg, div, sg[lr + r]);
        const float uv = qdot_epilogue(du, div, su[lr + r]);
        const int32_t hv = f2i_trunc_x86(silu_mul_t(gv, uv, exp_tab) * div);
        dots[0][t][4 * q + r] = (uint32_t)hv;
        const int32_t hc = 8 * q + r < rows_left ? hv : 0;
        lo = hc < lo ? hc : lo;
        hi = hc > hi ? hc : hi;
        hs += (uint32_t)hc;
      }
    }
    int nl = max(limbs_needed(lo), limbs_needed(hi));
    // lanes j and j + 32 hold the same pair
    const int o = __shfl_xor(nl, 32, kWave);
    nl = o > nl ? o : nl;
    hs += (uint32_t)__shfl_xor((int)hs, 32, kWave);
    if (h == 0 && i < n) {
      atomicMax(&sp.red_nl[i], nl);
      atomicAdd(&sp.red_sum[i], hs);
    }
    multi |= i < n && nl > 1;   // rows of pairs past the pass hold stale values
  }
  if (__any(multi) && lane == 0) atomicOr(flag, 1);
  __syncthreads();
  const bool bmulti = *flag != 0;
  // 2-3. limb planes in rounds of PR planes (one round unless the block
  // needs several limbs and the ring holds fewer than four planes): bytes
  // into the staging rows (every row of a live pair is written), then
  // 16-byte pieces of the planes each pair's segment needs
  const int nlw = bmulti ? 4 : 1;
  constexpr int NCH = BR / 16;
  const int live = min(n - pbase, NPP);
  for (int l0 = 0; l0 < nlw; l0 += PR) {
    const int nr = min(PR, nlw - l0);
#pragma unroll
    for (int t = 0; t < NTW; ++t) {
      if (t >= ntl) break;
      uint8_t* row = stg + (32 * (PG * t + pg) + j) * SROW;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lr = 32 * rg + 8 * q + 4 * h;
        uint32_t b[4][4];   // [r][limb]
#pragma unroll
        for (int r = 0; r < 4; ++r) split_limbs((int32_t)dots[0][t][4 * q + r], b[r]);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
          // rows lr .. lr + 3 (lr % 4 == 0): Q8 4 consecutive bytes; Q4 the
          // even rows 2 bytes in the unit's first half, the odd rows 2 in its
          // second
          if (l < l0 || l >= l0 + nr) continue;
          uint8_t* pl = row + (l - l0) * PLANE;
          if constexpr (!Q4) {
            *reinterpret_cast<uint32_t*>(pl + lr) = pack4(b[0][l], b[1][l], b[2][l], b[3][l]);
          } else {
            *reinterpret_cast<uint16_t*>(pl + unit_byte<true>(lr)) = (uint16_t)(b[0][l] | (b[2][l] << 8));
            *reinterpret_cast<uint16_t*>(pl + unit_byte<true>(lr + 1)) = (uint16_t)(b[1][l] | (b[3][l] << 8));
          }
        }
      }
    }
    __syncthreads();
    const int total = live * NCH * nr;
    for (int k = threadIdx.x; k < total; k += NTH) {
      const int kl = k / (live * NCH), rem = k - kl * live * NCH, p = rem / NCH, c = rem - p * NCH;
      const int i = pbase + p, l = l0 + kl;
      if (l < sp.red_nl[i] && rb + 16 * c < a.rows) {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(stg + kl * PLANE + p * SROW + 16 * c);
        u32x4 v;
        v[0] = src[0]; v[1] = src[1]; v[2] = src[2]; v[3] = src[3];
        uint8_t* tabq = a.htab + (size_t)sp.pair[i] * a.htab_bytes;
        *reinterpret_cast<u32x4*>(reinterpret_cast<uint8_t*>(const_cast<uint32_t*>(act_plane(tabq, a.rows, l))) +
                                  rb + 16 * c) = v;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) *flag = 0;
}

// gate/up + SwiGLU for one row tile (32 RG rows of d_ff) of one task.
template <bool Q4, int RG, int NTW, int D, int NW>
__global__ __launch_bounds__(64 * NW) void gate_up_eg_kernel(EgArgs a) {
  using C = EgCfg<Q4, RG, NTW, D, NW>;
  constexpr int NTH = 64 * NW;
  constexpr int BR = 32 * RG;   // h-rows per block
  extern __shared__ u32x4 lds_eg[];
  __shared__ EgPairs sp;
  __shared__ float sg[BR], su[BR];
  __shared__ uint64_t exp_tab[32];
  __shared__ int multi_flag;
  uint8_t* lds = reinterpret_cast<uint8_t*>(lds_eg);
  int ti, rt;
  if (!eg_block(a.ntask, (a.rows + BR - 1) / BR, &ti, &rt)) return;
  const int2 task = a.tasks[ti];
  if (task.x < 0) return;
  const int e = task.x & 0xFFFF, n = task.x >> 16, first = task.y;
  if (n > C::NP) return;   // group_kernel splits tasks at NP pairs
  const int tid = threadIdx.x;
  const int rb = rt * BR;
  if (tid < 32) exp_tab[tid] = kExp2Tab[tid];
  for (int t2 = tid; t2 < BR; t2 += NTH) {
    const int row = min(rb + t2, a.rows - 1);
    sg[t2] = a.s0[(size_t)e * a.rows + row];
    su[t2] = a.s1[(size_t)e * a.rows + row];
  }
  if (tid == 0) {
    sp.nl = 1;
    sp.rot = ti;
    multi_flag = 0;
  }
  __syncthreads();
  int nl = 1;
  for (int i = tid; i < n; i += NTH) {
    const int q = a.perm[first + i];
    const uint8_t* tb = a.tab + (size_t)(q / a.topk) * a.tab_bytes;
    sp.pair[i] = q;
    sp.tab[i] = tb;
    sp.asum[i] = act_asum(tb);
    sp.red_nl[i] = 1;
    sp.red_sum[i] = 0;
    const int v = min(act_nl(tb), 4);   // 1, 2 or 4; never past the table's planes
    nl = v > nl ? v : nl;
  }
  if (nl > 1) atomicMax(&sp.nl, nl);
  __syncthreads();
  // LDS row r: row group r / 64, gate (r % 64 < 32) or up, h-row rb + 32 (r
  // / 64) + r % 32
  const uint8_t* g0 = a.w0 + (size_t)e * a.rows * a.rb;
  const uint8_t* u0 = a.w1 + (size_t)e * a.rows * a.rb;
  auto wrow = [&](int r) {
    const int row = min(rb + 32 * (r / 64) + r % 32, a.rows - 1);
    return ((r % 64) < 32 ? g0 : u0) + (size_t)row * a.rb;
  };
  const int nlt = sp.nl;
  // half the tiles and one more ring stage (DH) when they fit the same LDS:
  // the 256-pair shape's tasks of at most 128 pairs, and its limb passes
  constexpr int NTM = NTW > 1 ? NTW / 2 : 1;
  constexpr int DH = EgCfg<Q4, RG, NTM, D + 1, NW>::BYTES <= C::BYTES && C::NP > 128 ? D + 1 : D;
  if (nlt == 1 && (DH == D || n > EgCfg<Q4, RG, NTM, DH, NW>::NP)) {
    v16u dots[2][NTW];
    eg_dots<Q4, RG, NTW, D, NW>(wrow, a.K, sp, 0, n, 1, nullptr, lds, dots);
    gate_up_epi<Q4, RG, C::PG, NTW, C::BYTES>(a, sp, dots, 0, n, rb, sg, su, exp_tab, lds, &multi_flag);
  } else {
    // limb passes over half as many pairs at a time (the totals take the
    // other half of the accumulator budget); one limb here when the task
    // fits a half pass
    constexpr int NPM = EgCfg<Q4, RG, NTM, DH, NW>::NP;
    v16u dots[2][NTM];
    for (int pb = 0; pb < n; pb += NPM) {
      eg_dots<Q4, RG, NTM, DH, NW>(wrow, a.K, sp, pb, n, nlt, nullptr, lds, dots);
      gate_up_epi<Q4, RG, C::PG, NTM, C::BYTES>(a, sp, dots, pb, n, rb, sg, su, exp_tab, lds, &multi_flag);
    }
  }
  __syncthreads();
  // this block's segment of each pair's h header
  for (int i = tid; i < n; i += NTH) {
    uint32_t* pp = a.hpart + ((size_t)sp.pair[i] * a.nseg + rt) * 2;
    pp[0] = (uint32_t)sp.red_nl[i];
    pp[1] = sp.red_sum[i];
  }
}

// ---------------------------------------------------------------- down

// y epilogue of one pass (:502-503): lane (j, h) of wave (rg, pg) holds, for
// pair pbase + 32 (t PG + pg) + j, the dots of rows rb + 64 rg + 32m + 8q +
// 4h + r.  Q8: y = ((float)dot / 127) * scale in fp32.  Q4: the int32 dot
// itself (after the -8 sum correction) as int16 when it lies in [-32767,
// 32767] -- y is a function of the dot and the row's scale, so the combine
// forms the same fp32 value from it -- else -32768 there and the fp32 y in
// a.y: half the bytes written here and read by the combine.
template <bool Q4, int RG, int PG, int NTW>
__device__ __forceinline__ void down_epi(const EgArgs& a, const EgPairs& sp, const v16u (&dots)[2][NTW],
                                         int pbase, int n, int rb, const float* sd) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave, j = lane % 32, h = lane / 32;
  const int rg = wave % RG, pg = wave / RG;
  const float div = Q4 ? 7.0f : 127.0f;
#pragma unroll
  for (int t = 0; t < NTW; ++t) {
    const int i = pbase + 32 * (PG * t + pg) + j;
    if (i >= n) continue;
    const uint32_t hs = sp.asum[i];
    float* yq = a.y + (size_t)sp.pair[i] * a.rows;
    int16_t* y16q = Q4 ? a.y16 + (size_t)sp.pair[i] * a.rows : nullptr;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lr = 64 * rg + 32 * m + 8 * q + 4 * h;
        if (rb + lr >= a.rows) continue;
        if constexpr (Q4) {
          uint32_t d[4];
          bool fits = true;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            d[r] = dots[m][t][4 * q + r] - 8u * hs;
            fits = fits && d[r] + 32767u <= 65534u;   // (int32)d in [-32767, 32767]
          }
          uint2 v;
          v.x = (d[0] & 0xFFFFu) | (d[1] << 16);
          v.y = (d[2] & 0xFFFFu) | (d[3] << 16);
          if (!fits) {
            // rare: the four outputs go to y, the int16 slots hold the marker
            float yv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) yv[r] = qdot_epilogue(d[r], div, sd[lr + r]);
            *reinterpret_cast<float4*>(yq + rb + lr) = make_float4(yv[0], yv[1], yv[2], yv[3]);
            v.x = v.y = 0x80008000u;
          }
          *reinterpret_cast<uint2*>(y16q + rb + lr) = v;
        } else {
          float yv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) yv[r] = qdot_epilogue(dots[m][t][4 * q + r], div, sd[lr + r]);
          *reinterpret_cast<float4*>(yq + rb + lr) = make_float4(yv[0], yv[1], yv[2], yv[3]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
  }
}

// Row tiles of down per block at most.
constexpr int kDownRowTiles = 4;

// down for a.rtpb consecutive row tiles (64 RG rows of D each) of one task:
// y per pair.  The tiles share the block's pair prologue and its load ring.
template <bool Q4, int RG, int NTW, int D, int NW>
__global__ __launch_bounds__(64 * NW) void down_eg_kernel(EgArgs a) {
  using C = EgCfg<Q4, RG, NTW, D, NW>;
  constexpr int NTH = 64 * NW;
  constexpr int BR = 64 * RG;   // rows per tile
  extern __shared__ u32x4 lds_eg[];
  __shared__ EgPairs sp;
  __shared__ float sd[kDownRowTiles * BR];
  __shared__ uint32_t segmask[3 * kEgPairs];
  uint8_t* lds = reinterpret_cast<uint8_t*>(lds_eg);
  const int nrt = (a.rows + BR - 1) / BR;
  int ti, rg;
  if (!eg_block(a.ntask, (nrt + a.rtpb - 1) / a.rtpb, &ti, &rg)) return;
  const int2 task = a.tasks[ti];
  if (task.x < 0) return;
  const int e = task.x & 0xFFFF, n = task.x >> 16, first = task.y;
  if (n > C::NP) return;   // group_kernel splits tasks at NP pairs
  const int tid = threadIdx.x;
  const int rt0 = rg * a.rtpb, R = min(a.rtpb, nrt - rt0);
  const int rb0 = rt0 * BR;
  for (int r = tid; r < R * BR; r += NTH) sd[r] = a.s0[(size_t)e * a.rows + min(rb0 + r, a.rows - 1)];
  if (tid == 0) {
    sp.nl = 1;
    sp.rot = ti;
  }
  for (int i = tid; i < n; i += NTH) {
    sp.pair[i] = a.perm[first + i];
    sp.red_nl[i] = 1;
    sp.red_sum[i] = 0;
    segmask[i] = segmask[kEgPairs + i] = segmask[2 * kEgPairs + i] = 0u;
  }
  __syncthreads();
  // the pairs' h headers: the sum of the segments' activation sums and the
  // largest limb count, one (pair, segment) entry per thread
  for (int k = tid; k < n * a.nseg; k += NTH) {
    const int i = k / a.nseg, sg = k - i * a.nseg;
    const uint32_t* pp = a.hpart + ((size_t)sp.pair[i] * a.nseg + sg) * 2;
    // 1, 2 or 4 limbs (limbs_needed); held to 4 so that no value can send
    // the limb passes past a table's four planes
    const int v = min((int)pp[0], 4);
    if (v > 1) {
      atomicMax(&sp.red_nl[i], v);
      for (int l = 1; l < v; ++l) atomicOr(&segmask[(l - 1) * kEgPairs + i], 1u << sg);
    }
    atomicAdd(&sp.red_sum[i], pp[1]);
  }
  __syncthreads();
  int nl = 1;
  for (int i = tid; i < n; i += NTH) {
    sp.tab[i] = a.tab + (size_t)sp.pair[i] * a.tab_bytes;
    sp.asum[i] = sp.red_sum[i];
    nl = sp.red_nl[i] > nl ? sp.red_nl[i] : nl;
  }
  if (nl > 1) atomicMax(&sp.nl, nl);
  __syncthreads();
  // LDS row r of tile t: row rb0 + t BR + r
  const uint8_t* w0 = a.w0 + (size_t)e * a.rows * a.rb;
  const int nlt = sp.nl;
  // half the tiles and one more ring stage (DH) when they fit the same LDS
  // (as in gate/up)
  constexpr int NTM = NTW > 1 ? NTW / 2 : 1;
  constexpr int DH = EgCfg<Q4, RG, NTM, D + 1, NW>::BYTES <= C::BYTES && C::NP > 128 ? D + 1 : D;
  auto wrow = [&](int r) { return w0 + (size_t)min(rb0 + r, a.rows - 1) * a.rb; };
  if (nlt == 1 && (DH == D || n > EgCfg<Q4, RG, NTM, DH, NW>::NP)) {
    auto epi = [&](int t, v16i (&acc)[2][NTW]) {
      v16u dots[2][NTW];
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int q = 0; q < NTW; ++q) dots[m][q] = __builtin_bit_cast(v16u, acc[m][q]);
      down_epi<Q4, RG, C::PG, NTW>(a, sp, dots, 0, n, rb0 + t * BR, sd + t * BR);
    };
    eg_rows<Q4, RG, NTW, D, NW>(wrow, a.K, sp, n, R, (size_t)BR * a.rb, lds, epi);
  } else if (nlt == 1) {
    auto epi = [&](int t, v16i (&acc)[2][NTM]) {
      v16u dots[2][NTM];
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int q = 0; q < NTM; ++q) dots[m][q] = __builtin_bit_cast(v16u, acc[m][q]);
      down_epi<Q4, RG, C::PG, NTM>(a, sp, dots, 0, n, rb0 + t * BR, sd + t * BR);
    };
    eg_rows<Q4, RG, NTM, DH, NW>(wrow, a.K, sp, n, R, (size_t)BR * a.rb, lds, epi);
  } else {
    constexpr int NPM = EgCfg<Q4, RG, NTM, DH, NW>::NP;
    v16u dots[2][NTM];
    for (int t = 0; t < R; ++t) {
      const int rb = rb0 + t * BR;
      auto wrow_t = [&](int r) { return w0 + (size_t)min(rb + r, a.rows - 1) * a.rb; };
      for (int pb = 0; pb < n; pb += NPM) {
        eg_dots<Q4, RG, NTM, DH, NW>(wrow_t, a.K, sp, pb, n, nlt, segmask, lds, dots);
        down_epi<Q4, RG, C::PG, NTM>(a, sp, dots, pb, n, rb, sd + t * BR);
      }
    }
  }
}

template <class Kern>
moe_status eg_lds_attr(Kern* fn, size_t lds, const char* what) {
  static_assert(sizeof(Kern*) > 0, "");
  return check_hip(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
                   what);
}

// Shapes per tile count (gate/up h-rows x pairs per task): NT = 1 (few
// pairs per expert): 128 x 32, 3 stages, two blocks per CU; NT = 2: 64 x
// 64, 4 stages, two blocks per CU; NT = 4: 128 x 256 in eight waves (four
// tiles each, those past the task's pairs skipped), 3 stages, one block per
// CU: one task per expert up to 256 pairs, so that an expert's weights
// are read once even when its pairs outnumber one pass of 128.  RTPB: row
// tiles of down per block (measured: 1 and 2 alike for NT = 1, 4 best for
// NT = 2, 2 best for NT = 4).
template <bool Q4, int RG, int NTW, int D, int NW, int RTPB>
moe_status launch_eg_shape(const LayerDev* L, int ntask, hipStream_t s) {
  static_assert(RTPB >= 1 && RTPB <= kDownRowTiles, "down row tiles per block");
  using C = EgCfg<Q4, RG, NTW, D, NW>;
  static bool attr = false;
  if (!attr && C::BYTES > 65536) {
    moe_status st = eg_lds_attr(gate_up_eg_kernel<Q4, RG, NTW, D, NW>, C::BYTES, "expert gate/up LDS attribute");
    if (!st) st = eg_lds_attr(down_eg_kernel<Q4, RG, NTW, D, NW>, C::BYTES, "expert down LDS attribute");
    if (st) return st;
    attr = true;
  }
  const unsigned tpad = (unsigned)((ntask + 7) / 8 * 8);
  const int nseg = (L->dff + 32 * RG - 1) / (32 * RG);
  EgArgs g{L->gq, L->uq, L->gs, L->us, L->rbg, L->dff, L->D, L->topk, L->perm, L->tasks, ntask,
           L->xtab, act_table_bytes(L->D), L->htab, act_table_bytes(L->dff), L->hpart, nseg,
           nullptr, nullptr, 1};
  hipLaunchKernelGGL((gate_up_eg_kernel<Q4, RG, NTW, D, NW>), dim3(tpad * (unsigned)nseg), dim3(64 * NW),
                     C::BYTES, s, g);
  moe_status st = check_hip(hipGetLastError(), "expert gate/up launch");
  if (st) return st;
  // down: row tiles per block (kDownRowTiles at most; one for a partial
  // last tile, whose rows the continued ring would overrun)
  const int nrt = (L->D + 64 * RG - 1) / (64 * RG);
  const int rtpb = L->D % (64 * RG) == 0 ? min(RTPB, nrt) : 1;
  EgArgs d{L->dq, nullptr, L->ds, nullptr, L->rbd, L->D, L->dff, L->topk, L->perm, L->tasks, ntask,
           L->htab, act_table_bytes(L->dff), nullptr, 0, L->hpart, nseg, L->y, L->y16, rtpb};
  hipLaunchKernelGGL((down_eg_kernel<Q4, RG, NTW, D, NW>),
                     dim3(tpad * (unsigned)((nrt + rtpb - 1) / rtpb)), dim3(64 * NW), C::BYTES, s, d);
  return check_hip(hipGetLastError(), "expert down launch");
}

template <bool Q4>
moe_status launch_eg(const LayerDev* L, int nt, int ntask, hipStream_t s) {
  switch (nt) {
    case 1: return launch_eg_shape<Q4, 4, 1, 3, 4, 2>(L, ntask, s);
    case 2: return launch_eg_shape<Q4, 2, 1, 4, 4, 4>(L, ntask, s);
    case 4: return launch_eg_shape<Q4, 4, 4, 3, 8, 2>(L, ntask, s);
    default: return set_error(MOE_ERR_ARG, "expert gemm: %d pair tiles", nt);
  }
}

}  // namespace

bool expert_gemm_ok(const LayerDev* L) {
  const int cols = L->dtype == 3 ? 128 : 64;
  // d_ff <= 2048: at most 32 gate/up segments of 64 rows (down's limb masks)
  return L->D % cols == 0 && L->dff % cols == 0 && L->dff <= 2048 && L->rbg % 16 == 0 &&
         L->rbd % 16 == 0;
}

int expert_gemm_tiles(const LayerDev* L, int T) {
  const int mean = T * L->topk / (L->E > 0 ? L->E : 1);
  return mean <= 24 ? 1 : (mean <= 64 ? 2 : 4);
}

int expert_gemm_split(int nt) { return nt == 4 ? 256 : 32 * nt; }

moe_status launch_expert_gemm(const LayerDev* L, int nt, int ntask, hipStream_t s) {
  return L->dtype == 3 ? launch_eg<true>(L, nt, ntask, s) : launch_eg<false>(L, nt, ntask, s);
}

}  // namespace moe
