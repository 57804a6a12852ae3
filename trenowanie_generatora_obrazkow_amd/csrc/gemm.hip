// Grouped bf16 GEMMs over ragged expert groups on gfx950 MFMA (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// One kernel template serves every grouped GEMM of the layer:
//   MGROUP  C[r, n] = sum_k A[r, k] B_e[k, n] for the sorted rows r of expert e (forward projections, dgrad,
//           the grouped_mm facade); the tiles are (m-tile of one expert, n-tile).
//   KGROUP  C_e[i, n] = sum_{r in e} X[r, i] Y[r, n] (weight gradients: the reduction runs over the expert's
//           ragged row range); the tiles are (expert, i-tile, n-tile).
// Both use a persistent grid: each workgroup walks tile ids blockIdx.x, +gridDim.x, ... up to a total computed on
// the device from `counts`, so no host readback and no per-expert launch; empty experts own no m-tiles (MGROUP) or
// produce zero tiles (KGROUP).  The block -> tile order is XCD-aware (the 8 XCDs get contiguous tile ranges) and
// groups GM m-tiles per band so A rows and B columns are reused from the XCD's L2.
//
// Data path: global memory -> LDS with global_load_lds_dwordx4 (no register staging) into an NSTAGE-deep ring of
// BK = 32 k-slices, one barrier per slice; fragments come out of LDS with ds_read_b128 for tiles stored k-contiguous
// and with ds_read_b64_tr_b16 (the gfx950 LDS transpose read) for tiles stored m/n-contiguous -- weights kept
// (K, N) with N contiguous, and both operands of a weight gradient -- so no operand is ever transposed in
// registers or in global memory.  Lanes whose source lies outside the operand (ragged expert ends, K / N tails)
// read a zero page instead, so every LDS slot is written each slice.
//
// MFMA roles: the N-side tile feeds the MFMA "A" operand and the M-side tile the "B" operand, so each lane's
// accumulator holds one output row and 4 consecutive output columns per group -> 8-byte bf16 / 16-byte fp32 stores.
#include "gemm_common.h"

#include <atomic>

namespace hmoe {

// byte offsets of a lane's four epilogue drain rows (-1: no row)
struct RowOffs {
  int64_t o[4];
};

// ----------------------------------------------------------------------------------------------------------------
// The kernel
// ----------------------------------------------------------------------------------------------------------------
// A_BLK: the A rows (MGROUP) come from the row-group tiles of the sorted rows (gemm_common.h), not from A's rows.
// F16: the 16-bit operands, row scales and outputs are fp16 (v_mfma_f32_32x32x16_f16) instead of bf16; forward
// epilogues (store, SwiGLU) only.
template <class C, int MODE, bool A_MN, bool B_MN, int EPI, bool A_BLK = false, bool F16 = false>
__global__ __launch_bounds__(C::NT, 1) void grouped_gemm_kernel(GemmParams p) {
  static_assert(!F16 || EPI == EPI_STORE || EPI == EPI_SWIGLU, "fp16: forward epilogues only");
  using X = Elt<F16>;
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  __shared__ int s_rstart[kMaxEGemm + 1];  // row starts (M < 2^31: checked on the host)
  __shared__ int s_tstart[kMaxEGemm + 1];  // MGROUP: prefix of ceil(count / BM); KGROUP: one m-tile per expert
  __shared__ int s_gstart[A_BLK ? kMaxEGemm + 1 : 1];  // A_BLK: prefix of ceil(count / 128) (row groups)
  // per-row epilogue inputs of the tile (scatter index, routing weight), double-buffered by tile parity: a wave
  // that has finished its epilogue may already fill the next tile's while others still read this one.  The copy
  // starts at the 16-byte boundary below row0 (up to 7 leading 2-byte elements) and writes whole 1 KB blocks: one
  // for 128-row tiles, two for 256-row tiles (whose rows reach past the first 1 KB).  The smaller buffers keep the
  // static LDS of the 128-row kernels low enough for two workgroups per CU.
  constexpr int RDW = C::BM > 128 ? 512 : 256;
  __shared__ __attribute__((aligned(16))) int s_rowy[2][RDW];
  __shared__ __attribute__((aligned(16))) float s_rowsc[2][RDW];
  // int8 weights: the tile's per-column weight scales (bf16 or fp32), by tile parity like the row data
  __shared__ __attribute__((aligned(16))) float s_colsc[2][256];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int E = p.E;

  // ---- per-expert row starts and tile starts (wave 0, lane-parallel scan) ----
  if (wave == 0) {
    const int per = (E + 63) / 64;
    int64_t rs = 0;
    int ts = 0, gs = 0;
    for (int i = 0; i < per; ++i) {
      const int e = lane * per + i;
      if (e < E) {
        int64_t c = read_count(p.counts, p.counts64, e);
        c = c < 0 ? 0 : (c > p.M ? p.M : c);  // garbage counts must not blow up the tile loop
        rs += c;
        ts += MODE == MGROUP ? (int)((c + C::BM - 1) / C::BM) : 1;
        if constexpr (A_BLK) gs += (int)((c + kTileGroupRows - 1) / kTileGroupRows);
      }
    }
    int64_t irs = rs;
    int its = ts, igs = gs;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
      const int64_t o = __shfl_up(irs, s, 64);
      const int ot = __shfl_up(its, s, 64);
      const int og = __shfl_up(igs, s, 64);
      if (lane >= s) {
        irs += o;
        its += ot;
        igs += og;
      }
    }
    int64_t r0 = irs - rs;
    int t0 = its - ts, g0 = igs - gs;
    for (int i = 0; i < per; ++i) {
      const int e = lane * per + i;
      if (e < E) {
        int64_t c = read_count(p.counts, p.counts64, e);
        c = c < 0 ? 0 : (c > p.M ? p.M : c);
        s_rstart[e] = (int)min(r0, p.M);  // (garbage counts can sum past M)
        s_tstart[e] = t0;
        r0 += c;
        t0 += MODE == MGROUP ? (int)((c + C::BM - 1) / C::BM) : 1;
        if constexpr (A_BLK) {
          s_gstart[e] = g0;
          g0 += (int)((c + kTileGroupRows - 1) / kTileGroupRows);
        }
      }
    }
    if (lane == 63) {
      s_rstart[E] = (int)min(irs, p.M);
      s_tstart[E] = its;
    }
  }
  lds_barrier();

  int nb_n;
  if (EPI == EPI_SWIGLU)
    nb_n = (p.N + C::BN / 2 - 1) / (C::BN / 2);
  else
    nb_n = (p.N + C::BN - 1) / C::BN;
  const int nb_i = MODE == KGROUP ? (p.P + C::BM - 1) / C::BM : 1;
  const int total_m = MODE == MGROUP ? s_tstart[E] : E * nb_i;
  const int total = total_m * nb_n;

  typename TileSel<A_MN, C::BM, C::NWAVES>::type ta;
  typename TileSel<B_MN, C::BN, C::NWAVES, C::BE, C::FN, F16>::type tb;
  // A wave's fragment f along a dimension covers 32 rows / columns from f * FS + 32 w: the lane part of the read
  // address is that of wave (w & 1) inside a 64-wide group, and 64 * (w >> 1) selects the group.
  static_assert(C::FSM % 64 == 0 && C::FSN % 64 == 0, "fragment reads work on 64-wide groups");
  const int loff_a = decltype(ta)::lane_off(wm & 1, lane);
  const int loff_b = decltype(tb)::lane_off(wn & 1, lane);
  const int wgrp_a = 64 * (wm >> 1), wgrp_b = 64 * (wn >> 1);

  // XCD-aware slot: consecutive workgroup ids are dealt round-robin over the 8 XCDs; give each XCD a contiguous
  // range of tile ids so the tiles it runs share A rows and B columns in its L2.
  const int G = gridDim.x;
  int slot = blockIdx.x;
  if ((G & 7) == 0) slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);

  // Work units.  Every workgroup takes units slot, slot + G, ...; when the tiles leave a final round at most half
  // full (MGROUP), each tile of that round becomes two units of BM/2 rows, so the round takes about half a tile's
  // time instead of a whole one (the half-row units run the main loop on their live fragment rows only).
  const int full_units = total / G * G;
  const int rem = total - full_units;
  const bool split_last = MODE == MGROUP && rem > 0 && 2 * rem <= G;
  const int units = split_last ? full_units + 2 * rem : total;

  int tile_iter = 0;
  for (int unit = slot; unit < units; unit += G, ++tile_iter) {
    int tile = unit, half = -1;  // half >= 0: rows [half * BM/2, (half + 1) * BM/2) of the tile
    if (unit >= full_units && split_last) {
      tile = full_units + (unit - full_units) % rem;
      half = (unit - full_units) / rem;
    }
    // ---- tile decode ----
    int mt, nb;
    {
      const int per_group = C::GM * nb_n;  // bands of GM m-tiles x all n-tiles
      // Band residency.  With the XCD-aware slots, XCD x runs tiles [r G + x G/8, r G + (x+1) G/8) in round r: one
      // block of G/8 tiles of a band.  In plain band order an XCD moves on to other bands every round and its L2
      // fetches new A rows each time.  Within every complete super-group of 8 bands the blocks are permuted so that
      // XCD x keeps band 8 s + x for per_group / (G/8) rounds in a row and walks its n-blocks, which keeps the band's
      // A rows in its L2.  Only the order in which workgroups take tiles changes, not what a tile computes.  (Not for
      // the weight gradients: their bands' A columns, 4 MB at the C5 shape, do not stay in a 4 MB L2, and the order
      // measured slower there.)
      if (MODE == MGROUP && (G & 7) == 0) {
        const int XB = G >> 3;
        if (per_group % XB == 0) {
          const int BPB = per_group / XB, SG = 8 * BPB;  // blocks per band, per super-group
          const int j = tile / XB, sg = j / SG, jj = j - sg * SG;
          if ((sg + 1) * SG * XB <= full_units) tile = (sg * SG + (jj & 7) * BPB + (jj >> 3)) * XB + tile % XB;
        }
      }
      const int g = tile / per_group;
      const int first = g * C::GM;
      const int gsz = min(total_m - first, C::GM);
      const int local = tile - g * per_group;
      mt = first + local % gsz;
      nb = local / gsz;
    }
    int e;
    int64_t row0 = 0, row_end = 0;  // MGROUP: sorted rows [row0, row_end) of this m-tile's expert
    int i0 = 0;                     // KGROUP: first output row
    int64_t kstart = 0;
    int kvalid = p.K;
    if (MODE == MGROUP) {
      int lo = 0, hi = E;  // largest e with s_tstart[e] <= mt (empty experts share the start of the next)
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (s_tstart[mid] <= mt)
          lo = mid;
        else
          hi = mid;
      }
      e = lo;
      row0 = s_rstart[e] + (int64_t)(mt - s_tstart[e]) * C::BM;
      row_end = min((int64_t)s_rstart[e + 1], p.M);
      if (half >= 0) {
        row0 += half * (C::BM / 2);
        row_end = min(row_end, row0 + C::BM / 2);
        if (row0 >= row_end) {  // no rows in this half (uniform over the workgroup): nothing to do, and the
          --tile_iter;          // LDS buffer parity of the next unit must still alternate with the previous one's
          continue;
        }
      }
    } else {
      e = mt / nb_i;
      i0 = (mt - e * nb_i) * C::BM;
      kstart = s_rstart[e];
      const int64_t kend = min((int64_t)s_rstart[e + 1], p.M);
      kvalid = (int)max((int64_t)0, kend - kstart);
    }
    const int n0 = nb * (EPI == EPI_SWIGLU ? C::BN / 2 : C::BN);

    // ---- copy sources for this tile (buffer bases and per-lane byte offsets) ----
    if constexpr (MODE == MGROUP) {
      static_assert(!A_MN, "MGROUP A is K-contiguous");
      ta.K = p.K;
      if constexpr (A_BLK) {
        // row-group tiles: instruction I's 16 rows (tile rows 16 I ..) are one 1 KB run of their group's slice
        ta.kmul = kTileSliceBytes / kBK;
        ta.rsrc = make_rsrc(p.A);
        const int64_t nsl = (p.K + kBK - 1) / kBK;
        const int64_t rel0 = row0 - s_rstart[e];  // tile start within the expert (a multiple of 64)
#pragma unroll
        for (int i = 0; i < ta.PER_WAVE; ++i) {
          const int rr = ta.row_of(wave, lane, i);
          const int64_t rel = rel0 + 16 * (wave * ta.PER_WAVE + i);  // the instruction's first row in the expert
          const int64_t g = s_gstart[e] + rel / kTileGroupRows;
          ta.voff[i] = row0 + rr < row_end
                           ? (uint32_t)(g * nsl * kTileSliceBytes + (rel % kTileGroupRows) * 64 + lane * 16)
                           : kOOB;
          ta.chunk[i] = (lane & 3) ^ swz_k(rr);
        }
      } else {
        // gathered rows are addressed from A itself; contiguous rows from the tile's first row
        ta.rsrc = make_rsrc(p.a_idx ? p.A : p.A + row0 * p.lda);
#pragma unroll
        for (int i = 0; i < ta.PER_WAVE; ++i) {
          const int rr = ta.row_of(wave, lane, i);
          const int64_t r = row0 + rr;
          const int c = (lane & 3) ^ swz_k(rr);
          uint32_t vo = kOOB;
          if (r < row_end) {
            const int64_t src = p.a_idx ? (int64_t)p.a_idx[r] : (int64_t)rr;
            vo = (uint32_t)(src * p.lda * 2 + c * 16);
          }
          ta.voff[i] = vo;
          ta.chunk[i] = c;
        }
      }
      tb.rsrc = make_rsrc(static_cast<const char*>(p.B) + (int64_t)e * p.strideBe * C::BE);
      auto gcol = [&](int nn, int& col) -> bool {  // tile column -> weight column
        if (EPI == EPI_SWIGLU) {
          const int half = nn / (C::BN / 2);  // tile columns [0, BN/2) gate, [BN/2, BN) the matching up
          const int ac = n0 + nn % (C::BN / 2);
          col = half * p.h + ac;
          return ac < p.N;
        } else {
          col = n0 + nn;
          return col < p.N;
        }
      };
      if constexpr (B_MN) {
        tb.kstep = (uint32_t)(p.ldb * C::BE);
        tb.Kvalid = p.K;
#pragma unroll
        for (int i = 0; i < tb.PER_WAVE; ++i) {
          int k, nn, col;
          tb.slot(wave, lane, i, k, nn);
          tb.krow[i] = k;
          tb.voff[i] = gcol(nn, col) ? (uint32_t)(((int64_t)k * p.ldb + col) * C::BE) : kOOB;
        }
      } else {
        static_assert(C::BE == 2, "int8 weights are read N-contiguous only");
        tb.K = p.K;
#pragma unroll
        for (int i = 0; i < tb.PER_WAVE; ++i) {
          const int nn = tb.row_of(wave, lane, i);
          const int c = (lane & 3) ^ swz_k(nn);
          int col;
          tb.voff[i] = gcol(nn, col) ? (uint32_t)((int64_t)col * p.ldb * 2 + c * 16) : kOOB;
          tb.chunk[i] = c;
        }
      }
    } else {
      static_assert(A_MN && B_MN, "KGROUP operands are MN-contiguous");
      ta.rsrc = make_rsrc(p.A + kstart * p.lda + i0);
      ta.kstep = (uint32_t)(p.lda * 2);
      ta.Kvalid = kvalid;
      static_assert(C::BE == 2, "weight gradients take bf16 operands");
      tb.rsrc = make_rsrc(static_cast<const uint16_t*>(p.B) + kstart * p.ldb + n0);
      tb.kstep = (uint32_t)(p.ldb * 2);
      tb.Kvalid = kvalid;
#pragma unroll
      for (int i = 0; i < ta.PER_WAVE; ++i) {
        int k, ic;
        ta.slot(wave, lane, i, k, ic);
        ta.krow[i] = k;
        ta.voff[i] = (i0 + ic < p.P) ? (uint32_t)(((int64_t)k * p.lda + ic) * 2) : kOOB;
      }
#pragma unroll
      for (int i = 0; i < tb.PER_WAVE; ++i) {
        int k, nc;
        tb.slot(wave, lane, i, k, nc);
        tb.krow[i] = k;
        tb.voff[i] = (n0 + nc < p.N) ? (uint32_t)(((int64_t)k * p.ldb + nc) * 2) : kOOB;
      }
    }

    // ---- per-row epilogue inputs: copied into LDS by wave 0 with the same direct loads as the operand tiles,
    // ahead of the first slice, so they are complete when slice 0 is and no compiler-visible load stays pending ----
    const int par = tile_iter & 1;
    constexpr bool ROWDATA = MODE == MGROUP && (EPI == EPI_STORE || EPI == EPI_STORE_F32 || EPI == EPI_SWIGLU_BWD);
    static_assert(!ROWDATA || C::BM <= 256, "row data buffers hold 256 rows");
    // The copies start at the 16-byte boundary at or below row0 (the direct loads move aligned 16-byte chunks); a
    // 256-row tile takes two instructions (1 KB + 16 bytes of data) so that its shifted rows are always covered.
    [[maybe_unused]] int y_sh = 0, sc_sh = 0;  // leading rows in front of row0
    if constexpr (ROWDATA) {
      auto copy_rows = [&](const void* arr, int esz, char* dst) -> int {
        const uintptr_t first = reinterpret_cast<uintptr_t>(arr) + (uintptr_t)row0 * esz;
        const uintptr_t base = first & ~(uintptr_t)15;
        const int sh = (int)(first - base) / esz;
        // valid bytes from the aligned base, rounded up to the 16-byte chunk: the range check zeroes every dword
        // that reaches past the range, so an unrounded end would drop a last 2-byte element in the dword's low half
        // (the chunk never crosses a page, so reading its tail is safe)
        const int64_t bytes = ((p.M - row0) * esz + (int64_t)(first - base) + 15) & ~(int64_t)15;
        if (wave == 0) {
          i32x4 rs = make_rsrc(reinterpret_cast<const void*>(base));
          rs.z = __builtin_amdgcn_readfirstlane((int)min(bytes, (int64_t)0x7FFFFFF0));
          buf2lds((uint32_t)lane * 16u, rs, 0u, dst);
          if constexpr (C::BM > 128) buf2lds(lane == 0 ? 1024u : kOOB, rs, 0u, dst + 1024);
        }
        return sh;
      };
      if (EPI != EPI_SWIGLU_BWD && p.y_idx) y_sh = copy_rows(p.y_idx, 4, reinterpret_cast<char*>(s_rowy[par]));
      if (p.scale) sc_sh = copy_rows(p.scale, p.scale_f32 ? 4 : 2, reinterpret_cast<char*>(s_rowsc[par]));
    }
    // int8 weights: the tile's column scales (w_scale[e][column], in tile-column order) by wave 1 (wave 0 with one
    // wave), ahead of the first slice like the row data
    if constexpr (C::BE == 1) {
      if (wave == (C::NWAVES > 1 ? 1 : 0)) {
        const int es = p.w_scale_f32 ? 4 : 2;
        const int per = 16 / es;  // columns per 16-byte copy
        i32x4 rs = make_rsrc(static_cast<const char*>(p.w_scale) + (int64_t)e * p.ldws * es);
        rs.z = __builtin_amdgcn_readfirstlane((int)min(p.ldws * es, (int64_t)0x7FFFFFF0));
        const int tc = lane * per;  // tile column of this lane's first scale
        int col = 0;
        bool ok = tc < C::BN;
        if (EPI == EPI_SWIGLU) {
          const int ac = n0 + tc % (C::BN / 2);
          col = (tc / (C::BN / 2)) * p.h + ac;
          ok = ok && ac < p.N;
        } else {
          col = n0 + tc;
          ok = ok && col < p.N;
        }
        buf2lds(ok ? (uint32_t)(col * es) : kOOB, rs, 0u, reinterpret_cast<char*>(s_colsc[par]));
      }
    }

    const int nk = (kvalid + kBK - 1) / kBK;  // k-slices of this tile

    // ---- epilogue staging (defined here: the SwiGLU backward starts loading its first pass inside the loop) ----
    // The sub-planes live in the ring bytes this wave's own direct loads fill (its A and B parts of each stage),
    // which no other wave writes.  Chunk q is part q & 1 of stage q >> 1 (bf16 weights; int8: the A part of stage
    // q), the stage rotated by srot: the SwiGLU backward's first staging buffer (stages srot, srot + 1) is then the
    // pair of stages whose slices (nk - 4, nk - 3) every wave has read by the barrier of iteration nk - 2.
    const int lrow = lane & 31;
    const int lcol = 4 * (lane >> 5);
    constexpr int CH = C::A_BYTES / C::NWAVES;  // bytes per ring part filled by one wave
    static_assert(CH >= 1024 && 4096 % CH == 0 && (C::BE == 1 || C::A_BYTES == C::B_BYTES), "staging chunks");
    const int srot = EPI == EPI_SWIGLU_BWD ? (nk & (kNStage - 1)) : 0;
    auto chunk = [&](int q) -> char* {
      if constexpr (C::BE == 1) return smem + q * C::STAGE_BYTES + wave * CH;
      return smem + (((q >> 1) + srot) & (kNStage - 1)) * C::STAGE_BYTES + (q & 1) * C::A_BYTES + wave * CH;
    };
    // sub-plane sp, row r (0..31), byte offset within the 128-byte row; 16-byte chunks XOR-swizzled by r & 7
    auto sp_addr = [&](int sp, int r, int byte) -> char* {
      const int lin = r * 128;
      return chunk(sp * (4096 / CH) + lin / CH) + lin % CH + ((((byte >> 4) ^ r) & 7) << 4) + (byte & 15);
    };
    // SwiGLU backward: pass pa's forward [g | u] rows into staging buffer pa & 1 (g in sub-planes
    // [2 (pa & 1) NSP, (2 (pa & 1) + 1) NSP), u in the next NSP) with direct loads: instruction (array, sp, i) fills
    // rows 8i..8i+7 of a sub-plane, lane l row 8i + l/8, physical chunk l%8 = logical chunk (l%8) ^ (l/8).  The
    // descriptor starts at the pass's first row and its range ends at the expert's last row, so rows past it read
    // zeros; a lane's columns past N use an out-of-range offset; the row and array parts of each address are
    // uniform (the scalar offset), so a lane holds one offset per sub-plane.
    constexpr int GU_RB = C::FN * 32 * 2, GU_NSP = (GU_RB + 127) / 128;
    [[maybe_unused]] auto issue_gu = [&](int pa) {
      const int rb = pa * C::FSM + wm * 32;
      const int64_t prow = row0 + rb;
      i32x4 rs = make_rsrc(p.gu_in + prow * (int64_t)(2 * p.h));
      const int64_t live = row_end > prow ? (row_end - prow) * (int64_t)(2 * p.h) * 2 : 0;
      rs.z = __builtin_amdgcn_readfirstlane((int)min(live, (int64_t)0x7FFFFFF0));
      const int rl = lane >> 3, cl = (lane & 7) ^ rl;
#pragma unroll
      for (int sp = 0; sp < GU_NSP; ++sp) {
        const int cw = sp * 64 + 8 * cl;  // column within the wave's FN*32
        const int tc = (cw / 32) * C::FSN + wn * 32 + cw % 32;
        const bool ok = n0 + tc < p.N && sp * 128 + cl * 16 < GU_RB;
        const uint32_t vo = ok ? (uint32_t)((rl * (2 * p.h) + n0 + tc) * 2) : kOOB;
#pragma unroll
        for (int arr = 0; arr < 2; ++arr)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            buf2lds(vo, rs, (uint32_t)((8 * i * (2 * p.h) + arr * p.h) * 2),
                    sp_addr((2 * (pa & 1) + arr) * GU_NSP + sp, 8 * i, 0));
      }
    };
    // SwiGLU backward: pass 0's rows are loaded from the barrier of iteration nk - 2 on (nk >= 2)
    const bool gu_early = EPI == EPI_SWIGLU_BWD && nk >= 2;

    // ---- main loop: NSTAGE-deep ring of k-slices ----
    f32x16 acc[C::FM][C::FN];
#pragma unroll
    for (int a = 0; a < C::FM; ++a)
#pragma unroll
      for (int b = 0; b < C::FN; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    constexpr int LOADS = decltype(ta)::PER_WAVE + decltype(tb)::PER_WAVE;  // direct loads per thread per slice
    char* const ring_end = smem + C::LDS_BYTES;
    char* fill = smem;        // next ring slot to fill
    const char* cons = smem;  // ring slot consumed by the current slice
    auto issue = [&](int kslice) {
      ta.issue(fill, wave, lane, kslice * kBK);
      tb.issue(fill + C::A_BYTES, wave, lane, kslice * kBK);
      fill += C::STAGE_BYTES;
      if (fill == ring_end) fill = smem;
    };
    // Fragment-level software pipeline over the ring (two k16 steps per slice):
    //   iteration kt:  read ks1 fragments of slice kt      | MFMAs on ks0 fragments of slice kt
    //                  wait for slice kt+1, barrier, refill the slot of slice kt with slice kt+4
    //                  read ks0 fragments of slice kt+1    | MFMAs on ks1 fragments of slice kt
    // The barrier comes after every wave has read all of slice kt, so its slot can be refilled at once: four
    // slices are in flight while one is consumed, and LDS read latency hides under the MFMAs.
    // FE = fragment rows (of FM) that hold tile rows: a partial m-tile (an expert's last rows) with at most 64 or 128
    // rows runs the loop with FE = 1 or 2, skipping the MFMAs and fragment reads of the empty rows (its copies are
    // unchanged, so the wait counts hold); the accumulators of the other rows stay zero and are not stored.  Such a
    // tile takes about FE/FM of a full tile's time.
    typedef typename TileSel<A_MN, C::BM, C::NWAVES>::type TA;
    typedef typename TileSel<B_MN, C::BN, C::NWAVES, C::BE, C::FN, F16>::type TB;
    struct Frags {
      bf16x8 xa[C::FM], wb[C::FN];
    };
    static_assert(kNStage == 4 && kBK == 32, "pipeline written for a 4-deep ring of two-step slices");
    // NL = live B fragments: all FN, or, for a SwiGLU n-tile whose gate (and up) columns fill at most half of
    // their 128, the first fragment of each half (the other half's columns are past N: their copies are zeros).
    auto main_loop = [&](auto fe_tag, auto nl_tag) {
      constexpr int FE = decltype(fe_tag)::value;
      constexpr int NL = decltype(nl_tag)::value;
      static_assert(NL == C::FN || (NL == 2 && C::FN == 4), "live B fragments: all, or one per SwiGLU half");
      auto bf = [](int j) { return NL == C::FN ? j : j * (C::FN / 2); };  // fragment of live fragment j
      constexpr int RD = FE * (A_MN ? 2 : 1) + NL * (B_MN ? 2 : 1);  // LDS reads per k16 step
      constexpr int NMF = FE * NL;                                     // MFMAs per k16 step
      constexpr int PAIRS = RD < NMF ? RD : NMF;
      auto read = [&](const char* slot, int ks) {
        Frags f;
#pragma unroll
        for (int a = 0; a < FE; ++a) f.xa[a] = TA::frag(slot, a * C::FSM + wgrp_a, loff_a, ks);
#pragma unroll
        for (int j = 0; j < NL; ++j)
          f.wb[bf(j)] = TB::frag(slot + C::A_BYTES, bf(j) * C::FSN + wgrp_b, loff_b, ks);
        return f;
      };
      auto mfmas = [&](const Frags f) {
#pragma unroll
        for (int a = 0; a < FE; ++a)
#pragma unroll
          for (int j = 0; j < NL; ++j)
            acc[a][bf(j)] = mfma16<F16>(f.wb[bf(j)], f.xa[a], acc[a][bf(j)]);
      };
      // one LDS read after each MFMA while both last, then whichever is left
      auto interleave = [&]() {
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
        }
        if constexpr (NMF > PAIRS) __builtin_amdgcn_sched_group_barrier(0x008, NMF - PAIRS, 0);
        if constexpr (RD > PAIRS) __builtin_amdgcn_sched_group_barrier(0x100, RD - PAIRS, 0);
      };
#pragma unroll
      for (int s = 0; s < kNStage; ++s)
        if (s < nk) issue(s);
      Frags f0 = {}, f1 = {};
      if (nk > 0) {
        const int ahead = min(nk - 1, kNStage - 1);  // slices issued after slice 0
        if (ahead >= 3)
          wait_vm<3 * LOADS>();
        else if (ahead == 2)
          wait_vm<2 * LOADS>();
        else if (ahead == 1)
          wait_vm<LOADS>();
        else
          wait_vm<0>();
        lds_barrier();
        f0 = read(cons, 0);
      }
      // The two MFMA blocks are unconditional (a conditional copy would split the accumulators' live ranges); on
      // the last slice the ks0 read of the "next" slot reads stale LDS that is never used.
      // FAST iterations (all but the last kNStage, and not the one that refills a partial last slice) refill a
      // whole slice with two slices issued after slice kt+1: no per-copy tail test, no refill test and no
      // wait-count selection inside the MFMA stream.
      auto iter = [&](int kt, auto fast_tag) {
        constexpr bool FAST = decltype(fast_tag)::value;
        f1 = read(cons, 1);
        mfmas(f0);
        interleave();
        // every MFMA of this half stays ahead of the wait and barrier below: the trailing ones then run while the
        // last fragment reads complete (the barrier waits for those reads)
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (FAST) {
          wait_vm<2 * LOADS>();
        } else {
          const int ahead = min(nk - 1, kt + kNStage - 1) - (kt + 1);  // slices issued after slice kt+1
          if (ahead >= 2)
            wait_vm<2 * LOADS>();
          else if (ahead == 1)
            wait_vm<LOADS>();
          else if (!gu_early || kt + 1 < nk)  // the last iteration has no next slice to wait for: pass 0's [g | u]
            wait_vm<0>();                      // stay in flight
        }
        lds_barrier();
        if constexpr (EPI == EPI_SWIGLU_BWD) {
          if (kt == nk - 2) issue_gu(0);  // slices nk - 4 and nk - 3 have been read by every wave
        }
        // Second half: MFMAs on the ks1 fragments, the next slice's ks0 fragment reads and the refill of slice
        // kt's slot with slice kt+4 (fill == cons here), one step per MFMA so the reads and copies issue in its
        // shadow (in both modes: the weight gradients measured 6% faster than with the copies issued together).
        const bool refill = FAST || kt + kNStage < nk;
        const int kr = (kt + kNStage) * kBK;
        char* const dst = fill;
        cons += C::STAGE_BYTES;
        if (cons == ring_end) cons = smem;
        if (refill) {
          fill += C::STAGE_BYTES;
          if (fill == ring_end) fill = smem;
        }
        auto copy = [&](int l) {  // copy number l: A's first, then B's
          if constexpr (FAST) {
            if (l < TA::PER_WAVE)
              ta.issue_one_full(dst, wave, l, kr);
            else if (l < LOADS)
              tb.issue_one_full(dst + C::A_BYTES, wave, l - TA::PER_WAVE, kr);
          } else {
            if (l < TA::PER_WAVE)
              ta.issue_one(dst, wave, l, kr);
            else if (l < LOADS)
              tb.issue_one(dst + C::A_BYTES, wave, l - TA::PER_WAVE, kr);
          }
        };
#pragma unroll
        for (int a = 0; a < FE; ++a)
#pragma unroll
          for (int j = 0; j < NL; ++j) {
            const int i = a * NL + j, b = bf(j);
            acc[a][b] = mfma16<F16>(f1.wb[b], f1.xa[a], acc[a][b]);
            if (i < FE)
              f0.xa[i] = TA::frag(cons, i * C::FSM + wgrp_a, loff_a, 0);
            else if (i < FE + NL)
              f0.wb[bf(i - FE)] = TB::frag(cons + C::A_BYTES, bf(i - FE) * C::FSN + wgrp_b, loff_b, 0);
            if ((i & 1) && refill) copy(i >> 1);
            __builtin_amdgcn_sched_barrier(0);
          }
        // fragment reads and copies left over when there are fewer MFMAs than reads or copy pairs
#pragma unroll
        for (int i = FE * NL; i < FE + NL; ++i) {
          if (i < FE)
            f0.xa[i] = TA::frag(cons, i * C::FSM + wgrp_a, loff_a, 0);
          else
            f0.wb[bf(i - FE)] = TB::frag(cons + C::A_BYTES, bf(i - FE) * C::FSN + wgrp_b, loff_b, 0);
        }
#pragma unroll
        for (int l = FE * NL / 2; l < LOADS; ++l) {
          if (!refill) break;
          copy(l);
        }
      };
      // iterations whose refill slice kt + kNStage is whole: (kt + kNStage + 1) * kBK <= kvalid
      const int nfast = max(0, min(nk - kNStage, kvalid / kBK - kNStage));
      int kt = 0;
      for (; kt < nfast; ++kt) iter(kt, std::true_type{});
      for (; kt < nk; ++kt) iter(kt, std::false_type{});
    };
    // a SwiGLU n-tile whose gate columns end within the first 64 of its 128 (e.g. the last n-tile at h = 320)
    // runs with the live B fragments only
    constexpr bool NHALF = EPI == EPI_SWIGLU && C::FN == 4;
    auto run_loop = [&](auto fe_tag) {
      if constexpr (NHALF) {
        if (p.N - n0 <= C::BN / 4) {
          main_loop(fe_tag, std::integral_constant<int, 2>{});
          return;
        }
      }
      main_loop(fe_tag, std::integral_constant<int, C::FN>{});
    };
    if constexpr (MODE == MGROUP) {
      const int64_t rows = row_end - row0;
      if (C::FM >= 4 && rows <= C::FSM)
        run_loop(std::integral_constant<int, 1>{});
      else if (C::FM >= 4 && rows <= 2 * C::FSM)
        run_loop(std::integral_constant<int, 2>{});
      else
        run_loop(std::integral_constant<int, C::FM>{});
    } else {
      run_loop(std::integral_constant<int, C::FM>{});
    }
    // fragment rows holding tile rows (the epilogue passes to run)
    const int fe_rows = MODE == MGROUP ? (int)min((row_end - row0 + C::FSM - 1) / C::FSM, (int64_t)C::FM) : C::FM;
    lds_barrier();  // every wave is done with the ring before the next tile refills it
    // The epilogue's pin_agpr() hides the last MFMA write from the compiler's hazard tracking, so the wait states a
    // VALU read of an MFMA result needs (19 for a 16-pass MFMA; the 32x32x16 bf16 MFMA has 8 passes) are given here.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

    // ---- epilogue: per-wave staging in LDS, then row-contiguous 16-byte stores ----
    // Lane l of wave (wm, wn) holds, for fragment (a, b) and group g, output row a*FSM + wm*32 + l%32 and the 4
    // consecutive columns b*FSN + wn*32 + 8g + 4*(l/32) + 0..3 (acc[a][b][4g + 0..3]).  Pass a converts the wave's
    // 32 rows and parks them in "sub-planes" of 32 rows x 128 bytes, then reads them back row-contiguously: 8 lanes
    // per 128-byte row, each storing 16 bytes, so a store instruction writes 64-byte segments instead of scattered
    // 8-byte pieces.  The sub-planes live in the ring bytes this wave's own direct loads fill (its A and B parts of
    // each stage), which no other wave writes: the epilogue needs no barrier, and the wave's next-tile loads are
    // issued after its last read in program order.
    // the 4 column scales of int8 weights from tile column tc: fp32 (scf_tag true) or bf16 values
    [[maybe_unused]] auto col_scale4 = [&](auto scf_tag, int tc, float* ws) {
      if constexpr (decltype(scf_tag)::value) {
        const float4 v = *reinterpret_cast<const float4*>(&s_colsc[par][tc]);
        ws[0] = v.x; ws[1] = v.y; ws[2] = v.z; ws[3] = v.w;
      } else {
        const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(s_colsc[par]) + tc);
        ws[0] = bf_lo(v.x); ws[1] = bf_hi(v.x); ws[2] = bf_lo(v.y); ws[3] = bf_hi(v.y);
      }
    };
    // park the 4 values of fragment (a, b), group g (rows lrow) into a bf16 / fp32 array starting at sub-plane sp0
    auto park_bf16 = [&](int sp0, int b, int g, uint32_t lo, uint32_t hi) {
      const int byte = (b * 32 + 8 * g + lcol) * 2;
      *reinterpret_cast<uint2*>(sp_addr(sp0 + byte / 128, lrow, byte % 128)) = make_uint2(lo, hi);
    };
    [[maybe_unused]] auto park_f32 = [&](int sp0, int b, int g, float4 v) {
      const int byte = (b * 32 + 8 * g + lcol) * 4;
      *reinterpret_cast<float4*>(sp_addr(sp0 + byte / 128, lrow, byte % 128)) = v;
    };
    // Read back NSPX sub-planes from sp0 (an array of rowbytes bytes per row, es bytes per element) and store them.
    // Lane l holds the 16-byte piece l % 8 of every sub-plane in the wave's rows 8 j + l / 8 (j = 0..3); rows.o[j]
    // is the byte offset from base of its row j's column 0, or -1 for a row past the tile's rows, and a piece goes
    // to base + rows.o[j] + (n0 + tile column) * es when that column is below ncols.  The reads of two sub-planes
    // are issued before their stores, so a pass waits for LDS once per sub-plane pair, not once per store.
    // PAIRED false: each piece's read just ahead of its store instead (what the bf16 forward epilogues measured
    // fastest, by 1%)
    auto drain_rows = [&](auto nsp_tag, int sp0, int rowbytes, int es, char* base, const RowOffs rows, int ncols,
                          auto paired_tag) {
      constexpr int NSPX = decltype(nsp_tag)::value;
      constexpr bool PAIRED = decltype(paired_tag)::value;
      const int c = lane & 7;
      auto read4 = [&](int sp, uint4* v) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[j] = *reinterpret_cast<const uint4*>(sp_addr(sp0 + sp, 8 * j + (lane >> 3), c * 16));
      };
      auto store4 = [&](int sp, const uint4* v) {
        const int cw = (sp * 128 + c * 16) / es;  // column within the wave's FN*32
        const int n = n0 + (cw / 32) * C::FSN + wn * 32 + cw % 32;
        const bool cok = sp * 128 + c * 16 < rowbytes && n < ncols;  // a narrow array fills part of a sub-plane
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (cok && rows.o[j] >= 0) *reinterpret_cast<uint4*>(base + rows.o[j] + (int64_t)n * es) = v[j];
      };
      if constexpr (PAIRED) {
#pragma unroll
        for (int sp = 0; sp + 1 < NSPX; sp += 2) {
          uint4 va[4], vb[4];
          read4(sp, va);
          read4(sp + 1, vb);
          store4(sp, va);
          store4(sp + 1, vb);
        }
        if constexpr (NSPX & 1) {
          uint4 va[4];
          read4(NSPX - 1, va);
          store4(NSPX - 1, va);
        }
      } else {
#pragma unroll
        for (int sp = 0; sp < NSPX; ++sp) {
          const int cw = (sp * 128 + c * 16) / es;
          const int n = n0 + (cw / 32) * C::FSN + wn * 32 + cw % 32;
          const bool cok = sp * 128 + c * 16 < rowbytes && n < ncols;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint4 v = *reinterpret_cast<const uint4*>(sp_addr(sp0 + sp, 8 * j + (lane >> 3), c * 16));
            if (cok && rows.o[j] >= 0) *reinterpret_cast<uint4*>(base + rows.o[j] + (int64_t)n * es) = v;
          }
        }
      }
    };
    // the lane's drain rows of pass rbase (tile rows rbase + 8 j + lane / 8): o[j] = off(tile row, sorted row), or -1
    // past the tile's rows
    [[maybe_unused]] auto rows_of = [&](int rbase, auto&& off) {
      RowOffs r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rt = rbase + 8 * j + (lane >> 3);
        const int64_t row = row0 + rt;
        r.o[j] = row < row_end ? off(rt, row) : (int64_t)-1;
      }
      return r;
    };
    [[maybe_unused]] auto row_scale = [&](int rt) -> float {
      if (!p.scale) return 1.0f;
      return p.scale_f32 ? s_rowsc[par][rt + sc_sh] : X::one(reinterpret_cast<const uint16_t*>(s_rowsc[par])[rt + sc_sh]);
    };
    auto col_of = [&](int b, int g) { return b * C::FSN + wn * 32 + 8 * g + lcol; };  // tile column (write phase)
#pragma unroll
    for (int a = 0; a < C::FM; ++a) {
      if (a >= fe_rows) break;  // no tile rows in this or later passes (partial m-tile)
      const int rbase = a * C::FSM + wm * 32;  // tile row of the wave's row 0 in this pass
      if constexpr (EPI == EPI_WGRAD) {
        auto park_all = [&](auto f32_tag) {
#pragma unroll
          for (int b = 0; b < C::FN; ++b) {
            pin_agpr(acc[a][b]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const f32x16& v = acc[a][b];
              if constexpr (decltype(f32_tag)::value)
                park_f32(0, b, g, make_float4(v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]));
              else
                park_bf16(0, b, g, cvt_bf2(v[4 * g], v[4 * g + 1]), cvt_bf2(v[4 * g + 2], v[4 * g + 3]));
            }
          }
        };
        const int es = p.c_f32 ? 4 : 2;
        RowOffs rows;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = i0 + rbase + 8 * j + (lane >> 3);
          rows.o[j] = i < p.P ? ((int64_t)e * p.strideCe + (int64_t)i * p.ldc) * es : (int64_t)-1;
        }
        char* const base = reinterpret_cast<char*>(p.C);
        if (p.c_f32) {
          park_all(std::true_type{});
          drain_rows(std::integral_constant<int, C::FN * 32 * 4 / 128>{}, 0, C::FN * 32 * 4, 4, base, rows, p.N,
                     std::true_type{});
        } else {
          park_all(std::false_type{});
          drain_rows(std::integral_constant<int, C::FN * 32 * 2 / 128>{}, 0, C::FN * 32 * 2, 2, base, rows, p.N,
                     std::true_type{});
        }
      } else if constexpr (EPI == EPI_STORE || EPI == EPI_STORE_F32) {
        constexpr int ES = EPI == EPI_STORE_F32 ? 4 : 2;
        constexpr int RB = C::FN * 32 * ES, NSP = (RB + 127) / 128;  // y's row bytes, sub-planes; yhat (bf16) follows
        const float sc = row_scale(rbase + lrow);   // 1 without a scale: the product is then exact
        // aux: also park yhat (bf16 weights only); scf_tag: fp32 int8 column scales, chosen once per pass so that the
        // int8 column scales of a fragment's four groups are read together
        auto park_all = [&](bool aux, auto scf_tag) {
#pragma unroll
          for (int b = 0; b < C::FN; ++b) {
            pin_agpr(acc[a][b]);
            [[maybe_unused]] float ws[4][4];
            if constexpr (C::BE == 1) {
#pragma unroll
              for (int g = 0; g < 4; ++g) col_scale4(scf_tag, col_of(b, g), ws[g]);
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const f32x16& v = acc[a][b];
              if (C::BE == 2 && aux)
                park_bf16(NSP, b, g, X::pack2(v[4 * g], v[4 * g + 1]), X::pack2(v[4 * g + 2], v[4 * g + 3]));
              float v0, v1, v2, v3;
              if constexpr (C::BE == 1) {  // int8 weights: column scale first, then the row scale (two products)
                v0 = (v[4 * g] * ws[g][0]) * sc, v1 = (v[4 * g + 1] * ws[g][1]) * sc;
                v2 = (v[4 * g + 2] * ws[g][2]) * sc, v3 = (v[4 * g + 3] * ws[g][3]) * sc;
              } else {
                v0 = v[4 * g] * sc, v1 = v[4 * g + 1] * sc, v2 = v[4 * g + 2] * sc, v3 = v[4 * g + 3] * sc;
              }
              if constexpr (EPI == EPI_STORE_F32)
                park_f32(0, b, g, make_float4(v0, v1, v2, v3));
              else
                park_bf16(0, b, g, X::pack2(v0, v1), X::pack2(v2, v3));
            }
          }
        };
        // the int8 entry points keep no yhat (aux is NULL with int8 weights)
        const bool aux = C::BE == 2 && p.aux;
        if (C::BE == 1 && p.w_scale_f32)
          park_all(aux, std::true_type{});
        else
          park_all(aux, std::false_type{});
        const RowOffs rows = rows_of(rbase, [&](int rt, int64_t row) {
          return (p.y_idx ? (int64_t)s_rowy[par][rt + y_sh] : row) * p.ldc * ES;
        });
        constexpr std::bool_constant<C::BE == 1> paired{};  // int8 weights: paired reads (bf16: one by one)
        drain_rows(std::integral_constant<int, NSP>{}, 0, RB, ES, reinterpret_cast<char*>(p.C), rows, p.N, paired);
        if constexpr (C::BE == 2) {
          if (aux)
            drain_rows(std::integral_constant<int, (C::FN * 32 * 2 + 127) / 128>{}, NSP, C::FN * 32 * 2, 2,
                       reinterpret_cast<char*>(p.aux),
                       rows_of(rbase, [&](int, int64_t row) { return row * p.ldc * 2; }), p.N, paired);
        }
      } else if constexpr (EPI == EPI_SWIGLU) {
        // fragments b < FN/2 hold gate columns, b + FN/2 the matching up columns (tile columns + BN/2); the wave's
        // activation columns are b*32 + ... for b < FN/2: sub-plane 0 = act, 1 = g, 2 = u (one each for FN = 4)
        constexpr int RB = C::FN / 2 * 32 * 2, NSP = (RB + 127) / 128;  // row bytes and sub-planes of each array
        // aux: also park [g | u] (bf16 weights only); scf_tag: fp32 int8 column scales (chosen once per pass)
        auto park_all = [&](bool aux, auto scf_tag) {
#pragma unroll
          for (int b = 0; b < C::FN / 2; ++b) {
            pin_agpr(acc[a][b]);
            pin_agpr(acc[a][b + C::FN / 2]);
            [[maybe_unused]] float wg[4][4], wu[4][4];
            if constexpr (C::BE == 1) {  // int8 weights: per-column scales of the gate and up columns
#pragma unroll
              for (int g = 0; g < 4; ++g) {
                col_scale4(scf_tag, col_of(b, g), wg[g]);
                col_scale4(scf_tag, col_of(b + C::FN / 2, g), wu[g]);
              }
            }
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const f32x16& gv = acc[a][b];
              const f32x16& uv = acc[a][b + C::FN / 2];
              float gs[4] = {gv[4 * g], gv[4 * g + 1], gv[4 * g + 2], gv[4 * g + 3]};
              float us[4] = {uv[4 * g], uv[4 * g + 1], uv[4 * g + 2], uv[4 * g + 3]};
              if constexpr (C::BE == 1) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                  gs[t] *= wg[g][t];
                  us[t] *= wu[g][t];
                }
              }
              const uint32_t gb0 = X::pack2(gs[0], gs[1]), gb1 = X::pack2(gs[2], gs[3]);
              const uint32_t ub0 = X::pack2(us[0], us[1]), ub1 = X::pack2(us[2], us[3]);
              const float gg[4] = {X::lo(gb0), X::hi(gb0), X::lo(gb1), X::hi(gb1)};
              const float uu[4] = {X::lo(ub0), X::hi(ub0), X::lo(ub1), X::hi(ub1)};
              // act = R(R(silu(g)) * u) with g, u the rounded projections (R: to bf16, or fp16 with F16)
              const uint32_t sl0 = X::pack2(silu_f(gg[0]), silu_f(gg[1])), sl1 = X::pack2(silu_f(gg[2]), silu_f(gg[3]));
              park_bf16(0, b, g, X::pack2(X::lo(sl0) * uu[0], X::hi(sl0) * uu[1]),
                        X::pack2(X::lo(sl1) * uu[2], X::hi(sl1) * uu[3]));
              if (C::BE == 2 && aux) {
                park_bf16(NSP, b, g, gb0, gb1);
                park_bf16(2 * NSP, b, g, ub0, ub1);
              }
            }
          }
        };
        // the int8 entry point keeps no [g | u] (aux is NULL with int8 weights)
        const bool aux = C::BE == 2 && p.aux;
        if (C::BE == 1 && p.w_scale_f32)
          park_all(aux, std::true_type{});
        else
          park_all(aux, std::false_type{});
        constexpr std::bool_constant<C::BE == 1> paired{};  // int8 weights: paired reads (bf16: one by one)
        drain_rows(std::integral_constant<int, NSP>{}, 0, RB, 2, reinterpret_cast<char*>(p.C),
                   rows_of(rbase, [&](int, int64_t row) { return row * p.ldc * 2; }), p.N, paired);
        if constexpr (C::BE == 2) {
          if (aux) {
            const RowOffs rows = rows_of(rbase, [&](int, int64_t row) { return row * (int64_t)(2 * p.h) * 2; });
            drain_rows(std::integral_constant<int, NSP>{}, NSP, RB, 2, reinterpret_cast<char*>(p.aux), rows, p.N,
                       paired);
            drain_rows(std::integral_constant<int, NSP>{}, 2 * NSP, RB, 2, reinterpret_cast<char*>(p.aux + p.h), rows,
                       p.N, paired);
          }
        }
      } else if constexpr (EPI == EPI_SWIGLU_BWD) {
        // Two staging buffers per wave, in the layout park_bf16 writes (so a lane reads its accumulator-shaped 8
        // bytes back): buffer q holds a pass's forward g in sub-planes [2q NSP, (2q+1) NSP) and u in
        // [(2q+1) NSP, (2q+2) NSP).  The pass's dg and du are parked over its g and u (each lane overwrites exactly
        // the bytes it has just read), then drained.  Pass a uses buffer a & 1: the [g | u] of pass a + 1 load while
        // pass a computes and drains, and those of pass a + 2 are issued once pass a's drain has read its buffer.
        constexpr int RB = GU_RB, NSP = GU_NSP;
        constexpr int LG = 2 * NSP * 4;  // direct loads per pass of [g | u]
        static_assert(4 * NSP * 4096 <= 8 * CH, "SwiGLU backward staging: two buffers of g and u sub-planes");
        const float sc = row_scale(rbase + lrow);
        if (a == 0) {
          if (!gu_early) issue_gu(0);
          if (fe_rows > 1) issue_gu(1);
        }
        // this pass's [g | u]: the direct loads are counted in issue order with the stores, and the only memory
        // operations issued after them are the next pass's LG loads (every one issued: absent lanes load kOOB)
        if (a + 1 < fe_rows)
          wait_vm<LG>();
        else
          wait_vm<0>();
        asm volatile("" ::: "memory");
        const int gsp = 2 * (a & 1) * NSP, usp = gsp + NSP;
        // With dw_part: the routing-weight gradient of the lane's row, sum over its columns of the unscaled product
        // (dy @ wd^T) times the forward's act = bf16(bf16(silu(g)) * u), in a fixed order (b, g, t).
        float dwl = 0.0f;
#pragma unroll
        for (int b = 0; b < C::FN; ++b) {
          pin_agpr(acc[a][b]);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int byte = (b * 32 + 8 * g + lcol) * 2;
            const uint2 gl = *reinterpret_cast<const uint2*>(sp_addr(gsp + byte / 128, lrow, byte % 128));
            const uint2 ul = *reinterpret_cast<const uint2*>(sp_addr(usp + byte / 128, lrow, byte % 128));
            const uint32_t gw[2] = {gl.x, gl.y}, uw[2] = {ul.x, ul.y};
            uint32_t dgw[2], duw[2];
#pragma unroll
            for (int tp = 0; tp < 2; ++tp) {  // element pairs (t, t + 1), t = 2 tp
              const float g0 = bf_lo(gw[tp]), g1 = bf_hi(gw[tp]), u0 = bf_lo(uw[tp]), u1 = bf_hi(uw[tp]);
              const float s0 = sigmoid_f(g0), s1 = sigmoid_f(g1);
              const float l0 = g0 * s0, l1 = g1 * s1;  // silu_f(g), as the forward computes it
              // du uses the forward's stored factor bf16(silu(g))
              const uint32_t sb = cvt_bf2(l0, l1);
              const float b0 = bf_lo(sb), b1 = bf_hi(sb);
              const float a0 = acc[a][b][4 * g + 2 * tp], a1 = acc[a][b][4 * g + 2 * tp + 1];
              const float da0 = a0 * sc, da1 = a1 * sc;
              duw[tp] = cvt_bf2(da0 * b0, da1 * b1);
              // silu'(g) = sig (1 + g (1 - sig)) = sig + silu(g) (1 - sig)
              dgw[tp] = cvt_bf2((da0 * u0) * __builtin_fmaf(l0, 1.0f - s0, s0),
                                (da1 * u1) * __builtin_fmaf(l1, 1.0f - s1, s1));
              if (p.dw_part) {
                const uint32_t av = cvt_bf2(b0 * u0, b1 * u1);
                dwl = __builtin_fmaf(a0, bf_lo(av), dwl);
                dwl = __builtin_fmaf(a1, bf_hi(av), dwl);
              }
            }
            *reinterpret_cast<uint2*>(sp_addr(gsp + byte / 128, lrow, byte % 128)) = make_uint2(dgw[0], dgw[1]);
            *reinterpret_cast<uint2*>(sp_addr(usp + byte / 128, lrow, byte % 128)) = make_uint2(duw[0], duw[1]);
          }
        }
        if (p.dw_part) {  // lanes l and l + 32 hold the two column halves of one row
          dwl += __shfl_xor(dwl, 32);
          const int64_t row = row0 + rbase + lrow;
          if (lane < 32 && row < row_end) p.dw_part[(int64_t)(2 * nb + wn) * p.M + row] = dwl;  // (partial, row)
        }
        // (one piece read, one stored: fewer live registers than the batched drain, and as fast here)
        for (int q = 0; q < 2; ++q)
          for (int sp = 0; sp < NSP; ++sp)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const int idx = j * 64 + lane, rr = idx >> 3, c = idx & 7;
              if (sp * 128 + c * 16 >= RB) continue;
              const uint4 v = *reinterpret_cast<const uint4*>(sp_addr((q ? usp : gsp) + sp, rr, c * 16));
              const int cw = (sp * 128 + c * 16) / 2;
              const int64_t row = row0 + rbase + rr;
              const int jc = n0 + (cw / 32) * C::FSN + wn * 32 + cw % 32;
              if (row < row_end && jc < p.N)
                *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.C) + row * (int64_t)(2 * p.h) + q * p.h + jc) = v;
            }
        // the drain's LDS reads have returned (the stores above consumed them): the buffer takes pass a + 2's rows
        if (a + 2 < fe_rows) issue_gu(a + 2);
      }
    }
  }
}

// ----------------------------------------------------------------------------------------------------------------
// Launch helpers
// ----------------------------------------------------------------------------------------------------------------
static std::atomic<int> g_num_cus[64];  // per-device CU count (0 = not yet read); host threads may race to fill it

static int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
  int n = g_num_cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return -1;
    g_num_cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <class C, int MODE, bool A_MN, bool B_MN, int EPI, bool A_BLK = false, bool F16 = false>
static int launch(const GemmParams& p, int64_t tiles_upper, hipStream_t s) {
  auto kern = grouped_gemm_kernel<C, MODE, A_MN, B_MN, EPI, A_BLK, F16>;
  static std::atomic<bool> attr_set[64];  // per device: the (idempotent) attribute call is done
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return HMOE_ERR_DEVICE;
  if (!attr_set[dev].load(std::memory_order_acquire)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            C::LDS_BYTES) != hipSuccess)
      return HMOE_ERR_LAUNCH;
    attr_set[dev].store(true, std::memory_order_release);
  }
  const int cus = num_cus();
  if (cus <= 0) return HMOE_ERR_DEVICE;
  const int per_cu = C::LDS_BYTES <= 72 * 1024 ? 2 : 1;  // LDS-limited residency (160 KB per CU)
  int64_t grid = (int64_t)cus * per_cu;
  if (tiles_upper < grid) grid = tiles_upper;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, s, p);
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

// Tile configurations.  Large: 256x256 tile, 4 waves of 128x128 (FM = FN = 4: 256 fp32 accumulators per lane,
// LDS ring 4 x 32 KB).  Small: 128x128, 4 waves of 64x64 (ring 4 x 16 KB, two workgroups per CU), for problems
// with few tiles.
using CfgL = Cfg<256, 256, 2, 2, 4>;
using CfgS = Cfg<128, 128, 2, 2, 4>;
using CfgL8 = Cfg<256, 256, 2, 2, 4, 1>;  // int8 weights (N-contiguous), bf16 activations
using CfgS8 = Cfg<128, 128, 2, 2, 4, 1>;

template <class C, int EPI>
static inline int64_t mgroup_tiles(int64_t M, int64_t E, int64_t ncols) {
  const int64_t mt = (M + C::BM - 1) / C::BM + E;
  const int64_t nbn = EPI == EPI_SWIGLU ? (ncols + C::BN / 2 - 1) / (C::BN / 2) : (ncols + C::BN - 1) / C::BN;
  return mt * nbn;
}

template <class C>
static inline int64_t kgroup_tiles(int64_t E, int64_t P, int64_t N) {
  return E * ((P + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN);
}

static inline int env_force() {
  const char* v = getenv("HMOE_GEMM_TILE");
  if (!v) return 0;
  return v[0] == 'L' ? 1 : v[0] == 'S' ? 2 : 0;
}

static inline int64_t cu_count() {
  const int c = num_cus();
  return c > 0 ? c : 256;
}

// Large (256x256) or small (128x128) tiles.  The rules follow a sweep of every grouped GEMM (forward, both dgrads,
// both weight gradients; bf16 and int8 weights) over 512-16384 tokens, d 256-2048, 8-128 experts, top-2 and top-8,
// h 320-4096, with large tiles, small tiles and the rule alternated in one process on MI355X.  A large tile costs
// about 1.5x less per flop than two co-resident small ones, so large tiles win unless they leave too few tiles to
// spread over the CUs or pad much more of the output.
//
// Row-grouped launches (bf16 weights): large tiles from 5/8 of a tile per CU on (160 tiles on 256 CUs): at 64-128
// tiles small ones ran 15-55% faster, from 160 tiles on large ones ran 10-57% faster, also at K = 320 (the h = 320
// down GEMM, 20-47%).  int8 weights: large tiles only with K of at least 16 slices (the h = 320 down GEMM ran 5-25%
// faster on small int8 tiles) and, for the gate/up GEMM, from 2.5 tiles per CU (at 384-576 tiles the small int8
// tiles ran up to 34% faster).  Either way, once the large tiles give two per CU, small ones where the large would
// pad the output columns by more than 10% (a SwiGLU n-tile with at most 64 live columns of 128 counts as 64: its
// main loop skips the dead half); with fewer tiles the rounds they save matter more (the h = 320 down dgrad ran 53%
// faster on large tiles at 2048 tokens, 3% slower at 8192).
template <int EPI>
static bool pick_large_mgroup(int64_t tiles_large, int64_t ncols, int64_t K, bool int8) {
  const int f = env_force();
  if (f) return f == 1;
  const int64_t cus = cu_count();
  if (tiles_large >= 2 * cus) {
    const int64_t bl = EPI == EPI_SWIGLU ? CfgL::BN / 2 : CfgL::BN, bs = EPI == EPI_SWIGLU ? CfgS::BN / 2 : CfgS::BN;
    int64_t padl = (ncols + bl - 1) / bl * bl;
    const int64_t pads = (ncols + bs - 1) / bs * bs;
    if (EPI == EPI_SWIGLU && ncols % bl && ncols % bl <= bl / 2) padl -= bl / 2;
    if (padl * 10 > pads * 11) return false;
  }
  if (!int8) return tiles_large * 8 >= cus * 5;
  if (K < 16 * kBK) return false;
  return EPI == EPI_SWIGLU ? tiles_large * 2 >= cus * 5 : tiles_large * 8 >= cus * 5;
}

template <int MODE, bool A_MN, bool B_MN, int EPI, bool A_BLK = false, bool F16 = false>
static int launch_mgroup(const GemmParams& p, int64_t ncols, hipStream_t s) {
  const int64_t tl = mgroup_tiles<CfgL, EPI>(p.M, p.E, ncols);
  if (pick_large_mgroup<EPI>(tl, ncols, p.K, false))
    return launch<CfgL, MODE, A_MN, B_MN, EPI, A_BLK, F16>(p, tl, s);
  return launch<CfgS, MODE, A_MN, B_MN, EPI, A_BLK, F16>(p, mgroup_tiles<CfgS, EPI>(p.M, p.E, ncols), s);
}

// the bf16 (f16 = false) or fp16 form of a forward launch
template <int EPI, bool A_BLK = false>
static int launch_fwd(const GemmParams& p, int64_t ncols, bool f16, hipStream_t s) {
  return f16 ? launch_mgroup<MGROUP, false, true, EPI, A_BLK, true>(p, ncols, s)
             : launch_mgroup<MGROUP, false, true, EPI, A_BLK, false>(p, ncols, s);
}

// int8 weights: the int8 tile configurations
template <int EPI, bool F16 = false>
static int launch_mgroup_i8_t(const GemmParams& p, int64_t ncols, hipStream_t s) {
  const int64_t tl = mgroup_tiles<CfgL8, EPI>(p.M, p.E, ncols);
  bool large = pick_large_mgroup<EPI>(tl, ncols, p.K, true);
  // gate/up with many experts (E >= 128): the tile bound counts a partial tile per expert, and below 3.25 large
  // tiles per CU by it the small tiles ran faster (E = 128, h = 320, top-8, 4096 tokens, bound 3.0: gate/up 186 ->
  // 166 us, the BailingMoeV2 block 407 -> 379 us).  At 5120 tokens (3.375) the gate/up alone still ran 5% faster
  // on small tiles but the block, where it shares the CUs with the shared expert, 5% slower; at 3.75 the large
  // tiles ran 5% faster alone.  With 16 or 64 experts the large tiles stay ahead over that range.
  if (large && EPI == EPI_SWIGLU && !env_force() && p.E >= 128 && tl * 4 < cu_count() * 13) large = false;
  if (large) return launch<CfgL8, MGROUP, false, true, EPI, false, F16>(p, tl, s);
  return launch<CfgS8, MGROUP, false, true, EPI, false, F16>(p, mgroup_tiles<CfgS8, EPI>(p.M, p.E, ncols), s);
}
template <int EPI>
static int launch_mgroup_i8(const GemmParams& p, int64_t ncols, bool f16, hipStream_t s) {
  return f16 ? launch_mgroup_i8_t<EPI, true>(p, ncols, s) : launch_mgroup_i8_t<EPI, false>(p, ncols, s);
}

// activation element type of the forward entry points: bf16 or fp16 (rc: HMOE_OK or HMOE_ERR_DTYPE)
static inline bool act16(int dtype, int* rc) {
  *rc = (dtype == HMOE_DT_BF16 || dtype == HMOE_DT_F16) ? HMOE_OK : HMOE_ERR_DTYPE;
  return dtype == HMOE_DT_F16;
}

// Weight gradients: large tiles once they give every CU two tiles, unless they pad the (P, N) output area by more
// than 10% over the small ones (at h = 320 the 256-row tiles pad 320 rows to 512: small ones ran 9-41% faster for
// the down weight gradient and up to 8% for the gate/up one, N = 640).
static bool pick_large_kgroup(int64_t E, int64_t P, int64_t N) {
  const int f = env_force();
  if (f) return f == 1;
  if (kgroup_tiles<CfgL>(E, P, N) < 2 * cu_count()) return false;
  const int64_t al = (P + CfgL::BM - 1) / CfgL::BM * CfgL::BM * ((N + CfgL::BN - 1) / CfgL::BN * CfgL::BN);
  const int64_t as = (P + CfgS::BM - 1) / CfgS::BM * CfgS::BM * ((N + CfgS::BN - 1) / CfgS::BN * CfgS::BN);
  return al * 10 <= as * 11;
}

static inline bool al16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The direct loads address an operand with a 32-bit byte offset from a per-tile (or per-expert) base: a span that
// must stay below 2^31 bytes.
static inline bool off32(int64_t bytes) { return bytes < ((int64_t)1 << 31); }

// int8 weight arguments: (E, K, N) int8 with N contiguous (row stride ld), scales (E, N) bf16 or fp32 with 16-byte
// aligned rows; every offset a tile reads must stay below 2^31 bytes from the expert's base.
static int check_i8(const void* w, int64_t ld, int64_t K, int64_t N, int64_t stride_we, const void* w_scale,
                    int w_scale_dtype) {
  if (!w || !w_scale) return HMOE_ERR_ARG;
  if (w_scale_dtype != HMOE_DT_BF16 && w_scale_dtype != HMOE_DT_F32) return HMOE_ERR_DTYPE;
  if (ld % 16 || stride_we % 16 || !al16(w) || !al16(w_scale)) return HMOE_ERR_ARG;
  if (N % 16) return HMOE_ERR_SHAPE;  // 16 int8 columns per direct-load chunk
  if (K * ld >= (int64_t)1 << 31) return HMOE_ERR_SHAPE;
  return HMOE_OK;
}

static GemmParams base_params(const void* counts, int counts_dtype, int64_t E, int64_t M) {
  GemmParams p = {};
  p.counts = counts;
  p.counts64 = counts_dtype == HMOE_DT_I64;
  p.E = (int)E;
  p.M = M;
  return p;
}

static int check_common(const void* counts, int counts_dtype, int64_t E, int64_t M) {
  if (!counts || E <= 0 || M < 0) return HMOE_ERR_ARG;
  if (E > kMaxEGemm || M > INT32_MAX) return HMOE_ERR_SHAPE;
  if (counts_dtype != HMOE_DT_I32 && counts_dtype != HMOE_DT_I64) return HMOE_ERR_DTYPE;
  return HMOE_OK;
}

}  // namespace hmoe

using namespace hmoe;

extern "C" {

int hmoe_grouped_mm(const void* a, int64_t lda, int a_dtype, const void* w, int w_dtype, int64_t E, int64_t K,
                    int64_t N, int64_t stride_we, int64_t stride_wk, const void* counts, int counts_dtype, int64_t M,
                    const int32_t* a_idx, const int32_t* y_idx, const void* scale, int scale_dtype,
                    const void* w_scale, int w_scale_dtype, void* y, int64_t ldy, hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!a || !w || !y || K <= 0 || N <= 0) return HMOE_ERR_ARG;
  const bool f16 = act16(a_dtype, &rc);  // a, 16-bit w, a 16-bit scale and y share one type: bf16 or fp16
  if (rc) return rc;
  const bool i8 = w_dtype == HMOE_DT_I8;
  if (!i8 && w_dtype != a_dtype) return HMOE_ERR_DTYPE;
  if (i8 != (w_scale != nullptr)) return i8 ? HMOE_ERR_ARG : HMOE_ERR_DTYPE;  // int8 weights come with scales
  if (scale && scale_dtype != a_dtype && scale_dtype != HMOE_DT_F32) return HMOE_ERR_DTYPE;
  if (K % 8 || N % 8 || lda % 8 || ldy % 8 || stride_wk % 8 || stride_we % 8) return HMOE_ERR_SHAPE;
  if (lda < K || ldy < N || stride_wk < N || !al16(a) || !al16(w) || !al16(y)) return HMOE_ERR_ARG;
  if (K > INT32_MAX || N > INT32_MAX || M > INT32_MAX) return HMOE_ERR_SHAPE;
  // direct-load offsets are 32-bit: gathered rows (a_idx < M) and one expert's weights within 2 GiB
  if ((a_idx && !off32(M * lda * 2)) || !off32(K * stride_wk * (i8 ? 1 : 2))) return HMOE_ERR_SHAPE;
  if (i8 && (rc = check_i8(w, stride_wk, K, N, stride_we, w_scale, w_scale_dtype))) return rc;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.a_idx = a_idx;
  p.B = w;
  p.ldb = stride_wk;
  p.strideBe = stride_we;
  p.K = (int)K;
  p.N = (int)N;
  p.C = y;
  p.ldc = ldy;
  p.y_idx = y_idx;
  p.scale = scale;
  p.scale_f32 = scale_dtype == HMOE_DT_F32;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (i8) {
    p.w_scale = w_scale;
    p.w_scale_f32 = w_scale_dtype == HMOE_DT_F32;
    p.ldws = N;
    return launch_mgroup_i8<EPI_STORE>(p, N, f16, s);
  }
  return launch_fwd<EPI_STORE>(p, N, f16, s);
}

int hmoe_gate_up_swiglu(const void* x, int64_t ldx, const int32_t* a_idx, const void* wgu, int64_t E, int64_t d,
                        int64_t h, const void* counts, int counts_dtype, int64_t M, void* act, void* gu, int dtype,
                        hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  const bool f16 = act16(dtype, &rc);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!x || !wgu || !act || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (d % 8 || h % 8 || ldx % 8 || ldx < d) return HMOE_ERR_SHAPE;
  if (!al16(x) || !al16(wgu) || !al16(act) || !al16(gu)) return HMOE_ERR_ARG;
  if ((a_idx && !off32(M * ldx * 2)) || !off32(d * 2 * h * 2)) return HMOE_ERR_SHAPE;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(x);
  p.lda = ldx;
  p.a_idx = a_idx;
  p.B = (wgu);
  p.ldb = 2 * h;
  p.strideBe = d * 2 * h;
  p.K = (int)d;
  p.N = (int)h;
  p.h = (int)h;
  p.C = act;
  p.ldc = h;
  p.aux = static_cast<uint16_t*>(gu);
  return launch_fwd<EPI_SWIGLU>(p, h, f16, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_gate_up_swiglu_tiles(const void* xs_tiles, const void* wgu, int64_t E, int64_t d, int64_t h,
                              const void* counts, int counts_dtype, int64_t M, void* act, void* gu, int dtype,
                              hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  const bool f16 = act16(dtype, &rc);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!xs_tiles || !wgu || !act || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (d % 8 || h % 8) return HMOE_ERR_SHAPE;
  if (!al16(xs_tiles) || !al16(wgu) || !al16(act) || !al16(gu)) return HMOE_ERR_ARG;
  if (!off32(tiles_bytes(M, E, d)) || !off32(d * 2 * h * 2)) return HMOE_ERR_SHAPE;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(xs_tiles);
  p.lda = d;
  p.B = (wgu);
  p.ldb = 2 * h;
  p.strideBe = d * 2 * h;
  p.K = (int)d;
  p.N = (int)h;
  p.h = (int)h;
  p.C = act;
  p.ldc = h;
  p.aux = static_cast<uint16_t*>(gu);
  return launch_fwd<EPI_SWIGLU, true>(p, h, f16, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_down_scatter(const void* act, const void* wd, int64_t E, int64_t h, int64_t d, const void* counts,
                      int counts_dtype, int64_t M, const uint16_t* w_sorted, const int32_t* y_idx, void* y,
                      void* yhat, int dtype, hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  const bool f16 = act16(dtype, &rc);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!act || !wd || !y || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (d % 8 || h % 8) return HMOE_ERR_SHAPE;
  if (!al16(act) || !al16(wd) || !al16(y) || !al16(yhat)) return HMOE_ERR_ARG;
  if (!off32(h * d * 2)) return HMOE_ERR_SHAPE;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(act);
  p.lda = h;
  p.B = (wd);
  p.ldb = d;
  p.strideBe = h * d;
  p.K = (int)h;
  p.N = (int)d;
  p.C = y;
  p.ldc = d;
  p.y_idx = y_idx;
  p.scale = w_sorted;
  p.scale_f32 = 0;
  p.aux = static_cast<uint16_t*>(yhat);
  return launch_fwd<EPI_STORE>(p, d, f16, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_gate_up_swiglu_i8(const void* x, int64_t ldx, const int32_t* a_idx, const void* wgu_q, const void* wgu_s,
                           int wgu_s_dtype, int64_t E, int64_t d, int64_t h, const void* counts, int counts_dtype,
                           int64_t M, void* act, int dtype, hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  const bool f16 = act16(dtype, &rc);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!x || !act || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (d % 8 || h % 16 || ldx % 8 || ldx < d) return HMOE_ERR_SHAPE;
  if (!al16(x) || !al16(act)) return HMOE_ERR_ARG;
  if ((a_idx && !off32(M * ldx * 2)) || !off32(d * 2 * h)) return HMOE_ERR_SHAPE;
  if ((rc = check_i8(wgu_q, 2 * h, d, 2 * h, d * 2 * h, wgu_s, wgu_s_dtype))) return rc;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(x);
  p.lda = ldx;
  p.a_idx = a_idx;
  p.B = wgu_q;
  p.ldb = 2 * h;
  p.strideBe = d * 2 * h;
  p.K = (int)d;
  p.N = (int)h;
  p.h = (int)h;
  p.C = act;
  p.ldc = h;
  p.w_scale = wgu_s;
  p.w_scale_f32 = wgu_s_dtype == HMOE_DT_F32;
  p.ldws = 2 * h;
  return launch_mgroup_i8<EPI_SWIGLU>(p, h, f16, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_down_scatter_i8(const void* act, const void* wd_q, const void* wd_s, int wd_s_dtype, int64_t E, int64_t h,
                         int64_t d, const void* counts, int counts_dtype, int64_t M, const uint16_t* w_sorted,
                         const int32_t* y_idx, void* y, int dtype, hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  const bool f16 = act16(dtype, &rc);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!act || !y || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (h % 8 || d % 16) return HMOE_ERR_SHAPE;
  if (!al16(act) || !al16(y)) return HMOE_ERR_ARG;
  if (!off32(h * d)) return HMOE_ERR_SHAPE;
  if ((rc = check_i8(wd_q, d, h, d, h * d, wd_s, wd_s_dtype))) return rc;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(act);
  p.lda = h;
  p.B = wd_q;
  p.ldb = d;
  p.strideBe = h * d;
  p.K = (int)h;
  p.N = (int)d;
  p.C = y;
  p.ldc = d;
  p.y_idx = y_idx;
  p.scale = w_sorted;
  p.scale_f32 = 0;
  p.w_scale = wd_s;
  p.w_scale_f32 = wd_s_dtype == HMOE_DT_F32;
  p.ldws = d;
  return launch_mgroup_i8<EPI_STORE>(p, d, f16, reinterpret_cast<hipStream_t>(stream));
}

// Checks and parameters shared by the two down-dgrad entry points (rc: HMOE_OK, or the error to return).
static GemmParams down_dgrad_params(const void* dy, const int32_t* a_idx, const uint16_t* w_sorted, const void* wd,
                                    int64_t E, int64_t h, int64_t d, const void* counts, int counts_dtype, int64_t M,
                                    const void* gu, void* dgu, int* rc) {
  GemmParams p = {};
  *rc = check_common(counts, counts_dtype, E, M);
  if (*rc || M == 0) return p;
  if (!dy || !wd || !gu || !dgu || d <= 0 || h <= 0) *rc = HMOE_ERR_ARG;
  else if (d % 8 || h % 8) *rc = HMOE_ERR_SHAPE;
  else if (!al16(dy) || !al16(wd) || !al16(gu) || !al16(dgu)) *rc = HMOE_ERR_ARG;
  else if ((a_idx && !off32(M * d * 2)) || !off32(h * d * 2)) *rc = HMOE_ERR_SHAPE;
  if (*rc) return p;
  p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(dy);
  p.lda = d;
  p.a_idx = a_idx;
  p.B = (wd);  // (E, h, d): row n = h index, k = d contiguous
  p.ldb = d;
  p.strideBe = h * d;
  p.K = (int)d;
  p.N = (int)h;
  p.h = (int)h;
  p.C = dgu;
  p.scale = w_sorted;
  p.gu_in = static_cast<const uint16_t*>(gu);
  return p;
}

int hmoe_down_dgrad_swiglu(const void* dy, const int32_t* a_idx, const uint16_t* w_sorted, const void* wd,
                           int64_t E, int64_t h, int64_t d, const void* counts, int counts_dtype, int64_t M,
                           const void* gu, void* dgu, hmoe_stream_t stream) {
  int rc = HMOE_OK;
  GemmParams p = down_dgrad_params(dy, a_idx, w_sorted, wd, E, h, d, counts, counts_dtype, M, gu, dgu, &rc);
  if (rc || M == 0) return rc;
  return launch_mgroup<MGROUP, false, false, EPI_SWIGLU_BWD>(p, h, reinterpret_cast<hipStream_t>(stream));
}

// partials per row of hmoe_down_dgrad_swiglu_dw's routing-weight gradient: two per n-tile of the chosen tile size
static int64_t dw_partials(int64_t h, bool large) {
  const int64_t bn = large ? CfgL::BN : CfgS::BN;
  return 2 * ((h + bn - 1) / bn);
}

size_t hmoe_down_dgrad_dw_workspace_size(int64_t M, int64_t h) {
  if (M <= 0 || h <= 0) return 256;
  return (size_t)(M * dw_partials(h, false) * 4 + 255) / 256 * 256;  // the small tiles' count is the larger
}

// dtopk_w[order[r]] = sum over q of part[q * M + r], in q order (partial-major: a thread per row, coalesced rows)
__global__ __launch_bounds__(256) void dw_reduce_kernel(const float* __restrict__ part, int P, int64_t M,
                                                        const int32_t* __restrict__ order, float* __restrict__ dtw) {
  for (int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < M; r += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.0f;
    for (int q0 = 0; q0 < P; q0 += 8) {  // eight loads in flight, added in q order
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = q0 + u < P ? part[(int64_t)(q0 + u) * M + r] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (q0 + u < P) s += v[u];
    }
    dtw[order[r]] = s;
  }
}

int hmoe_down_dgrad_swiglu_dw(const void* dy, const int32_t* a_idx, const uint16_t* w_sorted, const void* wd,
                              int64_t E, int64_t h, int64_t d, const void* counts, int counts_dtype, int64_t M,
                              const void* gu, void* dgu, const int32_t* order, float* dtopk_w, void* workspace,
                              size_t workspace_bytes, hmoe_stream_t stream) {
  int rc = HMOE_OK;
  GemmParams p = down_dgrad_params(dy, a_idx, w_sorted, wd, E, h, d, counts, counts_dtype, M, gu, dgu, &rc);
  if (rc || M == 0) return rc;
  if (!order || !dtopk_w) return HMOE_ERR_ARG;
  if (!workspace || workspace_bytes < hmoe_down_dgrad_dw_workspace_size(M, h) || !al16(workspace))
    return HMOE_ERR_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t tl = mgroup_tiles<CfgL, EPI_SWIGLU_BWD>(M, E, h);
  const bool large = pick_large_mgroup<EPI_SWIGLU_BWD>(tl, h, d, false);
  p.dw_part = static_cast<float*>(workspace);
  p.dw_ld = (int)dw_partials(h, large);
  rc = large ? launch<CfgL, MGROUP, false, false, EPI_SWIGLU_BWD>(p, tl, s)
             : launch<CfgS, MGROUP, false, false, EPI_SWIGLU_BWD>(p, mgroup_tiles<CfgS, EPI_SWIGLU_BWD>(M, E, h), s);
  if (rc) return rc;
  hipLaunchKernelGGL(dw_reduce_kernel, dim3((unsigned)std::min<int64_t>((M + 255) / 256, 4096)), dim3(256), 0, s,
                     p.dw_part, p.dw_ld, M, order, dtopk_w);
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

int hmoe_gate_up_dgrad(const void* dgu, const void* wgu, int64_t E, int64_t d, int64_t h, const void* counts,
                       int counts_dtype, int64_t M, void* dxs, int dxs_dtype, hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!dgu || !wgu || !dxs || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (dxs_dtype != HMOE_DT_BF16 && dxs_dtype != HMOE_DT_F32) return HMOE_ERR_DTYPE;
  if (d % 8 || h % 8) return HMOE_ERR_SHAPE;
  if (!al16(dgu) || !al16(wgu) || !al16(dxs)) return HMOE_ERR_ARG;
  if (!off32(d * 2 * h * 2)) return HMOE_ERR_SHAPE;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(dgu);
  p.lda = 2 * h;
  p.B = (wgu);  // (E, d, 2h): row n = d index, k = 2h contiguous
  p.ldb = 2 * h;
  p.strideBe = d * 2 * h;
  p.K = (int)(2 * h);
  p.N = (int)d;
  p.C = dxs;
  p.ldc = d;
  if (dxs_dtype == HMOE_DT_F32)
    return launch_mgroup<MGROUP, false, false, EPI_STORE_F32>(p, d, reinterpret_cast<hipStream_t>(stream));
  return launch_mgroup<MGROUP, false, false, EPI_STORE>(p, d, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_grouped_wgrad(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t E, int64_t P, int64_t N,
                       const void* counts, int counts_dtype, int64_t M, void* dw, int dw_dtype,
                       hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  // M = 0 still writes dw (zeros); no operand row is read then, so a and b may be NULL
  if (!dw || P <= 0 || N <= 0 || (M > 0 && (!a || !b))) return HMOE_ERR_ARG;
  if (dw_dtype != HMOE_DT_F32 && dw_dtype != HMOE_DT_BF16) return HMOE_ERR_DTYPE;
  if (P % 8 || N % 8 || lda % 8 || ldb % 8 || lda < P || ldb < N) return HMOE_ERR_SHAPE;
  if (!al16(a) || !al16(b) || !al16(dw)) return HMOE_ERR_ARG;
  if (!off32(M * lda * 2) || !off32(M * ldb * 2)) return HMOE_ERR_SHAPE;  // an expert's rows from its first
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.B = (b);
  p.ldb = ldb;
  p.P = (int)P;
  p.N = (int)N;
  p.K = 0;
  p.C = dw;
  p.ldc = N;
  p.strideCe = P * N;
  p.c_f32 = dw_dtype == HMOE_DT_F32;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (pick_large_kgroup(E, P, N)) return launch<CfgL, KGROUP, true, true, EPI_WGRAD>(p, kgroup_tiles<CfgL>(E, P, N), s);
  return launch<CfgS, KGROUP, true, true, EPI_WGRAD>(p, kgroup_tiles<CfgS>(E, P, N), s);
}

}  // extern "C"
