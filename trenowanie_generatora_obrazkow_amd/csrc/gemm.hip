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
#include "hmoe_common.h"

namespace hmoe {

constexpr int kBK = 32;      // k per LDS slice
constexpr int kNStage = 4;   // slices in flight
constexpr int kMaxEGemm = 1024;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Source of masked lanes' direct loads: 64 zero bytes.
__device__ __attribute__((aligned(64))) uint16_t g_zero_page[32];

template <int BM_, int BN_, int WM_, int WN_, int GM_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, GM = GM_;
  static constexpr int NWAVES = WM * WN, NT = NWAVES * 64;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 32, FN = TN / 32;
  // a wave's fragments are interleaved with the other waves' along each dimension: fragment f of wave w covers
  // 32 rows / columns from f * FS + 32 w (FS = 32 * waves along that dimension)
  static constexpr int FSM = 32 * WM, FSN = 32 * WN;
  static constexpr int A_BYTES = BM * kBK * 2, B_BYTES = BN * kBK * 2;  // per slice
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = kNStage * STAGE_BYTES;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
};

// ----------------------------------------------------------------------------------------------------------------
// LDS tile layouts (one k-slice of BK = 32)
//   K-major  [ROWS][32]: 64-byte rows, four 16-byte chunks; chunk c of row r stored at c ^ ((r >> 2) & 3).
//   MN-major [32][ROWS]: k-rows of 2*ROWS bytes, ROWS/8 chunks; the low 3 bits of chunk c in k-row k are XORed
//            with ((2 * (k & 3)) | ((k >> 3) & 1)).
// Both swizzles make the fragment reads below conflict-free (K-major) or close to it (transpose reads).
// ----------------------------------------------------------------------------------------------------------------
__device__ __forceinline__ int swz_k(int row) { return (row >> 2) & 3; }
__device__ __forceinline__ int swz_mn(int k) { return ((2 * (k & 3)) | ((k >> 3) & 1)) & 7; }
__device__ __forceinline__ int mn_chunk(int k, int c) { return (c & ~7) | ((c ^ swz_mn(k)) & 7); }

// Direct global -> LDS copy of 16 bytes per lane: lane l's bytes land at lds + 16 l (lds is wave-uniform; it goes
// to M0).  Issued as inline asm so the compiler does not guard every later LDS read with a vmcnt(0) wait for it:
// completion of these copies is tracked explicitly (wait_vm + barrier before a slice is read).
__device__ __forceinline__ void g2lds(const uint16_t* src, char* lds) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src) : "memory", "m0");
}

// K-major operand: ROWS rows x 32 k per slice; ROWS/16 copy instructions per slice (each 16 rows x 64 bytes),
// spread over the workgroup's waves.
template <int ROWS, int NWAVES>
struct KTile {
  static constexpr int INSTR = ROWS / 16;
  static constexpr int PER_WAVE = INSTR / NWAVES;
  static_assert(INSTR % NWAVES == 0, "K tile copy instructions must divide over the waves");
  const uint16_t* rowp[PER_WAVE];  // row base (k = 0) of the row this lane copies, or the zero page
  int chunk[PER_WAVE];             // logical k-chunk this lane copies
  int K;
  // lane l of instruction (wave w, i) fills LDS row 16*(w*PER_WAVE + i) + l/4, physical chunk l%4
  __device__ __forceinline__ int row_of(int wave, int lane, int i) const { return 16 * (wave * PER_WAVE + i) + lane / 4; }
  __device__ __forceinline__ void issue(char* lds_tile, int wave, int lane, int k0) const {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int kk = k0 + chunk[i] * 8;
      const uint16_t* src = (rowp[i] != g_zero_page && kk < K) ? rowp[i] + kk : g_zero_page;
      g2lds(src, lds_tile + (wave * PER_WAVE + i) * 1024);
    }
  }
  // Lane part of a fragment read address: row w32*32 + lane%32, k-chunk lane/32 (ks = 0), swizzled.  The
  // swizzle of row grp64 + w32*32 + lane%32 is that of lane%32, and chunk 2 + c stored at (2 + c) ^ s = (c ^ s) ^ 2,
  // so the 64-row group and ks parts are compile-time offsets.
  __device__ __forceinline__ static int lane_off(int w32, int lane) {
    const int row = w32 * 32 + (lane & 31);
    return row * 64 + (((lane >> 5) ^ swz_k(row)) * 16);
  }
  // MFMA operand fragment: 32 rows (grp64 + 32 w32 + lane%32) x 16 k (ks*16 + (lane/32)*8 + 0..7)
  __device__ __forceinline__ static bf16x8 frag(const char* lds_tile, int grp64, int loff, int ks) {
    return *reinterpret_cast<const bf16x8*>(lds_tile + grp64 * 64 + (loff ^ (ks * 32)));
  }
};

// MN-major operand: 32 k-rows x ROWS columns per slice; ROWS/16 copy instructions (each 1 KB = 512/ROWS k-rows).
template <int ROWS, int NWAVES>
struct MNTile {
  static constexpr int INSTR = ROWS / 16;
  static constexpr int PER_WAVE = INSTR / NWAVES;
  static constexpr int CPR = ROWS / 8;      // 16-byte chunks per k-row
  static constexpr int KPI = 64 / CPR;      // k-rows per copy instruction
  static_assert(INSTR % NWAVES == 0, "MN tile copy instructions must divide over the waves");
  const uint16_t* colp[PER_WAVE];  // (k = 0, first of the 8 columns) of the chunk this lane copies, or zero page
  int krow[PER_WAVE];              // k-row within the slice
  int64_t ld;
  int Kvalid;
  __device__ __forceinline__ void issue(char* lds_tile, int wave, int lane, int k0) const {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int k = k0 + krow[i];
      const uint16_t* src = (colp[i] != g_zero_page && k < Kvalid) ? colp[i] + (int64_t)k * ld : g_zero_page;
      g2lds(src, lds_tile + (wave * PER_WAVE + i) * 1024);
    }
  }
  // lane l of instruction (wave w, i): k-row (w*PER_WAVE + i)*KPI + l / CPR, physical chunk l % CPR
  __device__ __forceinline__ static void slot(int wave, int lane, int i, int& k, int& col) {
    k = (wave * PER_WAVE + i) * KPI + lane / CPR;
    col = mn_chunk(k, lane % CPR) * 8;  // the logical column this physical slot holds
  }
  // Lane part of a fragment read address (see frag): k-row (g/2)*8 + j, columns w32*32 + (g%2)*16 + 4a of the
  // 64-column group, swizzled.  k & 3 = j and (k >> 3) & 1 = g / 2 for every (ks, hh), so the swizzle is a lane
  // constant and the (ks, hh, 64-column group) parts of the address are compile-time offsets.
  __device__ __forceinline__ static int lane_off(int w32, int lane) {
    const int g = lane >> 4, j = (lane >> 2) & 3, a = lane & 3;
    const int k = (g >> 1) * 8 + j;
    const int c = w32 * 4 + (g & 1) * 2 + (a >> 1);  // chunk within the 64-column group, 0..7
    const int s = (2 * j) | (g >> 1);                 // swz_mn(k) for every k this lane reads
    return k * (ROWS * 2) + ((c ^ s) & 7) * 16 + (a & 1) * 8;
  }
  // MFMA operand fragment via two transpose reads: 32 columns (grp64 + 32 w32 + lane%32) x 16 k
  // (ks*16 + (lane/32)*8 + 0..7); `loff` = lane_off(w32, lane).
  __device__ __forceinline__ static bf16x8 frag(const char* lds_tile, int grp64, int loff, int ks) {
    s16x4 h[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const char* p = lds_tile + loff + (ks * 16 + 4 * hh) * (ROWS * 2) + grp64 * 2;
      h[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
    }
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 v = __builtin_shufflevector(h[0], h[1], 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, v);
  }
};

template <bool MN, int ROWS, int NWAVES>
struct TileSel;
template <int ROWS, int NWAVES>
struct TileSel<false, ROWS, NWAVES> {
  using type = KTile<ROWS, NWAVES>;
};
template <int ROWS, int NWAVES>
struct TileSel<true, ROWS, NWAVES> {
  using type = MNTile<ROWS, NWAVES>;
};

// Workgroup barrier that orders LDS only.  __syncthreads() is a workgroup release/acquire fence over all address
// spaces, which on gfx9 also drains every outstanding global store (vmcnt(0)) -- the epilogue's stores would then be
// waited for at each band pass.  Global data staged by the direct loads is ordered by wait_vm() before this barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// wait until at most N vector-memory operations of this thread are outstanding (s_waitcnt vmcnt(N); the
// expcnt / lgkmcnt fields are left at their maxima so they do not wait)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ----------------------------------------------------------------------------------------------------------------
// Kernel parameters
// ----------------------------------------------------------------------------------------------------------------
enum Mode { MGROUP = 0, KGROUP = 1 };
enum Epi { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_SWIGLU_BWD = 2, EPI_WGRAD = 3 };

struct GemmParams {
  // M side (A).  MGROUP: rows of A (sorted row r, or a_idx[r] when gather), K contiguous, row stride lda.
  //              KGROUP: X (M, P) with P contiguous, row stride lda.
  const uint16_t* A;
  int64_t lda;
  const int32_t* a_idx;
  // N side (B).  MGROUP: weights of expert e at B + e*strideBe; B_MN: element (k, n) at k*ldb + n, else n*ldb + k.
  //              KGROUP: Y (M, N) with N contiguous, row stride ldb.
  const uint16_t* B;
  int64_t ldb, strideBe;
  // groups
  const void* counts;
  int counts64;
  int E;
  int64_t M;  // total sorted rows (clamp)
  int K;      // MGROUP reduction length
  int N;      // output columns (EPI_SWIGLU / EPI_SWIGLU_BWD: h)
  int P;      // KGROUP output rows per expert
  int h;      // SwiGLU: offset of the up half in wgu / gu / dgu
  // epilogue
  void* C;  // EPI_STORE: y; EPI_SWIGLU: act (M, h); EPI_SWIGLU_BWD: dgu (M, 2h); EPI_WGRAD: dw (E, P, N)
  int64_t ldc, strideCe;
  int c_f32;                // EPI_WGRAD / EPI_STORE: fp32 output
  const int32_t* y_idx;     // EPI_STORE scatter
  const void* scale;        // EPI_STORE / EPI_SWIGLU_BWD per-row scale
  int scale_f32;
  uint16_t* aux;            // EPI_STORE: yhat (unscaled, sorted); EPI_SWIGLU: gu store
  const uint16_t* gu_in;    // EPI_SWIGLU_BWD: [g | u]
};

// ----------------------------------------------------------------------------------------------------------------
// The kernel
// ----------------------------------------------------------------------------------------------------------------
template <class C, int MODE, bool A_MN, bool B_MN, int EPI>
__global__ __launch_bounds__(C::NT, 1) void grouped_gemm_kernel(GemmParams p) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  __shared__ int64_t s_rstart[kMaxEGemm + 1];
  __shared__ int s_tstart[kMaxEGemm + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int E = p.E;

  // ---- per-expert row starts and tile starts (wave 0, lane-parallel scan) ----
  if (wave == 0) {
    const int per = (E + 63) / 64;
    int64_t rs = 0;
    int ts = 0;
    for (int i = 0; i < per; ++i) {
      const int e = lane * per + i;
      if (e < E) {
        int64_t c = read_count(p.counts, p.counts64, e);
        c = c < 0 ? 0 : (c > p.M ? p.M : c);  // garbage counts must not blow up the tile loop
        rs += c;
        ts += MODE == MGROUP ? (int)((c + C::BM - 1) / C::BM) : 1;
      }
    }
    int64_t irs = rs;
    int its = ts;
#pragma unroll
    for (int s = 1; s < 64; s <<= 1) {
      const int64_t o = __shfl_up(irs, s, 64);
      const int ot = __shfl_up(its, s, 64);
      if (lane >= s) {
        irs += o;
        its += ot;
      }
    }
    int64_t r0 = irs - rs;
    int t0 = its - ts;
    for (int i = 0; i < per; ++i) {
      const int e = lane * per + i;
      if (e < E) {
        int64_t c = read_count(p.counts, p.counts64, e);
        c = c < 0 ? 0 : (c > p.M ? p.M : c);
        s_rstart[e] = r0;
        s_tstart[e] = t0;
        r0 += c;
        t0 += MODE == MGROUP ? (int)((c + C::BM - 1) / C::BM) : 1;
      }
    }
    if (lane == 63) {
      s_rstart[E] = irs;
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
  typename TileSel<B_MN, C::BN, C::NWAVES>::type tb;
  static_assert(C::FSM == 64 && C::FSN == 64, "fragment reads assume two waves along each tile dimension");
  const int loff_a = decltype(ta)::lane_off(wm, lane);
  const int loff_b = decltype(tb)::lane_off(wn, lane);

  // XCD-aware slot: consecutive workgroup ids are dealt round-robin over the 8 XCDs; give each XCD a contiguous
  // range of tile ids so the tiles it runs share A rows and B columns in its L2.
  const int G = gridDim.x;
  int slot = blockIdx.x;
  if ((G & 7) == 0) slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);

  for (int tile = slot; tile < total; tile += G) {
    // ---- tile decode ----
    int mt, nb;
    {
      const int per_group = C::GM * nb_n;
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
      row_end = min(s_rstart[e + 1], p.M);
    } else {
      e = mt / nb_i;
      i0 = (mt - e * nb_i) * C::BM;
      kstart = s_rstart[e];
      const int64_t kend = min(s_rstart[e + 1], p.M);
      kvalid = (int)max((int64_t)0, kend - kstart);
    }
    const int n0 = nb * (EPI == EPI_SWIGLU ? C::BN / 2 : C::BN);

    // ---- copy sources for this tile ----
    if constexpr (MODE == MGROUP) {
      static_assert(!A_MN, "MGROUP A is K-contiguous");
      ta.K = p.K;
#pragma unroll
      for (int i = 0; i < ta.PER_WAVE; ++i) {
        const int rr = ta.row_of(wave, lane, i);
        const int64_t r = row0 + rr;
        const uint16_t* ptr = g_zero_page;
        if (r < row_end) {
          const int64_t src = p.a_idx ? (int64_t)p.a_idx[r] : r;
          ptr = p.A + src * p.lda;
        }
        ta.rowp[i] = ptr;
        ta.chunk[i] = (lane & 3) ^ swz_k(rr);
      }
      const uint16_t* Be = p.B + (int64_t)e * p.strideBe;
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
        tb.ld = p.ldb;
        tb.Kvalid = p.K;
#pragma unroll
        for (int i = 0; i < tb.PER_WAVE; ++i) {
          int k, nn, col;
          tb.slot(wave, lane, i, k, nn);
          tb.krow[i] = k;
          tb.colp[i] = gcol(nn, col) ? Be + col : g_zero_page;
        }
      } else {
        tb.K = p.K;
#pragma unroll
        for (int i = 0; i < tb.PER_WAVE; ++i) {
          const int nn = tb.row_of(wave, lane, i);
          int col;
          tb.rowp[i] = gcol(nn, col) ? Be + (int64_t)col * p.ldb : g_zero_page;
          tb.chunk[i] = (lane & 3) ^ swz_k(nn);
        }
      }
    } else {
      static_assert(A_MN && B_MN, "KGROUP operands are MN-contiguous");
      ta.ld = p.lda;
      ta.Kvalid = kvalid;
      tb.ld = p.ldb;
      tb.Kvalid = kvalid;
#pragma unroll
      for (int i = 0; i < ta.PER_WAVE; ++i) {
        int k, ic;
        ta.slot(wave, lane, i, k, ic);
        ta.krow[i] = k;
        ta.colp[i] = (i0 + ic < p.P) ? p.A + kstart * p.lda + i0 + ic : g_zero_page;
      }
#pragma unroll
      for (int i = 0; i < tb.PER_WAVE; ++i) {
        int k, nc;
        tb.slot(wave, lane, i, k, nc);
        tb.krow[i] = k;
        tb.colp[i] = (n0 + nc < p.N) ? p.B + kstart * p.ldb + n0 + nc : g_zero_page;
      }
    }

    // ---- main loop: NSTAGE-deep ring of k-slices ----
    f32x16 acc[C::FM][C::FN];
#pragma unroll
    for (int a = 0; a < C::FM; ++a)
#pragma unroll
      for (int b = 0; b < C::FN; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    constexpr int LOADS = decltype(ta)::PER_WAVE + decltype(tb)::PER_WAVE;  // direct loads per thread per slice
    const int nk = (kvalid + kBK - 1) / kBK;
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
    typedef typename TileSel<A_MN, C::BM, C::NWAVES>::type TA;
    typedef typename TileSel<B_MN, C::BN, C::NWAVES>::type TB;
    constexpr int RD = C::FM * (A_MN ? 2 : 1) + C::FN * (B_MN ? 2 : 1);  // LDS reads per k16 step
    constexpr int NMF = C::FM * C::FN;                                     // MFMAs per k16 step
    constexpr int PAIRS = RD < NMF ? RD : NMF;
    struct Frags {
      bf16x8 xa[C::FM], wb[C::FN];
    };
    auto read = [&](const char* slot, int ks) {
      Frags f;
#pragma unroll
      for (int a = 0; a < C::FM; ++a) f.xa[a] = TA::frag(slot, a * C::FSM, loff_a, ks);
#pragma unroll
      for (int b = 0; b < C::FN; ++b) f.wb[b] = TB::frag(slot + C::A_BYTES, b * C::FSN, loff_b, ks);
      return f;
    };
    auto mfmas = [&](const Frags f) {
#pragma unroll
      for (int a = 0; a < C::FM; ++a)
#pragma unroll
        for (int b = 0; b < C::FN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.wb[b], f.xa[a], acc[a][b], 0, 0, 0);
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
    static_assert(kNStage == 4 && kBK == 32, "pipeline written for a 4-deep ring of two-step slices");
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
    // The two MFMA blocks are unconditional (a conditional copy would split the accumulators' live ranges); on the
    // last slice the ks0 read of the "next" slot reads stale LDS that is never used.
    for (int kt = 0; kt < nk; ++kt) {
      f1 = read(cons, 1);
      mfmas(f0);
      interleave();
      const int ahead = min(nk - 1, kt + kNStage - 1) - (kt + 1);  // slices issued after slice kt+1
      if (ahead >= 2)
        wait_vm<2 * LOADS>();
      else if (ahead == 1)
        wait_vm<LOADS>();
      else
        wait_vm<0>();
      lds_barrier();
      if (kt + kNStage < nk) issue(kt + kNStage);  // into the slot of slice kt (fill == cons here)
      cons += C::STAGE_BYTES;
      if (cons == ring_end) cons = smem;
      f0 = read(cons, 0);
      mfmas(f1);
      interleave();
    }
    lds_barrier();  // every wave is done with the ring before the epilogue reuses it

    // ---- epilogue, through LDS in bands of 64 rows ----
    // Pass a: every wave parks its fragment row a (rows a*64 + wm*32 + 0..31 of the tile, all its columns) in LDS
    // as fp32 [64][BN + 4] (the padding makes both phases' 16-byte accesses bank-conflict free), then the workgroup
    // walks the band row-contiguously: thread t owns band row t/4 and the 8-column groups (t%4)*8 + 32m, so each
    // global store is a 16- or 32-byte vector and four neighbouring threads cover 64 contiguous bytes of a row.
    constexpr int EP = C::BN + 4;  // band row pitch, floats
    static_assert(64 * EP * 4 <= C::LDS_BYTES, "epilogue band must fit in the ring");
    float* band = reinterpret_cast<float*>(smem);
    const int lrow = lane & 31;
    const int lcol = 4 * (lane >> 5);
    const int q = tid >> 2, s = tid & 3;
#pragma unroll
    for (int a = 0; a < C::FM; ++a) {
      // SwiGLU backward: issue this pass's [g | u] loads first, so their latency overlaps phase 1 and the barrier
      // (rows / columns outside the tile load a valid location and are never used)
      [[maybe_unused]] uint4 gpre[C::BN / 32], upre[C::BN / 32];
      if constexpr (EPI == EPI_SWIGLU_BWD) {
        const int64_t r = row0 + a * 64 + q;
        const uint16_t* gurow = p.gu_in + (r < row_end ? r : row0) * (int64_t)(2 * p.h);
#pragma unroll
        for (int m = 0; m < C::BN / 32; ++m) {
          const int j = n0 + 32 * m + 8 * s;
          const int jc = j < p.N ? j : 0;
          gpre[m] = *reinterpret_cast<const uint4*>(gurow + jc);
          upre[m] = *reinterpret_cast<const uint4*>(gurow + p.h + jc);
        }
      }
      // phase 1: park fragment row a
#pragma unroll
      for (int b = 0; b < C::FN; ++b)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float* dst = band + (wm * 32 + lrow) * EP + b * C::FSN + wn * 32 + 8 * g + lcol;
          *reinterpret_cast<float4*>(dst) =
              make_float4(acc[a][b][4 * g], acc[a][b][4 * g + 1], acc[a][b][4 * g + 2], acc[a][b][4 * g + 3]);
        }
      lds_barrier();
      // phase 2: band row q, columns 32m + 8s + 0..7
      const float* brow = band + q * EP + 8 * s;
      auto ld8 = [&](int col, float* v) {
        const float4 x0 = *reinterpret_cast<const float4*>(brow + col);
        const float4 x1 = *reinterpret_cast<const float4*>(brow + col + 4);
        v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
        v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
      };
      auto pack8 = [](const float* v) {
        return make_uint4(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]), pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7]));
      };
      if constexpr (EPI == EPI_WGRAD) {
        const int i = i0 + a * 64 + q;
        if (i < p.P) {
          char* crow = reinterpret_cast<char*>(p.C) + ((int64_t)e * p.strideCe + (int64_t)i * p.ldc) * (p.c_f32 ? 4 : 2);
#pragma unroll
          for (int m = 0; m < C::BN / 32; ++m) {
            const int n = n0 + 32 * m + 8 * s;
            if (n >= p.N) continue;
            float v[8];
            ld8(32 * m, v);
            if (p.c_f32) {
              float4* d = reinterpret_cast<float4*>(crow + (int64_t)n * 4);
              d[0] = make_float4(v[0], v[1], v[2], v[3]);
              d[1] = make_float4(v[4], v[5], v[6], v[7]);
            } else {
              *reinterpret_cast<uint4*>(crow + (int64_t)n * 2) = pack8(v);
            }
          }
        }
      } else if constexpr (EPI == EPI_STORE) {
        const int64_t r = row0 + a * 64 + q;
        if (r < row_end) {
          float sc = 1.0f;
          if (p.scale) sc = p.scale_f32 ? reinterpret_cast<const float*>(p.scale)[r]
                                        : bf2f(reinterpret_cast<const uint16_t*>(p.scale)[r]);
          const int64_t yr = p.y_idx ? (int64_t)p.y_idx[r] : r;
          char* yrow = reinterpret_cast<char*>(p.C) + yr * p.ldc * (p.c_f32 ? 4 : 2);
#pragma unroll
          for (int m = 0; m < C::BN / 32; ++m) {
            const int n = n0 + 32 * m + 8 * s;
            if (n >= p.N) continue;
            float v[8];
            ld8(32 * m, v);
            if (p.aux) *reinterpret_cast<uint4*>(p.aux + r * p.ldc + n) = pack8(v);
            if (p.scale) {
#pragma unroll
              for (int t = 0; t < 8; ++t) v[t] = v[t] * sc;
            }
            if (p.c_f32) {
              float4* d = reinterpret_cast<float4*>(yrow + (int64_t)n * 4);
              d[0] = make_float4(v[0], v[1], v[2], v[3]);
              d[1] = make_float4(v[4], v[5], v[6], v[7]);
            } else {
              *reinterpret_cast<uint4*>(yrow + (int64_t)n * 2) = pack8(v);
            }
          }
        }
      } else if constexpr (EPI == EPI_SWIGLU) {
        // tile columns [0, BN/2) are gate, [BN/2, BN) the matching up columns
        const int64_t r = row0 + a * 64 + q;
        if (r < row_end) {
          uint16_t* arow = reinterpret_cast<uint16_t*>(p.C) + r * p.ldc;
          uint16_t* grow = p.aux ? p.aux + r * (int64_t)(2 * p.h) : nullptr;
#pragma unroll
          for (int m = 0; m < C::BN / 64; ++m) {
            const int j = n0 + 32 * m + 8 * s;
            if (j >= p.N) continue;
            float gv[8], uv[8], o[8];
            ld8(32 * m, gv);
            ld8(C::BN / 2 + 32 * m, uv);
            uint32_t gb[8], ub[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              gb[t] = f2bf(gv[t]);
              ub[t] = f2bf(uv[t]);
              const float sl = bf2f(f2bf(silu_f(bf2f(gb[t]))));
              o[t] = sl * bf2f(ub[t]);
            }
            *reinterpret_cast<uint4*>(arow + j) = pack8(o);
            if (grow) {
              *reinterpret_cast<uint4*>(grow + j) = make_uint4(gb[0] | (gb[1] << 16), gb[2] | (gb[3] << 16),
                                                               gb[4] | (gb[5] << 16), gb[6] | (gb[7] << 16));
              *reinterpret_cast<uint4*>(grow + p.h + j) = make_uint4(ub[0] | (ub[1] << 16), ub[2] | (ub[3] << 16),
                                                                     ub[4] | (ub[5] << 16), ub[6] | (ub[7] << 16));
            }
          }
        }
      } else if constexpr (EPI == EPI_SWIGLU_BWD) {
        const int64_t r = row0 + a * 64 + q;
        if (r < row_end) {
          float sc = 1.0f;
          if (p.scale) sc = bf2f(reinterpret_cast<const uint16_t*>(p.scale)[r]);
          uint16_t* drow = reinterpret_cast<uint16_t*>(p.C) + r * (int64_t)(2 * p.h);
#pragma unroll
          for (int m = 0; m < C::BN / 32; ++m) {
            const int j = n0 + 32 * m + 8 * s;
            if (j >= p.N) continue;
            float v[8];
            ld8(32 * m, v);
            const uint4 gv = gpre[m];
            const uint4 uv = upre[m];
            const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, uw[4] = {uv.x, uv.y, uv.z, uv.w};
            float dg[8], du[8];
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const float gg = (t & 1) ? bf_hi(gw[t >> 1]) : bf_lo(gw[t >> 1]);
              const float uu = (t & 1) ? bf_hi(uw[t >> 1]) : bf_lo(uw[t >> 1]);
              const float da = v[t] * sc;
              const float sig = sigmoid_f(gg);
              du[t] = da * bf2f(f2bf(gg * sig));  // the forward's stored factor bf16(silu(g)), silu_f(g) = g*sig
              dg[t] = da * uu * sig * (1.0f + gg * (1.0f - sig));
            }
            *reinterpret_cast<uint4*>(drow + j) = pack8(dg);
            *reinterpret_cast<uint4*>(drow + p.h + j) = pack8(du);
          }
        }
      }
      lds_barrier();  // the band is reused by the next pass / the ring by the next tile
    }
  }
}

// ----------------------------------------------------------------------------------------------------------------
// Launch helpers
// ----------------------------------------------------------------------------------------------------------------
static int g_num_cus[64];

static int num_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return -1;
  if (g_num_cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return -1;
    g_num_cus[dev] = n;
  }
  return g_num_cus[dev];
}

template <class C, int MODE, bool A_MN, bool B_MN, int EPI>
static int launch(const GemmParams& p, int64_t tiles_upper, hipStream_t s) {
  auto kern = grouped_gemm_kernel<C, MODE, A_MN, B_MN, EPI>;
  static bool attr_set[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return HMOE_ERR_DEVICE;
  if (!attr_set[dev]) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            C::LDS_BYTES) != hipSuccess)
      return HMOE_ERR_LAUNCH;
    attr_set[dev] = true;
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

// large tiles once they alone give every CU at least two tiles
static inline bool pick_large(int64_t tiles_large) {
  const int f = env_force();
  if (f) return f == 1;
  const int cus = num_cus();
  return tiles_large >= 2 * (int64_t)(cus > 0 ? cus : 256);
}

template <int MODE, bool A_MN, bool B_MN, int EPI>
static int launch_mgroup(const GemmParams& p, int64_t ncols, hipStream_t s) {
  const int64_t tl = mgroup_tiles<CfgL, EPI>(p.M, p.E, ncols);
  if (pick_large(tl)) return launch<CfgL, MODE, A_MN, B_MN, EPI>(p, tl, s);
  return launch<CfgS, MODE, A_MN, B_MN, EPI>(p, mgroup_tiles<CfgS, EPI>(p.M, p.E, ncols), s);
}

static inline bool al16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

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
  if (E > kMaxEGemm) return HMOE_ERR_SHAPE;
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
  (void)w_scale_dtype;
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!a || !w || !y || K <= 0 || N <= 0) return HMOE_ERR_ARG;
  if (a_dtype != HMOE_DT_BF16 || w_dtype != HMOE_DT_BF16) return HMOE_ERR_DTYPE;
  if (w_scale) return HMOE_ERR_DTYPE;
  if (scale && scale_dtype != HMOE_DT_BF16 && scale_dtype != HMOE_DT_F32) return HMOE_ERR_DTYPE;
  if (K % 8 || N % 8 || lda % 8 || ldy % 8 || stride_wk % 8 || stride_we % 8) return HMOE_ERR_SHAPE;
  if (lda < K || ldy < N || stride_wk < N || !al16(a) || !al16(w) || !al16(y)) return HMOE_ERR_ARG;
  if (K > INT32_MAX || N > INT32_MAX || M > INT32_MAX) return HMOE_ERR_SHAPE;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.a_idx = a_idx;
  p.B = static_cast<const uint16_t*>(w);
  p.ldb = stride_wk;
  p.strideBe = stride_we;
  p.K = (int)K;
  p.N = (int)N;
  p.C = y;
  p.ldc = ldy;
  p.y_idx = y_idx;
  p.scale = scale;
  p.scale_f32 = scale_dtype == HMOE_DT_F32;
return launch_mgroup<MGROUP, false, true, EPI_STORE>(p, N, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_gate_up_swiglu(const void* x, int64_t ldx, const int32_t* a_idx, const void* wgu, int64_t E, int64_t d,
                        int64_t h, const void* counts, int counts_dtype, int64_t M, void* act, void* gu,
                        hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!x || !wgu || !act || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (d % 8 || h % 8 || ldx % 8 || ldx < d) return HMOE_ERR_SHAPE;
  if (!al16(x) || !al16(wgu) || !al16(act) || !al16(gu)) return HMOE_ERR_ARG;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(x);
  p.lda = ldx;
  p.a_idx = a_idx;
  p.B = static_cast<const uint16_t*>(wgu);
  p.ldb = 2 * h;
  p.strideBe = d * 2 * h;
  p.K = (int)d;
  p.N = (int)h;
  p.h = (int)h;
  p.C = act;
  p.ldc = h;
  p.aux = static_cast<uint16_t*>(gu);
  return launch_mgroup<MGROUP, false, true, EPI_SWIGLU>(p, h, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_down_scatter(const void* act, const void* wd, int64_t E, int64_t h, int64_t d, const void* counts,
                      int counts_dtype, int64_t M, const uint16_t* w_sorted, const int32_t* y_idx, void* y,
                      void* yhat, hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!act || !wd || !y || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (d % 8 || h % 8) return HMOE_ERR_SHAPE;
  if (!al16(act) || !al16(wd) || !al16(y) || !al16(yhat)) return HMOE_ERR_ARG;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(act);
  p.lda = h;
  p.B = static_cast<const uint16_t*>(wd);
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
  return launch_mgroup<MGROUP, false, true, EPI_STORE>(p, d, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_down_dgrad_swiglu(const void* dy, const int32_t* a_idx, const uint16_t* w_sorted, const void* wd,
                           int64_t E, int64_t h, int64_t d, const void* counts, int counts_dtype, int64_t M,
                           const void* gu, void* dgu, hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  if (M == 0) return HMOE_OK;
  if (!dy || !wd || !gu || !dgu || d <= 0 || h <= 0) return HMOE_ERR_ARG;
  if (d % 8 || h % 8) return HMOE_ERR_SHAPE;
  if (!al16(dy) || !al16(wd) || !al16(gu) || !al16(dgu)) return HMOE_ERR_ARG;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(dy);
  p.lda = d;
  p.a_idx = a_idx;
  p.B = static_cast<const uint16_t*>(wd);  // (E, h, d): row n = h index, k = d contiguous
  p.ldb = d;
  p.strideBe = h * d;
  p.K = (int)d;
  p.N = (int)h;
  p.h = (int)h;
  p.C = dgu;
  p.scale = w_sorted;
  p.gu_in = static_cast<const uint16_t*>(gu);
  return launch_mgroup<MGROUP, false, false, EPI_SWIGLU_BWD>(p, h, reinterpret_cast<hipStream_t>(stream));
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
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(dgu);
  p.lda = 2 * h;
  p.B = static_cast<const uint16_t*>(wgu);  // (E, d, 2h): row n = d index, k = 2h contiguous
  p.ldb = 2 * h;
  p.strideBe = d * 2 * h;
  p.K = (int)(2 * h);
  p.N = (int)d;
  p.C = dxs;
  p.ldc = d;
  p.c_f32 = dxs_dtype == HMOE_DT_F32;
  return launch_mgroup<MGROUP, false, false, EPI_STORE>(p, d, reinterpret_cast<hipStream_t>(stream));
}

int hmoe_grouped_wgrad(const void* a, int64_t lda, const void* b, int64_t ldb, int64_t E, int64_t P, int64_t N,
                       const void* counts, int counts_dtype, int64_t M, void* dw, int dw_dtype,
                       hmoe_stream_t stream) {
  int rc = check_common(counts, counts_dtype, E, M);
  if (rc) return rc;
  if (!a || !b || !dw || P <= 0 || N <= 0) return HMOE_ERR_ARG;
  if (dw_dtype != HMOE_DT_F32 && dw_dtype != HMOE_DT_BF16) return HMOE_ERR_DTYPE;
  if (P % 8 || N % 8 || lda % 8 || ldb % 8 || lda < P || ldb < N) return HMOE_ERR_SHAPE;
  if (!al16(a) || !al16(b) || !al16(dw)) return HMOE_ERR_ARG;
  GemmParams p = base_params(counts, counts_dtype, E, M);
  p.A = static_cast<const uint16_t*>(a);
  p.lda = lda;
  p.B = static_cast<const uint16_t*>(b);
  p.ldb = ldb;
  p.P = (int)P;
  p.N = (int)N;
  p.K = 0;
  p.C = dw;
  p.ldc = N;
  p.strideCe = P * N;
  p.c_f32 = dw_dtype == HMOE_DT_F32;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t tl = kgroup_tiles<CfgL>(E, P, N);
  if (pick_large(tl)) return launch<CfgL, KGROUP, true, true, EPI_WGRAD>(p, tl, s);
  return launch<CfgS, KGROUP, true, true, EPI_WGRAD>(p, kgroup_tiles<CfgS>(E, P, N), s);
}

}  // extern "C"
