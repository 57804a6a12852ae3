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
// groups GROUP_M m-tiles per band so A rows and B columns are reused from the XCD's L2.
//
// Tiles are staged through LDS as [rows][64] bf16 (k contiguous, 16-byte chunks XOR-swizzled per row) in two
// buffers: the next k-tile's global loads are in flight while MFMAs run on the current one, one barrier per k-tile.
// Operands whose k index is strided in memory (weights stored (K, N) with N contiguous; the row-major activations
// of a weight gradient) are loaded as 8x8 bf16 blocks and transposed in registers before the LDS store.
//
// MFMA roles: the N-side tile feeds the MFMA "A" operand and the M-side tile the "B" operand, so each lane's
// accumulator holds one output row and 4 consecutive output columns per group -> 8-byte bf16 / 16-byte fp32 stores.
#include "hmoe_common.h"

namespace hmoe {

constexpr int kBK = 64;
constexpr int kKCH = kBK / 8;  // 16-byte chunks per LDS row
constexpr int kMaxEGemm = 1024;

__device__ __forceinline__ int lds_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int lds_idx(int row, int kc) { return row * kKCH + (kc ^ lds_swz(row)); }

template <int BM_, int BN_, int WM_, int WN_, int GM_>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, GM = GM_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 32, FN = TN / 32;
  static constexpr int LDS_A = BM * kKCH, LDS_B = BN * kKCH;  // uint4 per stage
  static constexpr int LDS_BYTES = 2 * (LDS_A + LDS_B) * 16;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
};

// ----------------------------------------------------------------------------------------------------------------
// Operand loaders.  A loader owns a tile of ROWS rows (the M or N side) x 64 k; it is initialised per tile with
// row / column pointers and masks, then load(k0) issues the global reads into registers and store() writes LDS.
// ----------------------------------------------------------------------------------------------------------------

// K-contiguous source: row p at base_p, elements k contiguous.
template <int ROWS, int NT>
struct LoadK {
  static constexpr int PER = ROWS * kKCH / NT;
  static_assert(ROWS * kKCH % NT == 0, "K loader: rows*8 must be a multiple of the thread count");
  static constexpr int RSTEP = NT / kKCH;
  const uint16_t* base[PER];
  uint4 r[PER];
  int kc, row0;
  __device__ __forceinline__ void set_thread(int tid) {
    kc = tid % kKCH;
    row0 = tid / kKCH;
  }
  __device__ __forceinline__ int row(int i) const { return row0 + i * RSTEP; }
  __device__ __forceinline__ void load(int k0, int K) {
    const int kk = k0 + kc * 8;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (base[i] != nullptr && kk < K)
        r[i] = *reinterpret_cast<const uint4*>(base[i] + kk);
      else
        r[i] = make_uint4(0, 0, 0, 0);
    }
  }
  __device__ __forceinline__ void store(uint4* lds) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) lds[lds_idx(row(i), kc)] = r[i];
  }
};

// MN-contiguous source: element (k, p) at col_p + k * ld (8 consecutive p per 16-byte load).  Each thread loads an
// 8 (k) x 8 (p) block and transposes it in registers.
template <int ROWS, int NT>
struct LoadMN {
  static constexpr int BLOCKS = (ROWS / 8) * kKCH;
  static constexpr int PER = (BLOCKS + NT - 1) / NT;
  const uint16_t* col[PER];  // pointer to (k = 0, p = first of the 8 columns); nullptr -> zeros
  uint4 r[PER][8];
  int kc[PER], ng[PER];
  bool act[PER];
  int64_t ld;
  __device__ __forceinline__ void set_thread(int tid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int q = tid + i * NT;
      act[i] = q < BLOCKS;
      kc[i] = q % kKCH;
      ng[i] = q / kKCH;
    }
  }
  __device__ __forceinline__ void load(int k0, int Kvalid) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        const int krow = k0 + kc[i] * 8 + kk;
        if (act[i] && col[i] != nullptr && krow < Kvalid)
          r[i][kk] = *reinterpret_cast<const uint4*>(col[i] + (int64_t)krow * ld);
        else
          r[i][kk] = make_uint4(0, 0, 0, 0);
      }
    }
  }
  __device__ __forceinline__ static uint32_t w(const uint4& v, int j) {
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
  }
  __device__ __forceinline__ static uint32_t pk(uint32_t lo_src, uint32_t hi_src, bool odd) {
    return odd ? ((lo_src >> 16) | (hi_src & 0xffff0000u)) : ((lo_src & 0xffffu) | (hi_src << 16));
  }
  __device__ __forceinline__ void store(uint4* lds) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (!act[i]) continue;
#pragma unroll
      for (int nn = 0; nn < 8; ++nn) {
        const int j = nn >> 1;
        const bool odd = nn & 1;
        uint4 o;
        o.x = pk(w(r[i][0], j), w(r[i][1], j), odd);
        o.y = pk(w(r[i][2], j), w(r[i][3], j), odd);
        o.z = pk(w(r[i][4], j), w(r[i][5], j), odd);
        o.w = pk(w(r[i][6], j), w(r[i][7], j), odd);
        lds[lds_idx(ng[i] * 8 + nn, kc[i])] = o;
      }
    }
  }
};

template <bool MN, int ROWS, int NT>
struct LoaderSel;
template <int ROWS, int NT>
struct LoaderSel<false, ROWS, NT> {
  using type = LoadK<ROWS, NT>;
};
template <int ROWS, int NT>
struct LoaderSel<true, ROWS, NT> {
  using type = LoadMN<ROWS, NT>;
};

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
  // N side (B).  MGROUP: weights of expert e at B + e*strideBe; b_mn: element (k, n) at k*ldb + n, else n*ldb + k.
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
  int c_f32;                // EPI_WGRAD: fp32 output
  const int32_t* y_idx;     // EPI_STORE scatter
  const void* scale;        // EPI_STORE per-row scale
  int scale_f32;
  uint16_t* aux;            // EPI_STORE: yhat (unscaled, sorted); EPI_SWIGLU: gu store
  const uint16_t* gu_in;    // EPI_SWIGLU_BWD: [g | u]
};

// ----------------------------------------------------------------------------------------------------------------
// The kernel
// ----------------------------------------------------------------------------------------------------------------
template <class C, int MODE, bool A_MN, bool B_MN, int EPI>
__global__ __launch_bounds__(C::NT, 1) void grouped_gemm_kernel(GemmParams p) {
  extern __shared__ uint4 smem[];
  uint4* As = smem;                      // [2][LDS_A]
  uint4* Bs = smem + 2 * C::LDS_A;       // [2][LDS_B]
  __shared__ int64_t s_rstart[kMaxEGemm + 1];
  __shared__ int s_tstart[kMaxEGemm + 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
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
  __syncthreads();

  int nb_n;
  if (EPI == EPI_SWIGLU)
    nb_n = (p.N + C::BN / 2 - 1) / (C::BN / 2);
  else
    nb_n = (p.N + C::BN - 1) / C::BN;
  const int nb_i = MODE == KGROUP ? (p.P + C::BM - 1) / C::BM : 1;
  const int total_m = MODE == MGROUP ? s_tstart[E] : E * nb_i;
  const int total = total_m * nb_n;

  typename LoaderSel<A_MN, C::BM, C::NT>::type la;
  typename LoaderSel<B_MN, C::BN, C::NT>::type lb;
  la.set_thread(tid);
  lb.set_thread(tid);

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
      while (e + 1 < E && s_tstart[e + 1] <= mt) ++e;
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

    // ---- operand pointers ----
    if constexpr (MODE == MGROUP) {
      // A: K-contiguous rows (gathered or sorted)
      static_assert(!A_MN, "MGROUP A is K-contiguous");
#pragma unroll
      for (int i = 0; i < la.PER; ++i) {
        const int64_t r = row0 + la.row(i);
        const uint16_t* ptr = nullptr;
        if (r < row_end) {
          const int64_t src = p.a_idx ? (int64_t)p.a_idx[r] : r;
          ptr = p.A + src * p.lda;
        }
        la.base[i] = ptr;
      }
      const uint16_t* Be = p.B + (int64_t)e * p.strideBe;
      auto gcol = [&](int nn, int& col) -> bool {  // tile column -> weight column
        if (EPI == EPI_SWIGLU) {
          const int wnn = nn / C::TN, c = nn % C::TN;
          const int half = c / (C::TN / 2), j = c % (C::TN / 2);
          const int ac = n0 + wnn * (C::TN / 2) + j;
          col = half * p.h + ac;
          return ac < p.N;
        } else {
          col = n0 + nn;
          return col < p.N;
        }
      };
      if constexpr (B_MN) {
        lb.ld = p.ldb;
#pragma unroll
        for (int i = 0; i < lb.PER; ++i) {
          int col;
          const bool ok = gcol(lb.ng[i] * 8, col);
          lb.col[i] = ok ? Be + col : nullptr;
        }
      } else {
#pragma unroll
        for (int i = 0; i < lb.PER; ++i) {
          int col;
          const bool ok = gcol(lb.row(i), col);
          lb.base[i] = ok ? Be + (int64_t)col * p.ldb : nullptr;
        }
      }
    } else {
      static_assert(A_MN && B_MN, "KGROUP operands are MN-contiguous");
      la.ld = p.lda;
      lb.ld = p.ldb;
#pragma unroll
      for (int i = 0; i < la.PER; ++i) {
        const int ic = i0 + la.ng[i] * 8;
        la.col[i] = ic < p.P ? p.A + kstart * p.lda + ic : nullptr;
      }
#pragma unroll
      for (int i = 0; i < lb.PER; ++i) {
        const int nc = n0 + lb.ng[i] * 8;
        lb.col[i] = nc < p.N ? p.B + kstart * p.ldb + nc : nullptr;
      }
    }

    // ---- main loop ----
    f32x16 acc[C::FM][C::FN];
#pragma unroll
    for (int a = 0; a < C::FM; ++a)
#pragma unroll
      for (int b = 0; b < C::FN; ++b)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[a][b][v] = 0.0f;

    const int nk = (kvalid + kBK - 1) / kBK;
    if (nk > 0) {
      la.load(0, kvalid);
      lb.load(0, kvalid);
      la.store(As);
      lb.store(Bs);
      __syncthreads();
      for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) {
          la.load((kt + 1) * kBK, kvalid);
          lb.load((kt + 1) * kBK, kvalid);
        }
        const uint4* Ac = As + cur * C::LDS_A;
        const uint4* Bc = Bs + cur * C::LDS_B;
#pragma unroll
        for (int ks = 0; ks < kBK / 16; ++ks) {
          const int kc = ks * 2 + (lane >> 5);
          bf16x8 xa[C::FM], wb[C::FN];
#pragma unroll
          for (int a = 0; a < C::FM; ++a) {
            const uint4 v = Ac[lds_idx(wm * C::TM + a * 32 + (lane & 31), kc)];
            xa[a] = __builtin_bit_cast(bf16x8, v);
          }
#pragma unroll
          for (int b = 0; b < C::FN; ++b) {
            const uint4 v = Bc[lds_idx(wn * C::TN + b * 32 + (lane & 31), kc)];
            wb[b] = __builtin_bit_cast(bf16x8, v);
          }
#pragma unroll
          for (int a = 0; a < C::FM; ++a)
#pragma unroll
            for (int b = 0; b < C::FN; ++b)
              acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wb[b], xa[a], acc[a][b], 0, 0, 0);
        }
        if (kt + 1 < nk) {
          la.store(As + (cur ^ 1) * C::LDS_A);
          lb.store(Bs + (cur ^ 1) * C::LDS_B);
        }
        __syncthreads();
      }
    }

    // ---- epilogue ----
    // lane holds, for fragment (a, b) and group g: row m = wm*TM + a*32 + (lane&31), columns
    // n = wn*TN + b*32 + 8g + 4*(lane>>5) + {0..3}
    const int lrow = lane & 31;
    const int lcol = 4 * (lane >> 5);
    if constexpr (EPI == EPI_WGRAD) {
#pragma unroll
      for (int a = 0; a < C::FM; ++a) {
        const int i = i0 + wm * C::TM + a * 32 + lrow;
        if (i >= p.P) continue;
        char* crow = reinterpret_cast<char*>(p.C) +
                     ((int64_t)e * p.strideCe + (int64_t)i * p.ldc) * (p.c_f32 ? 4 : 2);
#pragma unroll
        for (int b = 0; b < C::FN; ++b)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn * C::TN + b * 32 + 8 * g + lcol;
            if (n >= p.N) continue;
            const float v0 = acc[a][b][4 * g], v1 = acc[a][b][4 * g + 1], v2 = acc[a][b][4 * g + 2],
                        v3 = acc[a][b][4 * g + 3];
            if (p.c_f32)
              *reinterpret_cast<float4*>(crow + (int64_t)n * 4) = make_float4(v0, v1, v2, v3);
            else
              *reinterpret_cast<uint2*>(crow + (int64_t)n * 2) = make_uint2(pack_bf2(v0, v1), pack_bf2(v2, v3));
          }
      }
    } else if constexpr (EPI == EPI_STORE) {
#pragma unroll
      for (int a = 0; a < C::FM; ++a) {
        const int64_t r = row0 + wm * C::TM + a * 32 + lrow;
        if (r >= row_end) continue;
        float sc = 1.0f;
        if (p.scale) sc = p.scale_f32 ? reinterpret_cast<const float*>(p.scale)[r]
                                      : bf2f(reinterpret_cast<const uint16_t*>(p.scale)[r]);
        const int64_t yr = p.y_idx ? (int64_t)p.y_idx[r] : r;
        uint16_t* yrow = reinterpret_cast<uint16_t*>(p.C) + yr * p.ldc;
        float* yrow32 = reinterpret_cast<float*>(p.C) + yr * p.ldc;
        uint16_t* hrow = p.aux ? p.aux + r * p.ldc : nullptr;
#pragma unroll
        for (int b = 0; b < C::FN; ++b)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int n = n0 + wn * C::TN + b * 32 + 8 * g + lcol;
            if (n >= p.N) continue;
            float v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = acc[a][b][4 * g + q];
            if (hrow) *reinterpret_cast<uint2*>(hrow + n) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
            if (p.scale) {
#pragma unroll
              for (int q = 0; q < 4; ++q) v[q] = v[q] * sc;
            }
            if (p.c_f32)
              *reinterpret_cast<float4*>(yrow32 + n) = make_float4(v[0], v[1], v[2], v[3]);
            else
              *reinterpret_cast<uint2*>(yrow + n) = make_uint2(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]));
          }
      }
    } else if constexpr (EPI == EPI_SWIGLU) {
      // fragments b < FN/2 hold gate columns, b + FN/2 the matching up columns
#pragma unroll
      for (int a = 0; a < C::FM; ++a) {
        const int64_t r = row0 + wm * C::TM + a * 32 + lrow;
        if (r >= row_end) continue;
        uint16_t* arow = reinterpret_cast<uint16_t*>(p.C) + r * p.ldc;
        uint16_t* grow = p.aux ? p.aux + r * (int64_t)(2 * p.h) : nullptr;
#pragma unroll
        for (int b = 0; b < C::FN / 2; ++b)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int j = n0 + wn * (C::TN / 2) + b * 32 + 8 * g + lcol;
            if (j >= p.N) continue;
            uint32_t gb[4], ub[4];
            float o[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              gb[q] = f2bf(acc[a][b][4 * g + q]);
              ub[q] = f2bf(acc[a][b + C::FN / 2][4 * g + q]);
              const float s = bf2f(f2bf(silu_f(bf2f(gb[q]))));
              o[q] = s * bf2f(ub[q]);
            }
            *reinterpret_cast<uint2*>(arow + j) = make_uint2(pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3]));
            if (grow) {
              *reinterpret_cast<uint2*>(grow + j) = make_uint2(gb[0] | (gb[1] << 16), gb[2] | (gb[3] << 16));
              *reinterpret_cast<uint2*>(grow + p.h + j) = make_uint2(ub[0] | (ub[1] << 16), ub[2] | (ub[3] << 16));
            }
          }
      }
    } else if constexpr (EPI == EPI_SWIGLU_BWD) {
#pragma unroll
      for (int a = 0; a < C::FM; ++a) {
        const int64_t r = row0 + wm * C::TM + a * 32 + lrow;
        if (r >= row_end) continue;
        float sc = 1.0f;
        if (p.scale) sc = bf2f(reinterpret_cast<const uint16_t*>(p.scale)[r]);
        const uint16_t* gurow = p.gu_in + r * (int64_t)(2 * p.h);
        uint16_t* drow = reinterpret_cast<uint16_t*>(p.C) + r * (int64_t)(2 * p.h);
#pragma unroll
        for (int b = 0; b < C::FN; ++b)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int j = n0 + wn * C::TN + b * 32 + 8 * g + lcol;
            if (j >= p.N) continue;
            const uint2 gv = *reinterpret_cast<const uint2*>(gurow + j);
            const uint2 uv = *reinterpret_cast<const uint2*>(gurow + p.h + j);
            const float gg[4] = {bf_lo(gv.x), bf_hi(gv.x), bf_lo(gv.y), bf_hi(gv.y)};
            const float uu[4] = {bf_lo(uv.x), bf_hi(uv.x), bf_lo(uv.y), bf_hi(uv.y)};
            float dg[4], du[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float da = acc[a][b][4 * g + q] * sc;
              const float sig = 1.0f / (1.0f + __expf(-gg[q]));
              const float s = gg[q] * sig;
              du[q] = da * s;
              dg[q] = da * uu[q] * sig * (1.0f + gg[q] * (1.0f - sig));
            }
            *reinterpret_cast<uint2*>(drow + j) = make_uint2(pack_bf2(dg[0], dg[1]), pack_bf2(dg[2], dg[3]));
            *reinterpret_cast<uint2*>(drow + p.h + j) = make_uint2(pack_bf2(du[0], du[1]), pack_bf2(du[2], du[3]));
          }
      }
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
  int64_t grid = cus;  // one workgroup per CU (LDS-limited)
  if (tiles_upper < grid) grid = tiles_upper;
  if (grid < 1) grid = 1;
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(C::NT), C::LDS_BYTES, s, p);
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

// Tile configurations.  Large: 256 (rows) x 128 (cols) tile, 4 waves of 128x64 (FM = 4, FN = 2: 128 fp32
// accumulators per lane).  Small: 128x128, 4 waves of 64x64, for problems with few tiles.
using CfgL = Cfg<256, 128, 2, 2, 4>;
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
