// Building blocks of the grouped GEMM kernel (gemm.hip): tile configuration, LDS layouts and swizzles, the direct
// global -> LDS copies, barriers and wait counts, and the kernel parameter block.
#pragma once
#include "hmoe_common.h"

namespace hmoe {

constexpr int kBK = 32;      // k per LDS slice
constexpr int kNStage = 4;   // slices in flight
constexpr int kMaxEGemm = 1024;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

template <int BM_, int BN_, int WM_, int WN_, int GM_, int BE_ = 2>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, GM = GM_;
  static constexpr int BE = BE_;  // bytes per B element: 2 (bf16) or 1 (int8 weights)
  static constexpr int NWAVES = WM * WN, NT = NWAVES * 64;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 32, FN = TN / 32;
  // a wave's fragments are interleaved with the other waves' along each dimension: fragment f of wave w covers
  // 32 rows / columns from f * FS + 32 w (FS = 32 * waves along that dimension)
  static constexpr int FSM = 32 * WM, FSN = 32 * WN;
  static constexpr int A_BYTES = BM * kBK * 2, B_BYTES = BN * kBK * BE;  // per slice
  static constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
  static constexpr int LDS_BYTES = kNStage * STAGE_BYTES;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
};

// Row-group tiles ("xs tiles"): a copy of the sorted rows of A laid out as the K-major LDS image, so that each direct
// copy reads 1 KB contiguous instead of 16 rows x 64 bytes.  The sorted rows of expert e form groups of 128 rows
// (the last one partial); group g of all experts (expert e's first is gstart[e] = sum over e' < e of
// ceil(count[e'] / 128)) and 32-wide k-slice s occupy the 8 KB at (g * nslices + s) * 8 KB, nslices = ceil(K / 32):
// row r of the group at r * 64 bytes, its logical 16-byte chunk c at physical chunk c ^ swz_k(r).  A 256-row tile
// reads two consecutive groups, a 128-row tile one (tiles start at multiples of 64 rows of an expert; the swizzle
// uses bits 2-3 of the row only, so any 16-row run of a group is a valid piece of a tile's image).
static_assert(kTileK == kBK, "row-group tiles hold one LDS slice per 32 k");
constexpr int kTileSliceBytes = kTileGroupRows * kBK * 2;

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

// ----------------------------------------------------------------------------------------------------------------
// Direct global -> LDS copies through buffer loads.  Each operand tile has a wave-uniform buffer descriptor whose
// base is the tile's (or expert's) origin; a lane's 32-bit byte offset inside it is fixed for the whole tile and the
// k-slice advance is the uniform scalar offset, so a slice costs one scalar add per operand plus one instruction
// per copy.  Lanes whose source lies outside the operand (ragged expert ends, N tails, K tails) use an offset of
// 2^31, beyond the descriptor's range: the hardware returns zeros for them and writes those zeros to LDS, so every
// LDS slot is written each slice.  Offsets of real data must stay below 2^31 - 16 bytes from the base (checked on the
// host).
// ----------------------------------------------------------------------------------------------------------------
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOOB = 0x80000000u;

__device__ __forceinline__ i32x4 make_rsrc(const void* base) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  // the base is the same for every lane; readfirstlane tells the compiler so, which puts the descriptor in SGPRs
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));  // base[47:32]; stride 0, no swizzle
  r.z = 0x7FFFFFF0;                // range in bytes (offsets at or above it read zeros)
  r.w = 0x00020000;                // 32-bit data format: a raw dword buffer
  return r;
}

// 16 bytes per lane from base + voff + soff into LDS at lds + 16 * lane (lds is wave-uniform; it goes to M0).
// Issued as inline asm so the compiler does not guard every later LDS read with a vmcnt(0) wait for it: completion
// of these copies is tracked explicitly (wait_vm + barrier before a slice is read).
// Wait states: a vector memory instruction that reads an SGPR written by a VALU instruction (v_readfirstlane of a
// descriptor word, the reload of a spilled SGPR) needs 5 wait states after that write, and a write of M0 needs 1
// before the LDS-bound load reads it.  The compiler provides neither for inline asm, so the s_nop 4 after the M0
// write covers both.
// The scalar operands go through readfirstlane: they are wave-uniform, but a value the compiler spilled comes back in
// a VGPR (where the value is already in an SGPR this folds away).
__device__ __forceinline__ void buf2lds(uint32_t voff, i32x4 rsrc, uint32_t soff, char* lds) {
  const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane(
      (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)(lds));
  rsrc.x = __builtin_amdgcn_readfirstlane(rsrc.x);
  rsrc.y = __builtin_amdgcn_readfirstlane(rsrc.y);
  rsrc.z = __builtin_amdgcn_readfirstlane(rsrc.z);
  rsrc.w = __builtin_amdgcn_readfirstlane(rsrc.w);
  soff = (uint32_t)__builtin_amdgcn_readfirstlane((int)soff);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 4\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(m0), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}

// K-major operand: ROWS rows x 32 k per slice; ROWS/16 copy instructions per slice (each 16 rows x 64 bytes),
// spread over the workgroup's waves.
template <int ROWS, int NWAVES>
struct KTile {
  static constexpr int INSTR = ROWS / 16;
  static constexpr int PER_WAVE = INSTR / NWAVES;
  static_assert(INSTR % NWAVES == 0, "K tile copy instructions must divide over the waves");
  uint32_t voff[PER_WAVE];  // byte offset of (row, k = 8 * chunk) from the base, or kOOB
  int chunk[PER_WAVE];      // logical k-chunk this lane copies
  i32x4 rsrc;
  int K;
  uint32_t kmul = 2;  // scalar-offset bytes per k: 2 (rows of A), 256 (row-group tiles: 8 KB per 32-k slice)
  // lane l of instruction (wave w, i) fills LDS row 16*(w*PER_WAVE + i) + l/4, physical chunk l%4
  __device__ __forceinline__ static int row_of(int wave, int lane, int i) { return 16 * (wave * PER_WAVE + i) + lane / 4; }
  __device__ __forceinline__ void issue(char* lds_tile, int wave, int lane, int k0) const {
    const uint32_t soff = (uint32_t)k0 * kmul;
    if (k0 + kBK <= K) {
#pragma unroll
      for (int i = 0; i < PER_WAVE; ++i) buf2lds(voff[i], rsrc, soff, lds_tile + (wave * PER_WAVE + i) * 1024);
    } else {  // K tail: chunks at or past K read zeros
#pragma unroll
      for (int i = 0; i < PER_WAVE; ++i)
        buf2lds(k0 + chunk[i] * 8 < K ? voff[i] : kOOB, rsrc, soff, lds_tile + (wave * PER_WAVE + i) * 1024);
    }
  }
  // the i-th of issue()'s copies alone (the caller spreads them between MFMAs)
  __device__ __forceinline__ void issue_one(char* lds_tile, int wave, int i, int k0) const {
    const uint32_t vo = (k0 + kBK <= K || k0 + chunk[i] * 8 < K) ? voff[i] : kOOB;
    buf2lds(vo, rsrc, (uint32_t)k0 * kmul, lds_tile + (wave * PER_WAVE + i) * 1024);
  }
  // the same for a slice known to lie inside K (no tail test)
  __device__ __forceinline__ void issue_one_full(char* lds_tile, int wave, int i, int k0) const {
    buf2lds(voff[i], rsrc, (uint32_t)k0 * kmul, lds_tile + (wave * PER_WAVE + i) * 1024);
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
  uint32_t voff[PER_WAVE];  // byte offset of (k-row, first of the lane's 8 columns) from the base, or kOOB
  int krow[PER_WAVE];       // k-row within the slice
  i32x4 rsrc;
  uint32_t kstep;           // bytes per k-row (ld * 2)
  int Kvalid;
  __device__ __forceinline__ void issue(char* lds_tile, int wave, int lane, int k0) const {
    const uint32_t soff = (uint32_t)k0 * kstep;
    if (k0 + kBK <= Kvalid) {
#pragma unroll
      for (int i = 0; i < PER_WAVE; ++i) buf2lds(voff[i], rsrc, soff, lds_tile + (wave * PER_WAVE + i) * 1024);
    } else {  // K tail: k-rows at or past Kvalid read zeros
#pragma unroll
      for (int i = 0; i < PER_WAVE; ++i)
        buf2lds(k0 + krow[i] < Kvalid ? voff[i] : kOOB, rsrc, soff, lds_tile + (wave * PER_WAVE + i) * 1024);
    }
  }
  __device__ __forceinline__ void issue_one(char* lds_tile, int wave, int i, int k0) const {
    const uint32_t vo = (k0 + kBK <= Kvalid || k0 + krow[i] < Kvalid) ? voff[i] : kOOB;
    buf2lds(vo, rsrc, (uint32_t)k0 * kstep, lds_tile + (wave * PER_WAVE + i) * 1024);
  }
  __device__ __forceinline__ void issue_one_full(char* lds_tile, int wave, int i, int k0) const {
    buf2lds(voff[i], rsrc, (uint32_t)k0 * kstep, lds_tile + (wave * PER_WAVE + i) * 1024);
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

// MFMA on one k16 step of 16-bit fragments (8 elements per lane, bf16 or fp16 bits), fp32 accumulation
template <bool F16>
__device__ __forceinline__ f32x16 mfma16(bf16x8 a, bf16x8 b, f32x16 c) {
  if constexpr (F16) {
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                   0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
}

// int8 MN-major operand (weights (K, N), N contiguous, as int8): 32 k-rows x ROWS columns = ROWS bytes per k-row.
// Each 16-byte chunk holds 16 columns.  Logical chunk c = 4b + 2wn + h of a k-row (fragment b of wave column wn,
// half h of its 32 columns) is stored at b + FN*((2wn + h) ^ (k & 3)), so the k-rows a transpose read touches spread
// over the banks while fragment b stays a compile-time offset.
template <int ROWS, int NWAVES, int FN, bool F16 = false>
struct MNTile8 {
  static constexpr int INSTR = ROWS * kBK / 1024;
  static constexpr int PER_WAVE = INSTR / NWAVES;
  static constexpr int CPR = ROWS / 16;  // 16-byte chunks per k-row
  static constexpr int KPI = 64 / CPR;   // k-rows per copy instruction
  static_assert(INSTR % NWAVES == 0 && CPR == 4 * FN, "int8 tile: 4 chunks per fragment column group");
  uint32_t voff[PER_WAVE];  // byte offset of (k-row, first of the lane's 16 columns) from the base, or kOOB
  int krow[PER_WAVE];
  i32x4 rsrc;
  uint32_t kstep;  // bytes per k-row (ld)
  int Kvalid;
  __device__ __forceinline__ void issue(char* lds_tile, int wave, int lane, int k0) const {
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) issue_one(lds_tile, wave, i, k0);
  }
  __device__ __forceinline__ void issue_one(char* lds_tile, int wave, int i, int k0) const {
    const uint32_t vo = (k0 + kBK <= Kvalid || k0 + krow[i] < Kvalid) ? voff[i] : kOOB;
    buf2lds(vo, rsrc, (uint32_t)k0 * kstep, lds_tile + (wave * PER_WAVE + i) * 1024);
  }
  __device__ __forceinline__ void issue_one_full(char* lds_tile, int wave, int i, int k0) const {
    buf2lds(voff[i], rsrc, (uint32_t)k0 * kstep, lds_tile + (wave * PER_WAVE + i) * 1024);
  }
  // lane l of instruction (wave w, i): k-row (w*PER_WAVE + i)*KPI + l / CPR, physical chunk l % CPR; col = the first
  // logical column the slot holds
  __device__ __forceinline__ static void slot(int wave, int lane, int i, int& k, int& col) {
    k = (wave * PER_WAVE + i) * KPI + lane / CPR;
    const int pp = lane % CPR, b = pp % FN, q = (pp / FN) ^ (k & 3);
    col = (4 * b + q) * 16;
  }
  // Transpose read (ds_read_b64_tr_b8): lane l = 16G + 8h + c receives byte c of the 8 lanes 16G + h + 2m, m = 0..7.
  // Lane S therefore points at k-row (S/32)*8 + (S%16)/2 and column 16*((S/16)%2) + 8*(S%2) of the fragment, so
  // lane l ends with column l%32 and the 8 consecutive k (l/32)*8 + 0..7 of it.
  __device__ __forceinline__ static int lane_off(int w32, int lane) {
    const int kr = (lane >> 5) * 8 + ((lane & 15) >> 1);
    const int h = (lane >> 4) & 1;
    return kr * ROWS + 16 * FN * ((2 * w32 + h) ^ (kr & 3)) + 8 * (lane & 1);
  }
  // fragment b (columns b*FSN + 32 w32 + 0..31) x 16 k (ks*16 + ...), converted exactly to bf16 (fp16 with F16)
  __device__ __forceinline__ static bf16x8 frag(const char* lds_tile, int grp64, int loff, int ks) {
    typedef int i32x2 __attribute__((ext_vector_type(2)));
    typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
    const int b = grp64 / 64;
    const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(lds_tile + loff + ks * 16 * ROWS + 16 * b));
    // signed bytes -> exact floats (|q| <= 128 has at most 8 significant bits) -> bf16; each byte converts in one
    // instruction (a sign-extending byte select on the int -> float conversion)
    const uint32_t lo = (uint32_t)v[0], hi = (uint32_t)v[1];
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[j] = (float)(int8_t)(lo >> (8 * j));
      f[4 + j] = (float)(int8_t)(hi >> (8 * j));
    }
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    using X = Elt<F16>;
    const u32x4 w = {X::pack2(f[0], f[1]), X::pack2(f[2], f[3]), X::pack2(f[4], f[5]), X::pack2(f[6], f[7])};
    return __builtin_bit_cast(bf16x8, w);
  }
};

template <bool MN, int ROWS, int NWAVES, int ES = 2, int FN = 4, bool F16 = false>
struct TileSel;
template <int ROWS, int NWAVES, int FN, bool F16>
struct TileSel<false, ROWS, NWAVES, 2, FN, F16> {
  using type = KTile<ROWS, NWAVES>;
};
template <int ROWS, int NWAVES, int FN, bool F16>
struct TileSel<true, ROWS, NWAVES, 2, FN, F16> {
  using type = MNTile<ROWS, NWAVES>;
};
template <int ROWS, int NWAVES, int FN, bool F16>
struct TileSel<true, ROWS, NWAVES, 1, FN, F16> {
  using type = MNTile8<ROWS, NWAVES, FN, F16>;
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

// Pins an accumulator fragment in AGPRs up to this point of the program.  Without it the register allocator may copy
// every accumulator to VGPRs at the end of the main loop (256 values: a spill); with it each fragment is read out of
// the AGPRs only where the epilogue uses it.  The empty asm counts as the fragment's last writer, so the MFMA -> VALU
// read wait states must be provided explicitly after the main loop (see the kernel).
__device__ __forceinline__ void pin_agpr(f32x16& v) { asm volatile("" : "+a"(v)); }

// ----------------------------------------------------------------------------------------------------------------
// Kernel parameters
// ----------------------------------------------------------------------------------------------------------------
enum Mode { MGROUP = 0, KGROUP = 1 };
enum Epi { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_SWIGLU_BWD = 2, EPI_WGRAD = 3, EPI_STORE_F32 = 4 };

struct GemmParams {
  // M side (A).  MGROUP: rows of A (sorted row r, or a_idx[r] when gather), K contiguous, row stride lda.
  //              KGROUP: X (M, P) with P contiguous, row stride lda.
  const uint16_t* A;
  int64_t lda;
  const int32_t* a_idx;
  // N side (B).  MGROUP: weights of expert e at B + e*strideBe; B_MN: element (k, n) at k*ldb + n, else n*ldb + k.
  //              KGROUP: Y (M, N) with N contiguous, row stride ldb.
  const void* B;             // bf16, or int8 weights (with w_scale)
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
  const void* scale;        // EPI_STORE / EPI_SWIGLU_BWD per-row scale: fp32, or the activations' 16-bit type
  int scale_f32;
  uint16_t* aux;            // EPI_STORE: yhat (unscaled, sorted); EPI_SWIGLU: gu store
  const uint16_t* gu_in;    // EPI_SWIGLU_BWD: [g | u]
  float* dw_part;           // EPI_SWIGLU_BWD: (partial, row) array of the routing-weight gradient's partials, or NULL
  int dw_ld;                //   partials per row: 2 per n-tile (one per wave column)
  const void* w_scale;      // int8 weights: per-(expert, column) scale (E, ldws), bf16 or fp32
  int w_scale_f32;
  int64_t ldws;             // scale row length (columns of the weight)
};

}  // namespace hmoe
