// Routing, dispatch (stable counting sort + row permutation), schedule and combine kernels, with their C entry
// points.  HBM-bound integer/byte work: vectorised 16-byte row copies, wave ballots for the stable ranks.
#include "hmoe_common.h"

#include <atomic>

namespace hmoe {

// ---------------------------------------------------------------------------------------------------------------
// Router: logits in the documented order, softmax, top-k, renormalisation.  One wave per token.
// ---------------------------------------------------------------------------------------------------------------
constexpr int kRouteMaxE = 256;  // experts per lane: 4
constexpr int kRouteEPL = kRouteMaxE / 64;
constexpr int kMaxK = 16;

// wave-wide argmax of (value, index): larger value wins, equal values go to the lower index; an index of 0x7fffffff
// marks an empty candidate.  The winner is unique, so any exchange pattern gives every lane the same result.
__device__ __forceinline__ void argmax_take(float& bv, int& be, float ov, int oe) {
  const bool take = oe != 0x7fffffff && (be == 0x7fffffff || ov > bv || (ov == bv && oe < be));
  if (take) {
    bv = ov;
    be = oe;
  }
}
__device__ __forceinline__ void wave_argmax(float& bv, int& be) {
  {
    float a0, a1, e0, e1;
    lane_swap<32>(bv, bv, a0, a1);
    lane_swap<32>(__int_as_float(be), __int_as_float(be), e0, e1);
    bv = a0; be = __float_as_int(e0);
    argmax_take(bv, be, a1, __float_as_int(e1));
  }
  {
    float a0, a1, e0, e1;
    lane_swap<16>(bv, bv, a0, a1);
    lane_swap<16>(__int_as_float(be), __int_as_float(be), e0, e1);
    bv = a0; be = __float_as_int(e0);
    argmax_take(bv, be, a1, __float_as_int(e1));
  }
  argmax_take(bv, be, lane_xor<8>(bv), lane_xor_i<8>(be));
  argmax_take(bv, be, lane_xor<4>(bv), lane_xor_i<4>(be));
  argmax_take(bv, be, lane_xor<2>(bv), lane_xor_i<2>(be));
  argmax_take(bv, be, lane_xor<1>(bv), lane_xor_i<1>(be));
}

// one arg-max exchange step over lanes l ^ S inside 16-lane rows, carrying a payload (argmax_take's rule)
template <int S>
__device__ __forceinline__ void seg_argmax_step(float& bv, int& be, float& bp) {
  const float ov = lane_xor<S>(bv), op = lane_xor<S>(bp);
  const int oe = lane_xor_i<S>(be);
  if (oe != 0x7fffffff && (be == 0x7fffffff || ov > bv || (ov == bv && oe < be))) {
    bv = ov;
    be = oe;
    bp = op;
  }
}

// Softmax selection for one token from its E logits held lane-wise (lane l: experts l, l + 64, ...), bias already
// in the logits: m = max logit, ex = hexp(logit - m), S = their sum by the xor butterfly (lane l holding experts l,
// l + 64, ...), probabilities ex / S; selection on the logits (descending, ties to the lower expert); weights the
// selected probabilities, renormalised (w / (sum + 1e-20)) and scaled.  `logits` receives the logits.
__device__ __forceinline__ void route_select(const float (&lg)[kRouteEPL], int t, int lane, int E, int k, int renorm,
                                             float scaling, float* __restrict__ logits, int32_t* __restrict__ ids,
                                             float* __restrict__ wout) {
#pragma clang fp contract(off)
    // key[i]: the selection key of expert i*64 + lane; num[i]: the value its weight is made of (divided by S)
    float key[kRouteEPL], num[kRouteEPL];
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < kRouteEPL; ++i)
      if (i * 64 + lane < E) m = fmaxf(m, lg[i]);
    m = wave_max_butterfly(m);
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < kRouteEPL; ++i) {
      num[i] = 0.0f;
      key[i] = lg[i];
      if (i * 64 + lane < E) {
        num[i] = hexp(__fsub_rn(lg[i], m));
        a = __fadd_rn(a, num[i]);
      }
    }
    const float S = wave_sum_butterfly(a);
    if (logits) {
#pragma unroll
      for (int i = 0; i < kRouteEPL; ++i)
        if (i * 64 + lane < E) logits[(int64_t)t * E + i * 64 + lane] = lg[i];
    }
    bool taken[kRouteEPL];
#pragma unroll
    for (int i = 0; i < kRouteEPL; ++i) taken[i] = false;
    float selp[kMaxK];
    int sele[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      selp[j] = 0.0f;
      sele[j] = 0;
      if (j < k) {
        float bv = 0.0f;
        int be = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < kRouteEPL; ++i) {
          int e = i * 64 + lane;
          if (e < E && !taken[i] && (be == 0x7fffffff || key[i] > bv)) {
            bv = key[i];
            be = e;
          }
        }
        wave_argmax(bv, be);
        float mynum = 0.0f;
#pragma unroll
        for (int i = 0; i < kRouteEPL; ++i)
          if (be == i * 64 + lane) {
            taken[i] = true;
            mynum = num[i];
          }
        const float pnum = __shfl(mynum, be & 63, 64);
        selp[j] = __fdiv_rn(pnum, S);
        sele[j] = be;
      }
    }
    if (lane == 0) {
      float den = 0.0f;
      if (renorm) {
        float s = selp[0];
#pragma unroll
        for (int j = 1; j < kMaxK; ++j)
          if (j < k) s = __fadd_rn(s, selp[j]);
        den = __fadd_rn(s, 1e-20f);
      }
#pragma unroll
      for (int j = 0; j < kMaxK; ++j)
        if (j < k) {
          float wj = renorm ? __fmul_rn(__fdiv_rn(selp[j], den), scaling) : __fmul_rn(selp[j], scaling);
          ids[(int64_t)t * k + j] = sele[j];
          wout[(int64_t)t * k + j] = wj;
        }
    }
}

// The softmax selection of route_select for E <= 16, NI groups of four tokens per wave: lane l holds, for each i < NI,
// the logit of expert l % 16 of token t0 + i + NI (l / 16) (ignored past E).  Segment (16-lane) butterflies give the
// 64-lane ones' results bit for bit (those only add exact zeros and compare with -inf from the lanes past E; the
// arg-max with ties to the lower index does not depend on the reduction tree), so ids, weights and logits equal
// route_select's.  The NI selections advance together (independent exchange chains side by side), the winner's
// probability numerator is carried through the arg-max exchanges, and lane j of a segment keeps selection j.
template <int NI>
__device__ __forceinline__ void route_select16(const float (&lg)[NI], int t0, int lane, int T, int E, int k,
                                               int renorm, float scaling, float* __restrict__ logits,
                                               int32_t* __restrict__ ids, float* __restrict__ wout) {
#pragma clang fp contract(off)
  const int e = lane & 15;
  const bool valid = e < E;
  float m[NI], num[NI], S[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) m[i] = valid ? lg[i] : -__builtin_inff();
  auto max_step = [&](auto sc) {
    constexpr int SS = decltype(sc)::value;
#pragma unroll
    for (int i = 0; i < NI; ++i) m[i] = fmaxf(m[i], lane_xor<SS>(m[i]));
  };
  max_step(std::integral_constant<int, 8>());
  max_step(std::integral_constant<int, 4>());
  max_step(std::integral_constant<int, 2>());
  max_step(std::integral_constant<int, 1>());
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    num[i] = valid ? hexp(__fsub_rn(lg[i], m[i])) : 0.0f;
    S[i] = num[i];
  }
  auto sum_step = [&](auto sc) {
    constexpr int SS = decltype(sc)::value;
#pragma unroll
    for (int i = 0; i < NI; ++i) S[i] = __fadd_rn(S[i], lane_xor<SS>(S[i]));
  };
  sum_step(std::integral_constant<int, 8>());
  sum_step(std::integral_constant<int, 4>());
  sum_step(std::integral_constant<int, 2>());
  sum_step(std::integral_constant<int, 1>());
  int64_t t[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    t[i] = (int64_t)t0 + i + NI * (lane >> 4);
    if (logits && t[i] < T && valid) logits[t[i] * E + e] = lg[i];
  }
  bool taken[NI];
  float ssum[NI], my_p[NI];
  int my_e[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    taken[i] = false;
    ssum[i] = my_p[i] = 0.0f;
    my_e[i] = 0;
  }
  for (int jj = 0; jj < k; ++jj) {
    float bv[NI], bp[NI];
    int be[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const bool cand = valid && !taken[i];
      bv[i] = cand ? lg[i] : 0.0f;
      be[i] = cand ? e : 0x7fffffff;
      bp[i] = num[i];
    }
    auto arg_step = [&](auto sc) {
      constexpr int SS = decltype(sc)::value;
#pragma unroll
      for (int i = 0; i < NI; ++i) seg_argmax_step<SS>(bv[i], be[i], bp[i]);
    };
    arg_step(std::integral_constant<int, 8>());
    arg_step(std::integral_constant<int, 4>());
    arg_step(std::integral_constant<int, 2>());
    arg_step(std::integral_constant<int, 1>());
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      if (be[i] == e) taken[i] = true;
      const float p = __fdiv_rn(bp[i], S[i]);
      ssum[i] = jj == 0 ? p : __fadd_rn(ssum[i], p);
      if (e == jj) {
        my_p[i] = p;
        my_e[i] = be[i];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    if (t[i] < T && e < k) {
      const float wj = renorm ? __fmul_rn(__fdiv_rn(my_p[i], __fadd_rn(ssum[i], 1e-20f)), scaling)
                              : __fmul_rn(my_p[i], scaling);
      ids[t[i] * k + e] = my_e[i];
      wout[t[i] * k + e] = wj;
    }
  }
}

// Selection of the sigmoid, group-limited router for four tokens per wave: the 16-lane segment q of the wave takes
// one token, lane j of it holds experts i * 16 + j (i < EPS).  The steps and orders (router.c states them): scores
// 1 / (1 + hexp(-logit)), routing values score + bias, group values as the sum of the two largest routing values with
// multiplicity, topk_group groups by descending value with ties to the lower group, then the k largest routing values
// among the kept groups with ties to the lower expert, weights = the selected scores over their sum in selection
// order plus 1e-20, times scaling; the reductions run over the segment's 16 lanes (row-local DPP exchanges), the
// winner's score carried through them.
// Every lane runs the same instructions (dead tokens included, with live false), so the exchanges see every lane.
template <int EPS>
__device__ __forceinline__ void route_select_sig16(const float (&lg)[EPS], const float (&bsv)[EPS], bool has_bias,
                                                   int64_t t, bool live, int lane, int E, int k, float scaling,
                                                   float* __restrict__ scores, int32_t* __restrict__ ids,
                                                   float* __restrict__ wout, int n_group, int topk_group) {
#pragma clang fp contract(off)
  const int j16 = lane & 15;
  float num[EPS], key[EPS];
#pragma unroll
  for (int i = 0; i < EPS; ++i) {
    const int e = i * 16 + j16;
    num[i] = 0.0f;
    key[i] = -__builtin_inff();
    if (e < E) {
      num[i] = __fdiv_rn(1.0f, __fadd_rn(1.0f, hexp(-lg[i])));
      key[i] = has_bias ? __fadd_rn(num[i], bsv[i]) : num[i];
      if (live && scores) scores[t * E + e] = num[i];
    }
  }
  if (topk_group < n_group) {
    const int eg = E / n_group;  // a power of two in [2, 64] (checked on the host)
    float m1[EPS], m2[EPS];
#pragma unroll
    for (int i = 0; i < EPS; ++i) {
      m1[i] = key[i];
      m2[i] = -__builtin_inff();
    }
    // the two largest values (with multiplicity) of each run of min(eg, 16) lanes
    auto fold = [&](auto sc) {
      constexpr int SS = decltype(sc)::value;
      if (SS < eg) {
#pragma unroll
        for (int i = 0; i < EPS; ++i) {
          const float o1 = lane_xor<SS>(m1[i]), o2 = lane_xor<SS>(m2[i]);
          const float n2 = fmaxf(fminf(m1[i], o1), fmaxf(m2[i], o2));
          m1[i] = fmaxf(m1[i], o1);
          m2[i] = n2;
        }
      }
    };
    fold(std::integral_constant<int, 1>());
    fold(std::integral_constant<int, 2>());
    fold(std::integral_constant<int, 4>());
    fold(std::integral_constant<int, 8>());
    // groups of 32 or 64 experts span 2 or 4 consecutive slots: merge their pairs in the lane
    auto merge = [&](auto nc) {
      constexpr int NS = decltype(nc)::value;
      if constexpr (NS <= EPS) {
#pragma unroll
        for (int b = 0; b < EPS; b += NS) {
          float a1 = m1[b], a2 = m2[b];
#pragma unroll
          for (int i = b + 1; i < b + NS; ++i) {
            const float n2 = fmaxf(fminf(a1, m1[i]), fmaxf(a2, m2[i]));
            a1 = fmaxf(a1, m1[i]);
            a2 = n2;
          }
#pragma unroll
          for (int i = b; i < b + NS; ++i) {
            m1[i] = a1;
            m2[i] = a2;
          }
        }
      }
    };
    if (eg == 32) merge(std::integral_constant<int, 2>());
    if (eg == 64) merge(std::integral_constant<int, 4>());
    float gs[EPS];
    bool gsel[EPS];
#pragma unroll
    for (int i = 0; i < EPS; ++i) {
      gs[i] = __fadd_rn(m1[i], m2[i]);
      gsel[i] = false;
    }
    for (int jj = 0; jj < topk_group; ++jj) {
      float bv = 0.0f, bp = 0.0f;
      int be = 0x7fffffff;
#pragma unroll
      for (int i = 0; i < EPS; ++i) {
        const int e = i * 16 + j16;
        if (e < E && !gsel[i]) argmax_take(bv, be, gs[i], e / eg);
      }
      seg_argmax_step<8>(bv, be, bp);
      seg_argmax_step<4>(bv, be, bp);
      seg_argmax_step<2>(bv, be, bp);
      seg_argmax_step<1>(bv, be, bp);
#pragma unroll
      for (int i = 0; i < EPS; ++i)
        if ((i * 16 + j16) / eg == be) gsel[i] = true;
    }
#pragma unroll
    for (int i = 0; i < EPS; ++i)
      if (!gsel[i]) key[i] = -__builtin_inff();
  }
  bool taken[EPS];
#pragma unroll
  for (int i = 0; i < EPS; ++i) taken[i] = false;
  float ssum = 0.0f, my_p = 0.0f;
  int my_e = 0;
  for (int jj = 0; jj < k; ++jj) {
    float bv = 0.0f, bp = 0.0f;
    int be = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < EPS; ++i) {
      const int e = i * 16 + j16;
      if (e < E && !taken[i] && (be == 0x7fffffff || key[i] > bv)) {
        bv = key[i];
        be = e;
        bp = num[i];
      }
    }
    seg_argmax_step<8>(bv, be, bp);
    seg_argmax_step<4>(bv, be, bp);
    seg_argmax_step<2>(bv, be, bp);
    seg_argmax_step<1>(bv, be, bp);
#pragma unroll
    for (int i = 0; i < EPS; ++i)
      if (be == i * 16 + j16) taken[i] = true;
    ssum = jj == 0 ? bp : __fadd_rn(ssum, bp);
    if (j16 == jj) {
      my_e = be;
      my_p = bp;
    }
  }
  if (live && j16 < k) {
    const float den = __fadd_rn(ssum, 1e-20f);
    ids[t * k + j16] = my_e;
    wout[t * k + j16] = __fmul_rn(__fdiv_rn(my_p, den), scaling);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Router logits on the fp32 matrix cores.  v_mfma_f32_16x16x4_f32 forms each output as four fused multiply-adds in
// k order, acc = fma(a3, b3, fma(a2, b2, fma(a1, b1, fma(a0, b0, acc)))), each rounded once with denormals kept (an
// in-bounds probe of 4.2 M outputs -- cancelling sums, products in the denormal range, denormal inputs -- matched that
// chain bit for bit and no other summation order).  The operands: lane l holds A = x[token l % 16][.] and
// B = w[expert l % 16][.] for k-lane q = l / 16; the 16 x 16 output block leaves tokens 4 (l / 16) + 0..3 of expert
// l % 16 in lane l.  Giving k-lane q the 16 consecutive elements 64b + 16q .. 64b + 16q + 15 of 64-element block b,
// step s of a chained accumulator takes elements 64b + 16q + s for q = 0..3, and each operand of a block is 32
// contiguous bytes of its row.  Block b feeds partial chain b % 4 (four independent accumulators: four products in
// flight where one chain would wait on each result), and the logit is (c0 + c1) + (c2 + c3): the fixed order of
// router.c (both routers), bit for bit.  Past d the token values are -0 and the weights +0: fma(-0, +0, acc) = acc
// for every acc (including either zero), so the padded steps change nothing.
//
// route_mfma_kernel (the sigmoid router, and the softmax router for E > 16): a workgroup of NW waves routes 16 TT
// tokens; wave w owns the expert blocks w NB .. w NB + NB - 1 (16 experts each).  Token rows and weight rows stream
// through LDS in chunks of 128 elements (double-buffered through registers; a chunk's products cover the next
// chunk's load latency), rows at a pitch of 272 bytes so that the 16 rows one 16-byte read touches fall on distinct
// banks.  The logits then go through LDS to the selection: four tokens per wave (route_select_sig16) for the
// sigmoid router, one per wave (route_select) for the softmax router.
// ---------------------------------------------------------------------------------------------------------------
constexpr int kSmChunk = 128, kSmPitch = 272;

template <int NW, int NB, int TT, bool SIG>
__global__ __launch_bounds__(64 * NW) void route_mfma_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             const uint16_t* __restrict__ wr,
                                                             const float* __restrict__ bias, int T, int d, int E,
                                                             int k, int renorm, float scaling,
                                                             float* __restrict__ scores, int32_t* __restrict__ ids,
                                                             float* __restrict__ wout, int n_group, int topk_group) {
#pragma clang fp contract(off)
  constexpr int NT = 64 * NW;
  constexpr int TB = 16 * TT;          // tokens per workgroup
  constexpr int ER = 16 * NB * NW;     // weight rows staged (rows past E are zero)
  constexpr int PIECES = (TB + ER) * 16;      // 16-byte pieces per chunk: token rows first, then weight rows
  constexpr int PPT = (PIECES + NT - 1) / NT;
  constexpr int STAGE = (TB + ER) * kSmPitch;
  constexpr int LP = ER + 16;                 // row pitch (floats) of the logits handed to the selection
  static_assert(TB * LP * 4 <= 2 * STAGE, "the logits reuse the staging buffers");
  extern __shared__ __attribute__((aligned(16))) char s_m[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tblk = blockIdx.x * TB;
  const int nch = (d + kSmChunk - 1) / kSmChunk;
  uint4 stage[PPT];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pc = tid + NT * j, row = pc >> 4, el = c * kSmChunk + (pc & 15) * 8;
      if (row < TB) {
        const int t = tblk + row;
        stage[j] = (t < T && el < d) ? *reinterpret_cast<const uint4*>(x + (int64_t)t * ldx + el)
                                     : make_uint4(0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u);
      } else {
        const int e = row - TB;
        stage[j] = (pc < PIECES && e < E && el < d) ? *reinterpret_cast<const uint4*>(wr + (int64_t)e * d + el)
                                                    : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int j = 0; j < PPT; ++j) {
      const int pc = tid + NT * j;
      if (PIECES % NT == 0 || pc < PIECES)
        *reinterpret_cast<uint4*>(s_m + buf * STAGE + (pc >> 4) * kSmPitch + (pc & 15) * 16) = stage[j];
    }
  };
  // a lane's 32 values of LDS row `row` in step order: k-lane q's 16 elements of each of the chunk's two blocks
  auto read_row = [&](const char* base, int row, uint4 (&u)[4]) {
    const char* src = base + row * kSmPitch + (lane >> 4) * 32;
#pragma unroll
    for (int h = 0; h < 4; ++h) u[h] = *reinterpret_cast<const uint4*>(src + (h >> 1) * 128 + (h & 1) * 16);
  };
  auto widen = [&](const uint4& u, float (&f)[8]) {
    f[0] = bf_lo(u.x); f[1] = bf_hi(u.x); f[2] = bf_lo(u.y); f[3] = bf_hi(u.y);
    f[4] = bf_lo(u.z); f[5] = bf_hi(u.z); f[6] = bf_lo(u.w); f[7] = bf_hi(u.w);
  };
  f32x4 acc[TT][NB][4];  // one per partial chain: chunk c holds blocks 2c, 2c + 1, chains 2 (c % 2) + 0, 1
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) acc[tt][nb][ch] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  float bsv[ER / 16];  // the bias of this lane's experts (i * 16 + lane % 16)
#pragma unroll
  for (int i = 0; i < ER / 16; ++i) {
    const int e = i * 16 + (lane & 15);
    bsv[i] = bias && e < E ? bias[e] : 0.0f;
  }
  const bool live = wave * NB * 16 < E;  // a wave whose experts all lie past E skips the products
  const int r = lane & 15;
  load_chunk(0);
  store_chunk(0);
  __syncthreads();
  // chunk c: its parity (a compile-time constant, so that the chain indices are) selects chains 2 PAR, 2 PAR + 1
  auto chunk = [&](int c, auto par) {
    constexpr int PAR = decltype(par)::value;
    if (c + 1 < nch) load_chunk(c + 1);
    const char* base = s_m + PAR * STAGE;
    if (live) {
      // every read of the chunk is issued before the first product (the LDS latency is paid once per chunk)
      uint4 ua[TT][4], ub[NB][4];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) read_row(base, tt * 16 + r, ua[tt]);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) read_row(base, TB + (wave * NB + nb) * 16 + r, ub[nb]);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        float a[TT][8], b[NB][8];
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) widen(ua[tt][h], a[tt]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) widen(ub[nb][h], b[nb]);
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
          for (int tt = 0; tt < TT; ++tt)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
              acc[tt][nb][2 * PAR + (h >> 1)] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                  a[tt][s], b[nb][s], acc[tt][nb][2 * PAR + (h >> 1)], 0, 0, 0);
      }
    }
    if (c + 1 < nch) store_chunk(1 - PAR);  // the other buffer: last read before the previous barrier
    __syncthreads();
  };
  for (int c = 0; c < nch; c += 2) {
    chunk(c, std::integral_constant<int, 0>());
    if (c + 1 < nch) chunk(c + 1, std::integral_constant<int, 1>());
  }
  // logits (token, expert) into LDS: lane l holds tokens 16 tt + 4 (l / 16) + i of expert 16 (w NB + nb) + l % 16
  float* lgs = reinterpret_cast<float*>(s_m);
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        lgs[(tt * 16 + 4 * (lane >> 4) + i) * LP + (wave * NB + nb) * 16 + r] =
            __fadd_rn(__fadd_rn(acc[tt][nb][0][i], acc[tt][nb][1][i]),
                      __fadd_rn(acc[tt][nb][2][i], acc[tt][nb][3][i]));
  __syncthreads();
  if constexpr (SIG) {
    // selection: token tok of the workgroup on segment tok % 4 of wave tok / 4 (four tokens per wave)
    constexpr int EPS = ER / 16;
    for (int tok0 = wave * 4; tok0 < TB; tok0 += NW * 4) {
      const int tok = tok0 + (lane >> 4);
      const int64_t t = (int64_t)tblk + tok;
      const bool on = tok < TB && t < T;
      float lg[EPS];
#pragma unroll
      for (int i = 0; i < EPS; ++i) lg[i] = lgs[min(tok, TB - 1) * LP + i * 16 + r];
      route_select_sig16<EPS>(lg, bsv, bias != nullptr, t, on, lane, E, k, scaling, scores, ids, wout, n_group,
                              topk_group);
    }
  } else {
    // softmax, E > 16: one token per wave, lane l holding experts l, l + 64, ... (bias added to the logit)
    for (int tok = wave; tok < TB; tok += NW) {
      const int t = tblk + tok;
      if (t >= T) break;
      float lg[kRouteEPL];
#pragma unroll
      for (int i = 0; i < kRouteEPL; ++i) {
        const int e = i * 64 + lane;
        lg[i] = -__builtin_inff();
        if (i * 64 < ER) {
          lg[i] = lgs[tok * LP + e];
          if (bias && e < E) lg[i] = __fadd_rn(lg[i], bias[e]);
        }
      }
      route_select(lg, t, lane, E, k, renorm, scaling, scores, ids, wout);
    }
  }
}

// The softmax router for E <= 16 without LDS staging: a 16-token tile against all experts, one 16 x 16 output block
// per partial chain, with each lane's 32 contiguous bytes of x and of w per block loaded straight into registers
// kRdPF blocks ahead.  Rows past T read row T - 1 and experts past E read expert 0: their logits are never stored nor
// selected.  SPLIT = 1: one wave runs all four chains of its tile (ring slot p holds block b0 + p, b0 a multiple of
// 4, so slot p feeds chain p) and selects the tile's 16 tokens, four per lane (route_select16<4>); no barrier.
// SPLIT = 2 or 4: SPLIT waves share a tile, wave c running chains c, c + SPLIT, ... (blocks c, c + SPLIT, ...; ring
// slot p feeds the wave's chain p % (4 / SPLIT)); the chain sums meet in LDS, and wave c then selects tokens
// 16 c / SPLIT .. of the tile, 4 / SPLIT per lane.  More waves per tile and fewer blocks per wave: for token counts
// that leave most of the chip idle.
constexpr int kRdPF = 4;  // blocks in flight per wave (8 and 12 measured slower: 22.8 and 24.0 against 21.7 us at C5)
static_assert(kRdPF % 4 == 0, "ring slot p feeds chain p % 4");

template <int SPLIT>
__global__ __launch_bounds__(256) void route_topk_direct_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                const uint16_t* __restrict__ wr,
                                                                const float* __restrict__ bias, int T, int d, int E,
                                                                int k, int renorm, float scaling,
                                                                float* __restrict__ logits,
                                                                int32_t* __restrict__ ids,
                                                                float* __restrict__ wout) {
#pragma clang fp contract(off)
  static_assert(SPLIT == 1 || SPLIT == 2 || SPLIT == 4, "one, two or four waves per tile");
  constexpr int NA = 4 / SPLIT;  // chains this wave accumulates: c, c + SPLIT, ...
  const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
  const int wave = threadIdx.x >> 6;
  const int tg = wave / SPLIT;  // the wave's tile within the workgroup
  const int t0 = (blockIdx.x * ((int)(blockDim.x >> 6) / SPLIT) + tg) * 16;
  // SPLIT = 1: a whole wave (no barrier); SPLIT = 4: the whole workgroup (one tile).  SPLIT = 2: the second tile of
  // the last workgroup may start past T; its waves run on clamped rows and store nothing (route_select16 checks t)
  if (SPLIT != 2 && t0 >= T) return;
  const int nbf = d / 64;  // whole blocks; a last partial block (d % 64 != 0) is handled after them
  const int c = wave % SPLIT;  // this wave's first chain
  const int nj = nbf > c ? (nbf - c + SPLIT - 1) / SPLIT : 0;  // whole blocks this wave runs: c, c + SPLIT, ...
  auto blk = [&](int j) { return c + SPLIT * j; };
  const uint16_t* xr = x + (int64_t)min(t0 + r, T - 1) * ldx + 16 * q;
  const uint16_t* wrow = wr + (int64_t)(r < E ? r : 0) * d + 16 * q;
  // loads with no per-lane condition, so that the compiler can keep them in flight across the products
  auto load = [&](int b, uint4 (&xv)[2], uint4 (&wv)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      xv[h] = *reinterpret_cast<const uint4*>(xr + 64 * b + 8 * h);
      wv[h] = *reinterpret_cast<const uint4*>(wrow + 64 * b + 8 * h);
    }
  };
  f32x4 acc[NA];
#pragma unroll
  for (int i = 0; i < NA; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto block = [&](const uint4 (&xv)[2], const uint4 (&wv)[2], float (&a)[16], float (&w)[16]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t xw[4] = {xv[h].x, xv[h].y, xv[h].z, xv[h].w};
      const uint32_t ww[4] = {wv[h].x, wv[h].y, wv[h].z, wv[h].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[8 * h + 2 * i] = bf_lo(xw[i]);
        a[8 * h + 2 * i + 1] = bf_hi(xw[i]);
        w[8 * h + 2 * i] = bf_lo(ww[i]);
        w[8 * h + 2 * i + 1] = bf_hi(ww[i]);
      }
    }
  };
  auto products = [&](f32x4& ac, const float (&a)[16], const float (&w)[16]) {
#pragma unroll
    for (int s2 = 0; s2 < 16; ++s2) ac = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s2], w[s2], ac, 0, 0, 0);
  };
  if (nj > 0) {
    // a ring of kRdPF blocks in registers; every load is unconditional (block indices past the end are clamped to
    // the last block and their values never used), so no slot value is merged across a branch and the loads stay
    // in flight across the products
    uint4 xs[kRdPF][2], ws[kRdPF][2];
#pragma unroll
    for (int p = 0; p < kRdPF; ++p) load(blk(min(p, nj - 1)), xs[p], ws[p]);
    for (int j0 = 0; j0 < nj; j0 += kRdPF) {
#pragma unroll
      for (int p = 0; p < kRdPF; ++p) {
        const int j = j0 + p;
        float a[16], w[16];
        block(xs[p], ws[p], a, w);
        load(blk(min(j + kRdPF, nj - 1)), xs[p], ws[p]);  // the slot's values are widened: refill it
        if (j < nj) products(acc[p % NA], a, w);
      }
    }
  }
  if ((d & 63) && c == (nbf & 3) % SPLIT) {
    // the partial block (chain nbf % 4): pieces past d read the row's first piece and become -0 (x) / +0 (w)
    uint4 xv[2], wv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool in = 64 * nbf + 16 * q + 8 * h < d;  // d % 8 == 0: a 16-byte piece is wholly in or out
      const int off = in ? 64 * nbf + 8 * h : -16 * q;
      const uint4 xl = *reinterpret_cast<const uint4*>(xr + off), wl = *reinterpret_cast<const uint4*>(wrow + off);
      xv[h] = in ? xl : make_uint4(0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u);
      wv[h] = in ? wl : make_uint4(0, 0, 0, 0);
    }
    float a[16], w[16];
    block(xv, wv, a, w);
#pragma unroll
    for (int i = 0; i < NA; ++i)
      if (NA == 1 || i == (nbf & 3) / SPLIT) products(acc[i], a, w);
  }
  const float bv = bias && r < E ? bias[r] : 0.0f;
  if constexpr (SPLIT == 1) {
    float lg[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float dot = __fadd_rn(__fadd_rn(acc[0][i], acc[1][i]), __fadd_rn(acc[2][i], acc[3][i]));
      lg[i] = bias && r < E ? __fadd_rn(dot, bv) : dot;
    }
    route_select16<4>(lg, t0, lane, T, E, k, renorm, scaling, logits, ids, wout);
  } else {
    // chain sums by (chain, token, expert); lane l holds tokens 4 (l / 16) + i of expert l % 16
    constexpr int NI = 4 / SPLIT;  // tokens per lane in the selection: wave c takes tokens 16 c / SPLIT ..
    __shared__ float part[SPLIT == 2 ? 2 : 1][4][16 * 16];
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[tg][c + SPLIT * a][(4 * q + i) * 16 + r] = acc[a][i];
    __syncthreads();
    float lg[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int tok = 16 / SPLIT * c + i + NI * q;  // route_select16's token for (lane, i)
      const float* pt = part[tg][0] + tok * 16 + r;
      const float dot = __fadd_rn(__fadd_rn(pt[0], pt[256]), __fadd_rn(pt[512], pt[768]));
      lg[i] = bias && r < E ? __fadd_rn(dot, bv) : dot;
    }
    route_select16<NI>(lg, t0 + 16 / SPLIT * c, lane, T, E, k, renorm, scaling, logits, ids, wout);
  }
}

// Both routers for E > 16 (the sigmoid router for any E) at small token counts, in two launches over the caller's
// (T, E) logits / scores buffer.  route_block_logits_kernel: a workgroup per (16-token tile, 16-expert block), its
// four waves running the four partial chains (wave c: blocks c, c + 4, ...; operands straight into registers as in
// route_topk_direct_kernel), the chain sums added in LDS as (c0 + c1) + (c2 + c3), the logits (no bias) stored.
// route_select_kernel then selects as route_mfma_kernel does (four tokens per wave for the sigmoid router, one per
// wave for the softmax router), writing the scores / biased logits over what it read.  route_mfma_kernel stages a
// tile's rows once in LDS for all experts, so with few tokens it runs on a few CUs, each walking the whole row with a
// barrier per 128-element chunk; here the tiles x blocks workgroups spread over the chip.
__global__ __launch_bounds__(256) void route_block_logits_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                 const uint16_t* __restrict__ wr, int T, int d,
                                                                 int E, float* __restrict__ out) {
#pragma clang fp contract(off)
  __shared__ float part[4][16 * 16];
  const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
  const int c = threadIdx.x >> 6;  // the chain this wave runs
  const int t0 = blockIdx.x * 16, e0 = blockIdx.y * 16;
  const int nbf = d / 64;
  const int nj = nbf > c ? (nbf - c + 3) >> 2 : 0;  // whole blocks c, c + 4, ...
  const uint16_t* xr = x + (int64_t)min(t0 + r, T - 1) * ldx + 16 * q;
  const uint16_t* wrow = wr + (int64_t)(e0 + r < E ? e0 + r : 0) * d + 16 * q;
  auto load = [&](int b, uint4 (&xv)[2], uint4 (&wv)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      xv[h] = *reinterpret_cast<const uint4*>(xr + 64 * b + 8 * h);
      wv[h] = *reinterpret_cast<const uint4*>(wrow + 64 * b + 8 * h);
    }
  };
  auto widen = [&](const uint4 (&xv)[2], const uint4 (&wv)[2], float (&a)[16], float (&w)[16]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t xw[4] = {xv[h].x, xv[h].y, xv[h].z, xv[h].w};
      const uint32_t ww[4] = {wv[h].x, wv[h].y, wv[h].z, wv[h].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[8 * h + 2 * i] = bf_lo(xw[i]);
        a[8 * h + 2 * i + 1] = bf_hi(xw[i]);
        w[8 * h + 2 * i] = bf_lo(ww[i]);
        w[8 * h + 2 * i + 1] = bf_hi(ww[i]);
      }
    }
  };
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  auto products = [&](const float (&a)[16], const float (&w)[16]) {
#pragma unroll
    for (int s2 = 0; s2 < 16; ++s2) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s2], w[s2], acc, 0, 0, 0);
  };
  if (nj > 0) {
    uint4 xs[kRdPF][2], ws[kRdPF][2];
#pragma unroll
    for (int p = 0; p < kRdPF; ++p) load(c + 4 * min(p, nj - 1), xs[p], ws[p]);
    for (int j0 = 0; j0 < nj; j0 += kRdPF) {
#pragma unroll
      for (int p = 0; p < kRdPF; ++p) {
        const int j = j0 + p;
        float a[16], w[16];
        widen(xs[p], ws[p], a, w);
        load(c + 4 * min(j + kRdPF, nj - 1), xs[p], ws[p]);
        if (j < nj) products(a, w);
      }
    }
  }
  if ((d & 63) && c == (nbf & 3)) {  // the partial block, as in route_topk_direct_kernel
    uint4 xv[2], wv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bool in = 64 * nbf + 16 * q + 8 * h < d;
      const int off = in ? 64 * nbf + 8 * h : -16 * q;
      const uint4 xl = *reinterpret_cast<const uint4*>(xr + off), wl = *reinterpret_cast<const uint4*>(wrow + off);
      xv[h] = in ? xl : make_uint4(0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u);
      wv[h] = in ? wl : make_uint4(0, 0, 0, 0);
    }
    float a[16], w[16];
    widen(xv, wv, a, w);
    products(a, w);
  }
  // lane l holds tokens 4 (l / 16) + i of expert e0 + l % 16
#pragma unroll
  for (int i = 0; i < 4; ++i) part[c][(4 * q + i) * 16 + r] = acc[i];
  __syncthreads();
  const int tok = threadIdx.x >> 4, e = threadIdx.x & 15;  // one (token, expert) of the tile per thread
  if (t0 + tok < T && e0 + e < E) {
    const int o = tok * 16 + e;
    out[(int64_t)(t0 + tok) * E + e0 + e] =
        __fadd_rn(__fadd_rn(part[0][o], part[1][o]), __fadd_rn(part[2][o], part[3][o]));
  }
}

template <bool SIG, int EPS>
__global__ __launch_bounds__(256) void route_select_kernel(const float* __restrict__ bias, int T, int E, int k,
                                                           int renorm, float scaling, float* __restrict__ lgbuf,
                                                           int32_t* __restrict__ ids, float* __restrict__ wout,
                                                           int n_group, int topk_group) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if constexpr (SIG) {
    // four tokens per wave: segment q takes one token, lane j of it experts i * 16 + j
    const int r = lane & 15;
    const int64_t t = ((int64_t)blockIdx.x * 4 + wave) * 4 + (lane >> 4);
    if (((int64_t)blockIdx.x * 4 + wave) * 4 >= T) return;  // a whole wave past T
    const bool live = t < T;
    float lg[EPS], bsv[EPS];
#pragma unroll
    for (int i = 0; i < EPS; ++i) {
      const int e = i * 16 + r;
      lg[i] = live && e < E ? lgbuf[t * E + e] : 0.0f;
      bsv[i] = bias && e < E ? bias[e] : 0.0f;
    }
    route_select_sig16<EPS>(lg, bsv, bias != nullptr, t, live, lane, E, k, scaling, lgbuf, ids, wout, n_group,
                            topk_group);
  } else {
    // softmax: one token per wave, lane l holding experts l, l + 64, ... (bias added to the logit)
    const int t = blockIdx.x * 4 + wave;
    if (t >= T) return;
    float lg[kRouteEPL];
#pragma unroll
    for (int i = 0; i < kRouteEPL; ++i) {
      const int e = i * 64 + lane;
      lg[i] = -__builtin_inff();
      if (e < E) {
        lg[i] = lgbuf[(int64_t)t * E + e];
        if (bias) lg[i] = __fadd_rn(lg[i], bias[e]);
      }
    }
    route_select(lg, t, lane, E, k, renorm, scaling, lgbuf, ids, wout);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Dispatch: stable counting sort of flat ids.  Pass 1 (one wave per block of kFPB flat rows): per-block expert
// histogram and the stable rank of each flat row among earlier rows of the same expert inside its block (wave
// ballots: a lane's peers are the lanes whose id agrees on every bit).  Pass 2 (one workgroup): per-expert totals,
// expert starts, and per-(block, expert) first sorted row.  Pass 3: positions, index arrays and the row copies
// (per token), or the index arrays alone (per flat row) when no rows are copied.
// ---------------------------------------------------------------------------------------------------------------
constexpr int kFPB = 256;        // flat rows per histogram block (one wave each: 128 waves at M = 32768)
constexpr int kMaxEDispatch = 1024;

// routing weight f of topk_w (fp32, bf16 or fp16) rounded to the activations' 16-bit type (fp16 when out_f16, else
// bf16): the .to(x.dtype) of aurora/hf_compat.py:80; a weight already in that type is copied unchanged
__device__ __forceinline__ uint16_t route_w16(const void* tw, int tw_dtype, int64_t f, int out_f16) {
  const uint16_t raw = tw_dtype == HMOE_DT_F32 ? 0 : reinterpret_cast<const uint16_t*>(tw)[f];
  if (tw_dtype == (out_f16 ? HMOE_DT_F16 : HMOE_DT_BF16)) return raw;
  const float v = tw_dtype == HMOE_DT_F32 ? reinterpret_cast<const float*>(tw)[f]
                  : tw_dtype == HMOE_DT_F16 ? Elt<true>::one(raw) : bf2f(raw);
  return out_f16 ? __builtin_bit_cast(uint16_t, (_Float16)v) : (uint16_t)f2bf(v);
}

// an int64 id outside the int32 range becomes -1 (invalid) rather than wrapping onto a valid expert
__device__ __forceinline__ int load_id(const void* ids, int is64, int64_t f) {
  if (is64) {
    const int64_t v = reinterpret_cast<const int64_t*>(ids)[f];
    return (v < 0 || v > INT32_MAX) ? -1 : (int)v;
  }
  return reinterpret_cast<const int32_t*>(ids)[f];
}

__global__ __launch_bounds__(64) void dispatch_hist_kernel(const void* __restrict__ ids, int ids64, int64_t M, int E,
                                                           int nbits, int32_t* __restrict__ hist,
                                                           int32_t* __restrict__ rank) {
  __shared__ int run[kMaxEDispatch];
  const int lane = threadIdx.x;
  for (int e = lane; e < E; e += 64) run[e] = 0;
  __syncthreads();
  const int64_t start = (int64_t)blockIdx.x * kFPB;
  const int64_t end = min(M, start + kFPB);
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // all of the block's ids are loaded up front (one memory round trip instead of one per 64 ids)
  constexpr int kSteps = kFPB / 64;
  int ev[kSteps];
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    const int64_t f = start + i * 64 + lane;
    ev[i] = f < end ? load_id(ids, ids64, f) : -1;
  }
#pragma unroll
  for (int i = 0; i < kSteps; ++i) {
    const int64_t base = start + i * 64;
    if (base >= end) break;
    const int64_t f = base + lane;
    const int e = ev[i];
    const bool valid = e >= 0 && e < E;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t m1 = __ballot(bit);
      peers &= ((e >> b) & 1) ? m1 : ~m1;
    }
    const int r = __popcll(peers & lt);
    const int cnt = __popcll(peers);
    int basecnt = 0;
    if (valid) basecnt = run[e];
    __syncthreads();
    if (valid) {
      rank[f] = basecnt + r;
      if (r == 0) run[e] = basecnt + cnt;
    }
    __syncthreads();
  }
  for (int e = lane; e < E; e += 64) hist[(int64_t)blockIdx.x * E + e] = run[e];
}

// Per-expert totals, expert starts and per-(block, expert) first sorted row, in one workgroup of 1024 threads.
// Thread (g, e) of the G x E grid (G = the largest power of two with G * E <= 1024) owns the histogram blocks
// [g * C, (g + 1) * C) of expert e (C = ceil(nblk / G)): it sums them, the group sums are scanned per expert, the
// totals are scanned over the experts by wave prefix sums, and each thread then rewrites its blocks' counts as
// running first rows.  All integer, so the order of the sums does not matter.
// n_invalid (optional): M minus the rows counted, i.e. the flat rows whose id lies outside [0, E).
__global__ __launch_bounds__(1024) void dispatch_scan_kernel(int32_t* __restrict__ hist, int nblk, int E,
                                                             int32_t* __restrict__ counts,
                                                             int64_t* __restrict__ counts64,
                                                             int32_t* __restrict__ starts,
                                                             int32_t* __restrict__ gstart, int64_t M,
                                                             int32_t* __restrict__ n_invalid) {
  __shared__ int part[1024];              // [G][E] group sums, then their exclusive prefix per expert
  __shared__ int tot[kMaxEDispatch + 1];  // totals, then exclusive starts
  __shared__ int wsum[16], gsum[16];
  const int tid = threadIdx.x;
  int G = 1;
  while (G * 2 * E <= 1024) G *= 2;
  const int C = (nblk + G - 1) / G;
  const int g = tid / E, e = tid - g * E;
  const bool mine = g < G;
  int b0 = 0, b1 = 0;
  if (mine) {
    b0 = min(nblk, g * C);
    b1 = min(nblk, b0 + C);
    int sum = 0;
    int b = b0;
    for (; b + 8 <= b1; b += 8) {  // eight loads in flight
      int v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = hist[(int64_t)(b + u) * E + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) sum += v[u];
    }
    for (; b < b1; ++b) sum += hist[(int64_t)b * E + e];
    part[tid] = sum;
  }
  __syncthreads();
  // exclusive prefix over the groups of each expert, and the expert totals
  for (int ee = tid; ee < E; ee += 1024) {
    int run = 0;
    for (int gg = 0; gg < G; ++gg) {
      const int v = part[gg * E + ee];
      part[gg * E + ee] = run;
      run += v;
    }
    tot[ee] = run;
    counts[ee] = run;
    if (counts64) counts64[ee] = run;
  }
  __syncthreads();
  // exclusive scan of the totals over the experts: a wave prefix per 64 experts, then the wave totals
  // (and, for the row-group tiles, of the experts' group counts ceil(total / 128))
  const int lane = tid & 63, w = tid >> 6;
  const int v = tid < E ? tot[tid] : 0;
  const int gv = (v + kTileGroupRows - 1) / kTileGroupRows;
  int incl = v, gincl = gv;
#pragma unroll
  for (int sft = 1; sft < 64; sft <<= 1) {
    const int o = __shfl_up(incl, sft, 64);
    const int og = __shfl_up(gincl, sft, 64);
    if (lane >= sft) {
      incl += o;
      gincl += og;
    }
  }
  if (lane == 63) {
    wsum[w] = incl;
    gsum[w] = gincl;
  }
  __syncthreads();
  int wbase = 0, gbase = 0;
  for (int ww = 0; ww < w; ++ww) {
    wbase += wsum[ww];
    gbase += gsum[ww];
  }
  __syncthreads();
  if (tid < E) {
    tot[tid] = wbase + incl - v;
    starts[tid] = wbase + incl - v;
    if (gstart) gstart[tid] = gbase + gincl - gv;
  }
  if (tid == 0) {
    int all = 0, gall = 0;
    for (int ww = 0; ww < 16; ++ww) {
      all += wsum[ww];
      gall += gsum[ww];
    }
    starts[E] = all;
    if (gstart) gstart[E] = gall;
    if (n_invalid) n_invalid[0] = (int32_t)(M - all);
  }
  __syncthreads();
  if (mine) {
    int run = tot[e] + part[tid];
    int b = b0;
    for (; b + 8 <= b1; b += 8) {
      int v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = hist[(int64_t)(b + u) * E + e];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        hist[(int64_t)(b + u) * E + e] = run;
        run += v[u];
      }
    }
    for (; b < b1; ++b) {
      const int c = hist[(int64_t)b * E + e];
      hist[(int64_t)b * E + e] = run;
      run += c;
    }
  }
}

// Pass 3 without row copies: the index arrays only, one thread per flat row f (token f / k), so that every row's
// lookups are in flight together (the per-token pass below visits a token's k rows one after another: at top-8 its
// lookups are eight dependent round trips per wave).  Same values as the per-token pass.
__global__ __launch_bounds__(256) void dispatch_index_kernel(const void* __restrict__ ids, int ids64,
                                                             const void* __restrict__ tw, int tw_dtype, int ws_f16,
                                                             int64_t M,
                                                             int k, int E, const int32_t* __restrict__ blkoff,
                                                             const int32_t* __restrict__ rank,
                                                             int32_t* __restrict__ order, int32_t* __restrict__ a_idx,
                                                             int32_t* __restrict__ inv_pos,
                                                             uint16_t* __restrict__ w_sorted) {
  for (int64_t f = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; f < M; f += (int64_t)gridDim.x * blockDim.x) {
    const int e = load_id(ids, ids64, f);
    const int64_t pos = (e >= 0 && e < E) ? (int64_t)blkoff[(f / kFPB) * E + e] + rank[f] : -1;
    if (pos >= 0) {
      order[pos] = (int32_t)f;
      if (a_idx) a_idx[pos] = (int32_t)(f / k);
      if (w_sorted) w_sorted[pos] = route_w16(tw, tw_dtype, f, ws_f16);
    }
    if (inv_pos) inv_pos[f] = (int32_t)pos;
  }
}

// Small inputs without row copies (M <= kSmallM flat rows, E <= kSmallE): the three passes in one workgroup of 16
// waves.  Wave w takes the flat rows [w C, (w + 1) C) (C = 64 ceil(M / 1024)), 64 at a time in flat order: a row's
// rank among the wave's earlier rows of its expert comes from the wave ballots of the histogram pass (peers agree on
// every id bit) plus the wave's running count, kept in LDS per (wave, expert).  The waves' counts are then scanned
// per expert (wave order = flat order) and the totals over the experts, and each row's position is its expert's
// start plus the earlier waves' count plus its rank: the same stable counting sort, so the same outputs as the three
// passes, with one launch instead of three.
constexpr int kSmallRows = 8;                   // flat rows per lane at most
constexpr int kSmallE = 256;                    // experts: four consecutive ones per lane in the scan
constexpr int64_t kSmallM = 16 * 64 * kSmallRows;  // 8192 flat rows

__global__ __launch_bounds__(1024) void dispatch_small_kernel(const void* __restrict__ ids, int ids64,
                                                              const void* __restrict__ tw, int tw_dtype, int ws_f16,
                                                              int64_t M, int k, int E, int nbits,
                                                              int32_t* __restrict__ counts,
                                                              int64_t* __restrict__ counts64,
                                                              int32_t* __restrict__ starts,
                                                              int32_t* __restrict__ order, int32_t* __restrict__ a_idx,
                                                              int32_t* __restrict__ inv_pos,
                                                              uint16_t* __restrict__ w_sorted,
                                                              int32_t* __restrict__ n_invalid) {
  __shared__ int run[16][kSmallE];  // per wave and expert: its rows so far, then the earlier waves' rows
  __shared__ int st[kSmallE + 1];   // expert starts
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int e = lane; e < E; e += 64) run[w][e] = 0;
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int steps = (int)((M + 1023) / 1024);  // 64-row steps per wave (at most kSmallRows)
  const int64_t f0 = (int64_t)w * 64 * steps;
  int ev[kSmallRows], rk[kSmallRows];
#pragma unroll
  for (int i = 0; i < kSmallRows; ++i) {
    const int64_t f = f0 + i * 64 + lane;
    ev[i] = i < steps && f < M ? load_id(ids, ids64, f) : -1;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSmallRows; ++i) {
    if (i >= steps) break;  // wave-uniform
    const int e = ev[i];
    const bool valid = e >= 0 && e < E;
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = valid && ((e >> b) & 1);
      const uint64_t m1 = __ballot(bit);
      peers &= ((e >> b) & 1) ? m1 : ~m1;
    }
    const int r = __popcll(peers & lt);
    int basecnt = 0;
    if (valid) basecnt = run[w][e];
    rk[i] = basecnt + r;
    __builtin_amdgcn_wave_barrier();  // every lane has read run[w][.] before the step's first lane updates it
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    if (valid && r == 0) run[w][e] = basecnt + __popcll(peers);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  // thread e: expert e's exclusive prefix over the waves and its total
  if ((int)threadIdx.x < E) {
    const int e = threadIdx.x;
    int tot = 0;
#pragma unroll
    for (int ww = 0; ww < 16; ++ww) {
      const int c = run[ww][e];
      run[ww][e] = tot;
      tot += c;
    }
    st[e] = tot;
  }
  __syncthreads();
  // wave 0, lane l: the starts of experts 4 l .. 4 l + 3 (in order, after a wave prefix of the lanes' sums)
  if (w == 0) {
    int tot[4], lsum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * lane + j;
      tot[j] = e < E ? st[e] : 0;
      lsum += tot[j];
    }
    int incl = lsum;
#pragma unroll
    for (int sft = 1; sft < 64; sft <<= 1) {
      const int o = __shfl_up(incl, sft, 64);
      if (lane >= sft) incl += o;
    }
    int at = incl - lsum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * lane + j;
      if (e < E) {
        st[e] = at;
        counts[e] = tot[j];
        if (counts64) counts64[e] = tot[j];
        starts[e] = at;
      }
      at += tot[j];
    }
    if (lane == 63) {
      st[E] = incl;
      starts[E] = incl;
      if (n_invalid) n_invalid[0] = (int32_t)(M - incl);
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kSmallRows; ++i) {
    const int64_t f = f0 + i * 64 + lane;
    if (i >= steps || f >= M) break;
    const int e = ev[i];
    const int64_t pos = (e >= 0 && e < E) ? (int64_t)st[e] + run[w][e] + rk[i] : -1;
    if (pos >= 0) {
      order[pos] = (int32_t)f;
      if (a_idx) a_idx[pos] = (int32_t)(f / k);
      if (w_sorted) w_sorted[pos] = route_w16(tw, tw_dtype, f, ws_f16);
    }
    if (inv_pos) inv_pos[f] = (int32_t)pos;
  }
}

// one wave per token: sorted positions of its k rows, index arrays, then the row copies x[t] -> xs[pos_j] and into
// the row-group tiles (64-byte pieces: slice s of row pos_j, its chunks swizzled as in the K-major LDS image)
// KT: the slot count k when it is 1, 2, 4 or 8 (0: any k up to kMaxK), so the per-slot arrays hold only k entries
template <int KT>
__global__ __launch_bounds__(256) void dispatch_scatter_kernel(
    const void* __restrict__ ids, int ids64, const void* __restrict__ tw, int tw_dtype, int ws_f16, int64_t T, int k,
    int E,
    const int32_t* __restrict__ blkoff, const int32_t* __restrict__ rank, const uint16_t* __restrict__ x,
    int64_t ldx, int64_t d, uint16_t* __restrict__ xs, int32_t* __restrict__ order, int32_t* __restrict__ a_idx,
    int32_t* __restrict__ inv_pos, uint16_t* __restrict__ w_sorted, char* __restrict__ xs_tiles,
    const int32_t* __restrict__ starts, const int32_t* __restrict__ gstart) {
  constexpr int KA = KT > 0 ? KT : kMaxK;
  if constexpr (KT > 0) k = KT;
  const int lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int64_t nvec = d / 8;
  // rows of up to 2048 elements: the lane's (at most 4) chunks of the token's row are loaded first, since their
  // address needs no lookup, and stay in registers while the positions are looked up
  const bool pre = (xs || xs_tiles) && nvec <= 256;
  for (int64_t t = (int64_t)blockIdx.x * nwaves + (threadIdx.x >> 6); t < T; t += (int64_t)gridDim.x * nwaves) {
    const uint4* src = reinterpret_cast<const uint4*>(x + t * ldx);
    uint4 xv[4];
    if (pre) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t c = lane + 64 * i;
        xv[i] = c < nvec ? src[c] : make_uint4(0, 0, 0, 0);
      }
    }
    int64_t pos[KA];
    int64_t tpos[KA];  // tiles: byte offset of the row's slice 0 (its group's slice 0 + 64 * row in group)
    int tsw[KA];       // tiles: the row's chunk swizzle
#pragma unroll
    for (int j = 0; j < KA; ++j) {
      pos[j] = -1;
      tpos[j] = 0;
      tsw[j] = 0;
      if (j < k) {
        const int64_t f = t * k + j;
        const int e = load_id(ids, ids64, f);
        if (e >= 0 && e < E) pos[j] = (int64_t)blkoff[(f / kFPB) * E + e] + rank[f];
        if (xs_tiles && pos[j] >= 0) {
          const int64_t rel = pos[j] - starts[e];
          const int64_t g = gstart[e] + rel / kTileGroupRows;
          const int rr = (int)(rel % kTileGroupRows);
          tpos[j] = g * ((d + kTileK - 1) / kTileK) * (kTileGroupRows * kTileK * 2) + rr * 64;
          tsw[j] = (rr >> 2) & 3;
        }
        if (lane == j && pos[j] >= 0) {
          order[pos[j]] = (int32_t)f;
          if (a_idx) a_idx[pos[j]] = (int32_t)t;
          if (w_sorted) w_sorted[pos[j]] = route_w16(tw, tw_dtype, f, ws_f16);
        }
        if (lane == j && inv_pos) inv_pos[f] = (int32_t)pos[j];
      }
    }
    if (xs || xs_tiles) {
      auto put = [&](int64_t c, const uint4 v) {
#pragma unroll
        for (int j = 0; j < KA; ++j)
          if (j < k && pos[j] >= 0) {
            if (xs) reinterpret_cast<uint4*>(xs + pos[j] * d)[c] = v;
            if (xs_tiles) {  // chunk c: slice c / 4, logical chunk c % 4 of the row's 64 bytes
              const int64_t off = tpos[j] + (c >> 2) * (kTileGroupRows * kTileK * 2) + (((c & 3) ^ tsw[j]) * 16);
              *reinterpret_cast<uint4*>(xs_tiles + off) = v;
            }
          }
      };
      if (pre) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (lane + 64 * i < nvec) put(lane + 64 * i, xv[i]);
      } else {
        for (int64_t c = lane; c < nvec; c += 64) put(c, src[c]);
      }
    }
  }
}

// make_schedule (aurora/moe_triton.py:93-107): one thread per block b; expert found by a scan over the counts.
__global__ __launch_bounds__(256) void make_schedule_kernel(const void* __restrict__ counts, int is64, int E,
                                                            int64_t nb, int block_m, int32_t* __restrict__ block_e,
                                                            int32_t* __restrict__ block_row,
                                                            int32_t* __restrict__ row_end) {
  __shared__ int64_t s_start[kMaxEDispatch + 1];
  __shared__ int64_t s_cum[kMaxEDispatch + 1];
  if (threadIdx.x == 0) {
    int64_t st = 0, cu = 0;
    for (int e = 0; e < E; ++e) {
      const int64_t c = read_count(counts, is64, e);
      s_start[e] = st;
      st += c;
      cu += (c + block_m - 1) / block_m;
      s_cum[e] = cu;
    }
  }
  __syncthreads();
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
    // e = searchsorted(cum, b, right=True): number of cum entries <= b
    int lo = 0, hi = E;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (s_cum[mid] <= b)
        lo = mid + 1;
      else
        hi = mid;
    }
    const int e = lo;
    const int ec = e < E ? e : E - 1;
    const int64_t c = read_count(counts, is64, ec);
    const int64_t nblk = (c + block_m - 1) / block_m;
    block_e[b] = e < E ? ec : -1;
    block_row[b] = (int32_t)(s_start[ec] + (b - (s_cum[ec] - nblk)) * block_m);
    row_end[b] = (int32_t)(s_start[ec] + c);
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Combine (forward) and its backward.
// ---------------------------------------------------------------------------------------------------------------
// out[t] = bf16(sum_j y[t*k + j]) (fp32 sum in slot order), or with `add`: bf16(that + add[t]) (bf16 + bf16
// computed in fp32 and rounded once, as torch adds two bf16 tensors)
// out[t] = bf16(sum_j y[t*k + j]) (+ add[t], rounded again), one thread per 8 columns of a token.  KT > 0 is the
// slot count at compile time: the thread issues its KT row loads before the first sum (KT = 0: a runtime loop).
// Either way the slots are summed in order j = 0, 1, ..., so the result does not depend on KT.  With inv_pos, a slot
// whose inv_pos is negative (an expert id outside [0, E): no GEMM wrote its row of y) is read as zeros.
template <int KT, bool F16>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ y,
                                                      const int32_t* __restrict__ inv_pos, int64_t T, int k,
                                                      int64_t d, const uint16_t* __restrict__ add,
                                                      uint16_t* __restrict__ out) {
  const int64_t nvec = d / 8;
  const int64_t total = T * nvec;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = i / nvec, c = i - t * nvec;
    const uint4* src = reinterpret_cast<const uint4*>(y + t * k * d) + c;
    float s[8];
    using X = Elt<F16>;
    // round to the element type: torch's bf16 rule (NaN -> 0x7fc0) for bf16, nearest even for fp16
    auto pack = [](float lo, float hi) { return F16 ? cvt_h2(lo, hi) : pack_bf2(lo, hi); };
    auto first = [&](const uint4 v) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s[2 * q] = X::lo(w[q]);
        s[2 * q + 1] = X::hi(w[q]);
      }
    };
    auto accum = [&](const uint4 v) {
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s[2 * q] += X::lo(w[q]);
        s[2 * q + 1] += X::hi(w[q]);
      }
    };
    const uint4 a = add ? reinterpret_cast<const uint4*>(add + t * d)[c] : make_uint4(0, 0, 0, 0);
    // the row is loaded whether or not its slot was routed (every slot's row lies inside y), and a slot routed
    // nowhere is zeroed afterwards: the row loads do not wait for inv_pos
    auto row = [&](int j) {
      const uint4 v = src[j * nvec];
      return (inv_pos && inv_pos[t * k + j] < 0) ? make_uint4(0, 0, 0, 0) : v;
    };
    if constexpr (KT > 0) {
      // every row load is issued before any inv_pos value is waited for
      uint4 v[KT];
#pragma unroll
      for (int j = 0; j < KT; ++j) v[j] = src[j * nvec];
      if (inv_pos) {
        int iv[KT];
#pragma unroll
        for (int j = 0; j < KT; ++j) iv[j] = inv_pos[t * k + j];
#pragma unroll
        for (int j = 0; j < KT; ++j)
          if (iv[j] < 0) v[j] = make_uint4(0, 0, 0, 0);
      }
      first(v[0]);
#pragma unroll
      for (int j = 1; j < KT; ++j) accum(v[j]);
    } else {
      first(row(0));
      for (int j = 1; j < k; ++j) accum(row(j));
    }
    uint4 o;
    o.x = pack(s[0], s[1]);
    o.y = pack(s[2], s[3]);
    o.z = pack(s[4], s[5]);
    o.w = pack(s[6], s[7]);
    if (add) {
      const uint32_t av[4] = {a.x, a.y, a.z, a.w};
      uint32_t ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int q = 0; q < 4; ++q)
        ov[q] = pack(__fadd_rn(X::lo(ov[q]), X::lo(av[q])), __fadd_rn(X::hi(ov[q]), X::hi(av[q])));
      o = make_uint4(ov[0], ov[1], ov[2], ov[3]);
    }
    reinterpret_cast<uint4*>(out + t * d)[c] = o;
  }
}

// one wave per sorted row: dys[r] = bf16(w_r * dout[t]); dtopk_w[f] = <dout[t], yhat[r]>
// DW: also dtopk_w[order[r]] = <dout[t], yhat[r]>; without it the scaled rows dys only.
template <bool DW>
__global__ __launch_bounds__(256) void combine_bwd_kernel(const uint16_t* __restrict__ dout,
                                                          const uint16_t* __restrict__ yhat,
                                                          const int32_t* __restrict__ order,
                                                          const int32_t* __restrict__ a_idx,
                                                          const uint16_t* __restrict__ w_sorted, int64_t M, int k,
                                                          int64_t d, uint16_t* __restrict__ dys,
                                                          float* __restrict__ dtopk_w) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  const int64_t nvec = d / 8;
  for (int64_t r = (int64_t)blockIdx.x * nwaves + (threadIdx.x >> 6); r < M; r += (int64_t)gridDim.x * nwaves) {
    const int64_t t = a_idx[r];
    const float wr = bf2f(w_sorted[r]);
    const uint4* go = reinterpret_cast<const uint4*>(dout + t * d);
    uint4* dy = reinterpret_cast<uint4*>(dys + r * d);
    float acc = 0.0f;
    for (int64_t c = lane; c < nvec; c += 64) {
      const uint4 g = go[c];
      uint4 yv = make_uint4(0, 0, 0, 0);
      if constexpr (DW) yv = reinterpret_cast<const uint4*>(yhat + r * d)[c];
      const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, yw[4] = {yv.x, yv.y, yv.z, yv.w};
      uint32_t ow[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float g0 = bf_lo(gw[q]), g1 = bf_hi(gw[q]);
        if constexpr (DW) {
          acc = __fadd_rn(acc, __fmul_rn(g0, bf_lo(yw[q])));
          acc = __fadd_rn(acc, __fmul_rn(g1, bf_hi(yw[q])));
        }
        ow[q] = pack_bf2(__fmul_rn(wr, g0), __fmul_rn(wr, g1));
      }
      dy[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
    if constexpr (DW) {
      acc = wave_sum_butterfly(acc);
      if (lane == 0) dtopk_w[order[r]] = acc;
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------
// Router backward: dlogits per token (lanes over experts), then dwr = dlogits^T x by token chunks + fixed-order
// reduction of the chunk partials.
// ---------------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void router_dlogits_kernel(const float* __restrict__ logits,
                                                             const int32_t* __restrict__ ids,
                                                             const float* __restrict__ dtw, int64_t T, int E, int k,
                                                             int renorm, float scaling,
                                                             float* __restrict__ dlogits) {
  const int lane = threadIdx.x & 63;
  const int nwaves = blockDim.x >> 6;
  for (int64_t t = (int64_t)blockIdx.x * nwaves + (threadIdx.x >> 6); t < T; t += (int64_t)gridDim.x * nwaves) {
    float lg[kRouteEPL];
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < kRouteEPL; ++i) {
      lg[i] = -__builtin_inff();
      if (i * 64 + lane < E) {
        lg[i] = logits[t * E + i * 64 + lane];
        m = fmaxf(m, lg[i]);
      }
    }
    m = wave_max_butterfly(m);
    float ex[kRouteEPL];
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < kRouteEPL; ++i) {
      ex[i] = 0.0f;
      if (i * 64 + lane < E) {
        ex[i] = hexp(__fsub_rn(lg[i], m));
        a = __fadd_rn(a, ex[i]);
      }
    }
    const float S = wave_sum_butterfly(a);
    float p[kRouteEPL];
#pragma unroll
    for (int i = 0; i < kRouteEPL; ++i) p[i] = __fdiv_rn(ex[i], S);
    // selected probabilities and their upstream grads
    float sp[kMaxK], dw[kMaxK];
    int se[kMaxK];
    float ssum = 0.0f, sdot = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      sp[j] = 0.0f;
      dw[j] = 0.0f;
      se[j] = -1;
      if (j < k) {
        se[j] = ids[t * k + j];
        float mine = 0.0f;
#pragma unroll
        for (int i = 0; i < kRouteEPL; ++i)
          if (se[j] == i * 64 + lane) mine = p[i];
        sp[j] = __shfl(mine, se[j] & 63, 64);
        dw[j] = dtw[t * k + j] * scaling;
        ssum += sp[j];
        sdot += dw[j] * sp[j];
      }
    }
    const float den = ssum + 1e-20f;
    float dsel[kMaxK];
    float pdp = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      dsel[j] = 0.0f;
      if (j < k) {
        dsel[j] = renorm ? dw[j] / den - sdot / (den * den) : dw[j];
        pdp += sp[j] * dsel[j];
      }
    }
#pragma unroll
    for (int i = 0; i < kRouteEPL; ++i) {
      const int e = i * 64 + lane;
      if (e < E) {
        float dp = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxK; ++j)
          if (j < k && se[j] == e) dp += dsel[j];
        dlogits[t * E + e] = p[i] * (dp - pdp);
      }
    }
  }
}

// The same for E <= 16: four tokens per wave, 16 lanes each (lane l: token l / 16, expert l % 16).  The 16-lane
// butterflies give the 64-lane ones' values bit for bit (those only add exact zeros / take maxima with -inf from
// the lanes past E).
__global__ __launch_bounds__(256) void router_dlogits16_kernel(const float* __restrict__ logits,
                                                               const int32_t* __restrict__ ids,
                                                               const float* __restrict__ dtw, int64_t T, int E, int k,
                                                               int renorm, float scaling,
                                                               float* __restrict__ dlogits) {
  const int lane = threadIdx.x & 63;
  const int e = lane & 15, seg = lane & ~15;
  const int nwaves = blockDim.x >> 6;
  for (int64_t t0 = ((int64_t)blockIdx.x * nwaves + (threadIdx.x >> 6)) * 4; t0 < T;
       t0 += (int64_t)gridDim.x * nwaves * 4) {
    const int64_t t = t0 + (lane >> 4);
    const bool live = t < T;
    const int64_t tc = live ? t : T - 1;  // rows past T read the last row and write nothing
    const float lg = e < E ? logits[tc * E + e] : -__builtin_inff();
    float m = lg;
    m = bfly_max<8>(m);
    m = bfly_max<4>(m);
    m = bfly_max<2>(m);
    m = bfly_max<1>(m);
    const float ex = e < E ? hexp(__fsub_rn(lg, m)) : 0.0f;
    float S = ex;
    S = bfly_add<8>(S);
    S = bfly_add<4>(S);
    S = bfly_add<2>(S);
    S = bfly_add<1>(S);
    const float p = __fdiv_rn(ex, S);
    float sp[kMaxK], dw[kMaxK];
    int se[kMaxK];
    float ssum = 0.0f, sdot = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      sp[j] = 0.0f;
      dw[j] = 0.0f;
      se[j] = -1;
      if (j < k) {
        se[j] = ids[tc * k + j];
        sp[j] = __shfl(se[j] == e ? p : 0.0f, seg | (se[j] & 15), 64);
        dw[j] = dtw[tc * k + j] * scaling;
        ssum += sp[j];
        sdot += dw[j] * sp[j];
      }
    }
    const float den = ssum + 1e-20f;
    float dsel[kMaxK];
    float pdp = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
      dsel[j] = 0.0f;
      if (j < k) {
        dsel[j] = renorm ? dw[j] / den - sdot / (den * den) : dw[j];
        pdp += sp[j] * dsel[j];
      }
    }
    if (live && e < E) {
      float dp = 0.0f;
#pragma unroll
      for (int j = 0; j < kMaxK; ++j)
        if (j < k && se[j] == e) dp += dsel[j];
      dlogits[t * E + e] = p * (dp - pdp);
    }
  }
}

// dwr = dlogits^T x.  A chunk of kDwrWaves * kDwrTok tokens per workgroup; wave w sums its kDwrTok tokens in token
// order for 8 columns per lane and up to kDwrEG experts per pass (dlogits of a token are wave-uniform scalar loads);
// the four waves' sums are added in wave order through LDS and stored as the chunk's partial.  The chunk partials
// are then added in chunk order, so the result does not depend on the launch.
constexpr int kDwrTok = 32;
constexpr int kDwrWaves = 4;
constexpr int kDwrChunk = kDwrTok * kDwrWaves;
constexpr int kDwrEG = 16;

// grid (nchunk, ceil(d / 512)), block 256
__global__ __launch_bounds__(256) void router_dwr_partial_kernel(const float* __restrict__ dlogits,
                                                                 const uint16_t* __restrict__ x, int64_t ldx,
                                                                 int64_t T, int E, int64_t d,
                                                                 float* __restrict__ part) {
  constexpr int U = 8;  // tokens whose x loads are in flight together
  static_assert(kDwrTok % U == 0, "token batch must divide the wave's tokens");
  __shared__ float s_dl[kDwrChunk][kDwrEG];
  __shared__ float4 red[kDwrWaves - 1][2][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t chunk = blockIdx.x;
  const int64_t col = (int64_t)blockIdx.y * 512 + lane * 8;
  const bool active = col < d;
  const int64_t t0 = chunk * kDwrChunk;
  const int64_t tb = t0 + (int64_t)wave * kDwrTok;
  for (int e0 = 0; e0 < E; e0 += kDwrEG) {
    // the chunk's dlogits for this expert pass (zero past T and past E)
    for (int i = threadIdx.x; i < kDwrChunk * kDwrEG; i += blockDim.x) {
      const int64_t t = t0 + i / kDwrEG;
      const int e = e0 + i % kDwrEG;
      s_dl[i / kDwrEG][i % kDwrEG] = (t < T && e < E) ? dlogits[t * E + e] : 0.0f;
    }
    __syncthreads();
    float acc[kDwrEG][8];
#pragma unroll
    for (int e = 0; e < kDwrEG; ++e)
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[e][q] = 0.0f;
    // tokens in order; rows past T load nothing and meet zero dlogits
    for (int u0 = 0; u0 < kDwrTok; u0 += U) {
      uint4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t t = tb + u0 + u;
        v[u] = make_uint4(0, 0, 0, 0);
        if (active && t < T) v[u] = *reinterpret_cast<const uint4*>(x + t * ldx + col);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float xv[8] = {bf_lo(v[u].x), bf_hi(v[u].x), bf_lo(v[u].y), bf_hi(v[u].y),
                             bf_lo(v[u].z), bf_hi(v[u].z), bf_lo(v[u].w), bf_hi(v[u].w)};
        const float* g = s_dl[wave * kDwrTok + u0 + u];
#pragma unroll
        for (int e = 0; e < kDwrEG; ++e) {
          const float ge = g[e];
#pragma unroll
          for (int q = 0; q < 8; ++q) acc[e][q] = __builtin_fmaf(ge, xv[q], acc[e][q]);
        }
      }
    }
    // wave-ordered sum of the four waves, one expert at a time
#pragma unroll
    for (int e = 0; e < kDwrEG; ++e) {
      if (e0 + e >= E) continue;  // uniform: every thread skips the same experts (and their barriers)
      if (wave > 0) {
        red[wave - 1][0][lane] = make_float4(acc[e][0], acc[e][1], acc[e][2], acc[e][3]);
        red[wave - 1][1][lane] = make_float4(acc[e][4], acc[e][5], acc[e][6], acc[e][7]);
      }
      __syncthreads();
      if (wave == 0 && active) {
        float s[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) s[q] = acc[e][q];
#pragma unroll
        for (int w = 0; w < kDwrWaves - 1; ++w) {
          const float4 a = red[w][0][lane], b = red[w][1][lane];
          s[0] += a.x; s[1] += a.y; s[2] += a.z; s[3] += a.w;
          s[4] += b.x; s[5] += b.y; s[6] += b.z; s[7] += b.w;
        }
        float4* dst = reinterpret_cast<float4*>(part + (chunk * E + e0 + e) * d + col);
        dst[0] = make_float4(s[0], s[1], s[2], s[3]);
        dst[1] = make_float4(s[4], s[5], s[6], s[7]);
      }
      __syncthreads();
    }
  }
}

// out[i] = sum over chunks c of part[c][i]: block 1024 = 64 outputs x kRedGroups chunk groups; each group adds its
// chunks in order (eight loads in flight), then the group sums are added in group order, so the result does not
// depend on the launch.
// dwr partials on the fp32 MFMA for E <= 16 (the chunks and partial layout of router_dwr_partial_kernel).  Wave
// w of the workgroup owns 128 columns (lane l: 8 columns 8 (l % 16) + 0..7 of them, 16 bytes of each token row) and
// all kDwrChunk tokens of the chunk, in steps of 4 tokens: v_mfma_f32_16x16x4_f32 with A = dlogits^T (16 experts x
// 4 tokens: lane l holds expert l % 16 of token l / 16) and, for column block b, B = x (4 tokens x 16 columns: lane l
// holds column 8 (l % 16) + b of token l / 16), so block b's output column n is column 8 n + b.  Experts past E get
// zero dlogits, tokens past T zero rows.  The fp32 MFMA accumulates in fp32 in a fixed order (deterministic); the
// result differs from the VALU kernel's only by fp32 rounding.
constexpr int kDwrQ = 16;  // 4-token steps whose loads are in flight together

__global__ __launch_bounds__(256) void router_dwr_mfma_kernel(const float* __restrict__ dlogits,
                                                              const uint16_t* __restrict__ x, int64_t ldx, int64_t T,
                                                              int E, int64_t d, float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int q = lane >> 4;   // token within a 4-token step (the MFMA k index)
  const int r = lane & 15;   // A: expert row; B: column group
  const int64_t chunk = blockIdx.x;
  const int64_t col = (int64_t)blockIdx.y * 512 + wave * 128 + 8 * r;  // the lane's first column
  const bool active = col < d;
  const bool expert = r < E;
  const int64_t t0 = chunk * kDwrChunk;
  f32x4 acc[8];
#pragma unroll
  for (int b = 0; b < 8; ++b) acc[b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < kDwrChunk; s0 += 4 * kDwrQ) {
    uint4 xv[kDwrQ];
    float dv[kDwrQ];
#pragma unroll
    for (int u = 0; u < kDwrQ; ++u) {
      const int64_t t = t0 + s0 + 4 * u + q;
      xv[u] = make_uint4(0, 0, 0, 0);
      dv[u] = 0.0f;
      if (t < T) {
        if (active) xv[u] = *reinterpret_cast<const uint4*>(x + t * ldx + col);
        if (expert) dv[u] = dlogits[t * E + r];
      }
    }
#pragma unroll
    for (int u = 0; u < kDwrQ; ++u) {
      const float xf[8] = {bf_lo(xv[u].x), bf_hi(xv[u].x), bf_lo(xv[u].y), bf_hi(xv[u].y),
                           bf_lo(xv[u].z), bf_hi(xv[u].z), bf_lo(xv[u].w), bf_hi(xv[u].w)};
#pragma unroll
      for (int b = 0; b < 8; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(dv[u], xf[b], acc[b], 0, 0, 0);
    }
  }
  // lane l holds, for block b, experts 4 (l / 16) + 0..3 at output column n = l % 16, i.e. column col + b
  if (!active) return;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = 4 * q + j;
    if (e >= E) continue;
    float* dst = part + (chunk * E + e) * d + col;
    *reinterpret_cast<float4*>(dst) = make_float4(acc[0][j], acc[1][j], acc[2][j], acc[3][j]);
    *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[4][j], acc[5][j], acc[6][j], acc[7][j]);
  }
}

constexpr int kRedGroups = 16;

__global__ __launch_bounds__(1024) void router_dwr_reduce_kernel(const float* __restrict__ part, int nchunk, int E,
                                                                 int64_t d, void* __restrict__ dwr, int dwr_bf16) {
  __shared__ float red[kRedGroups][64];
  const int64_t total = (int64_t)E * d;
  const int j = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int per = (nchunk + kRedGroups - 1) / kRedGroups;
  const int c0 = min(nchunk, q * per), c1 = min(nchunk, c0 + per);
  for (int64_t base = (int64_t)blockIdx.x * 64; base < total; base += (int64_t)gridDim.x * 64) {
    const int64_t i = base + j;
    float s = 0.0f;
    if (i < total) {
      int c = c0;
      for (; c + 8 <= c1; c += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(c + u) * total + i];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
      }
      for (; c < c1; ++c) s += part[(int64_t)c * total + i];
    }
    red[q][j] = s;
    __syncthreads();
    if (q == 0 && i < total) {
      float r = red[0][j];
#pragma unroll
      for (int g = 1; g < kRedGroups; ++g) r += red[g][j];
      if (dwr_bf16)
        reinterpret_cast<uint16_t*>(dwr)[i] = (uint16_t)f2bf(r);
      else
        reinterpret_cast<float*>(dwr)[i] = r;
    }
    __syncthreads();
  }
}

// dx[t] = bf16(sum_j dxs[inv_pos[t*k+j]] + sum_e dlogits[t,e] * wr[e]).  A workgroup walks tokens; each thread owns
// 8 columns of a column slab (blockIdx.y), so the token's row indices and router gradients are wave-uniform scalar
// loads.  EMAX > 0: the thread's wr columns for E <= EMAX experts stay in registers for all its tokens.
template <bool F32, int EMAX>
__global__ __launch_bounds__(256) void unpermute_bwd_kernel(const void* __restrict__ dxs,
                                                            const int32_t* __restrict__ inv_pos,
                                                            const float* __restrict__ dlogits,
                                                            const uint16_t* __restrict__ wr, int64_t T, int k,
                                                            int64_t d, int E, uint16_t* __restrict__ dx) {
  const int64_t col = ((int64_t)blockIdx.y * blockDim.x + threadIdx.x) * 8;
  const bool active = col < d;
  [[maybe_unused]] uint4 wreg[EMAX > 0 ? EMAX : 1];
  if constexpr (EMAX > 0) {
#pragma unroll
    for (int e = 0; e < EMAX; ++e) {
      wreg[e] = make_uint4(0, 0, 0, 0);
      if (dlogits && e < E && active) wreg[e] = *reinterpret_cast<const uint4*>(wr + (int64_t)e * d + col);
    }
  }
  // two tokens per pass so that both tokens' row loads are in flight together
  for (int64_t t0 = (int64_t)blockIdx.x * 2; t0 < T; t0 += (int64_t)gridDim.x * 2) {
    float s[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int q = 0; q < 8; ++q) s[u][q] = 0.0f;
    for (int j = 0; j < k; ++j) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int64_t t = t0 + u;
        if (t >= T || !active) continue;
        const int64_t r = inv_pos[t * k + j];
        if (r < 0) continue;  // an expert id outside [0, E): no sorted row, no gradient
        if constexpr (F32) {
          const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(dxs) + r * d + col);
          const float4 v0 = src[0], v1 = src[1];
          s[u][0] += v0.x;
          s[u][1] += v0.y;
          s[u][2] += v0.z;
          s[u][3] += v0.w;
          s[u][4] += v1.x;
          s[u][5] += v1.y;
          s[u][6] += v1.z;
          s[u][7] += v1.w;
        } else {
          const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(dxs) + r * d + col);
          const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            s[u][2 * q] += bf_lo(w[q]);
            s[u][2 * q + 1] += bf_hi(w[q]);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t t = t0 + u;
      if (t >= T) break;
      if (dlogits) {
        auto fma_row = [&](float g, const uint4 v) {
          const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            s[u][2 * q] = __builtin_fmaf(g, bf_lo(w[q]), s[u][2 * q]);
            s[u][2 * q + 1] = __builtin_fmaf(g, bf_hi(w[q]), s[u][2 * q + 1]);
          }
        };
        if constexpr (EMAX > 0) {
          if (E == EMAX) {  // the token's whole gradient row in four 16-byte (scalar) loads
            float g[EMAX];
#pragma unroll
            for (int q = 0; q < EMAX / 4; ++q) {
              const float4 v = reinterpret_cast<const float4*>(dlogits + t * EMAX)[q];
              g[4 * q] = v.x; g[4 * q + 1] = v.y; g[4 * q + 2] = v.z; g[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int e = 0; e < EMAX; ++e) fma_row(g[e], wreg[e]);
          } else {
            // experts past E have zero weight columns (wreg), so their (clamped, finite) router gradient adds 0
#pragma unroll
            for (int e = 0; e < EMAX; ++e) fma_row(dlogits[t * E + min(e, E - 1)], wreg[e]);
          }
        } else {
          for (int e = 0; e < E; ++e)
            fma_row(dlogits[t * E + e], active ? *reinterpret_cast<const uint4*>(wr + (int64_t)e * d + col)
                                               : make_uint4(0, 0, 0, 0));
        }
      }
      if (active) {
        uint4 o;
        o.x = pack_bf2(s[u][0], s[u][1]);
        o.y = pack_bf2(s[u][2], s[u][3]);
        o.z = pack_bf2(s[u][4], s[u][5]);
        o.w = pack_bf2(s[u][6], s[u][7]);
        *reinterpret_cast<uint4*>(dx + t * d + col) = o;
      }
    }
  }
}

static inline int grid_for(int64_t work, int per_block, int cap = 8192) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return (int)g;
}

static inline bool al16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <bool F16>
static void combine_launch(const uint16_t* y, const int32_t* inv_pos, int64_t T, int k, int64_t d,
                           const uint16_t* add, uint16_t* out, int64_t work, hipStream_t s) {
  const dim3 grid(grid_for(work, 256, 65536));
#define HMOE_COMBINE(KT) \
  hipLaunchKernelGGL((combine_kernel<KT, F16>), grid, dim3(256), 0, s, y, inv_pos, T, k, d, add, out)
  switch (k) {
    case 1: HMOE_COMBINE(1); break;
    case 2: HMOE_COMBINE(2); break;
    case 4: HMOE_COMBINE(4); break;
    case 6: HMOE_COMBINE(6); break;
    case 8: HMOE_COMBINE(8); break;
    default: HMOE_COMBINE(0); break;
  }
#undef HMOE_COMBINE
}

// the dynamic LDS of the larger router instantiations (up to 157 KB) is declared once per device before the launch
template <int NW, int NB, int TT, bool SIG>
static int mfma_route_launch(int grid, hipStream_t s, const uint16_t* x, int64_t ldx, const uint16_t* wr,
                             const float* bias, int T, int d, int E, int k, int renorm, float scaling, float* out,
                             int32_t* ids, float* w, int n_group, int topk_group) {
  auto kern = route_mfma_kernel<NW, NB, TT, SIG>;
  constexpr int TB = 16 * TT, ER = 16 * NB * NW;
  constexpr int kLds = 2 * (TB + ER) * kSmPitch;
  static std::atomic<bool> attr_set[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return HMOE_ERR_DEVICE;
  if (!attr_set[dev].load(std::memory_order_acquire)) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize, kLds) !=
        hipSuccess)
      return HMOE_ERR_LAUNCH;
    attr_set[dev].store(true, std::memory_order_release);
  }
  hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * NW), kLds, s, x, ldx, wr, bias, T, d, E, k, renorm, scaling, out,
                     ids, w, n_group, topk_group);
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

// Up to this many (token, expert) logits, given a logits / scores buffer, the routers with E > 16 (the sigmoid
// router for any E) take the two-launch form (route_block_logits_kernel + route_select_kernel).  Same-process A/Bs
// against route_mfma_kernel: sigmoid E = 128 at 64 / 512 / 2048 / 4096 tokens 20.1 / 20.5 / 36.2 / 59.0 against
// 40.1 / 40.7 / 40.8 / 42.8 us, E = 256 at 333 tokens 33.8 against 60.2; softmax E = 64 at 256 / 2048 / 4096 / 16384
// tokens 14.1 / 16.2 / 25.7 / 104.8 against 36.2 / 26.7 / 27.2 / 68.2.
constexpr int64_t kRouteBlockTE = 1 << 18;

// the two-launch form: block logits into lgbuf, then the selection over it
template <bool SIG>
static int block_route_launch(hipStream_t s, const uint16_t* x, int64_t ldx, const uint16_t* wr, const float* bias,
                              int T, int d, int E, int k, int renorm, float scaling, float* lgbuf, int32_t* ids,
                              float* w, int n_group, int topk_group) {
  hipLaunchKernelGGL(route_block_logits_kernel, dim3((unsigned)((T + 15) / 16), (unsigned)((E + 15) / 16)),
                     dim3(256), 0, s, x, ldx, wr, T, d, E, lgbuf);
  HMOE_CHECK_LAUNCH();
  const int nwv = SIG ? (T + 3) / 4 : T;  // waves: four tokens each (sigmoid) or one
  const dim3 grid((unsigned)((nwv + 3) / 4));
  // the sigmoid selection holds E / 16 expert slots per lane (4, 8 or 16, as in route_mfma_kernel)
  constexpr int EPS_MID = SIG ? 8 : 4, EPS_MAX = SIG ? 16 : 4;
  if (!SIG || E <= 64)
    hipLaunchKernelGGL((route_select_kernel<SIG, 4>), grid, dim3(256), 0, s, bias, T, E, k, renorm, scaling, lgbuf,
                       ids, w, n_group, topk_group);
  else if (E <= 128)
    hipLaunchKernelGGL((route_select_kernel<SIG, EPS_MID>), grid, dim3(256), 0, s, bias, T, E, k, renorm, scaling,
                       lgbuf, ids, w, n_group, topk_group);
  else
    hipLaunchKernelGGL((route_select_kernel<SIG, EPS_MAX>), grid, dim3(256), 0, s, bias, T, E, k, renorm, scaling,
                       lgbuf, ids, w, n_group, topk_group);
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

// waves per 16-token tile of the E <= 16 router by token count, from same-process A/Bs at d = 1536, E = 16 (one /
// two / four waves): 2048 tokens 17.0 / 12.3 / 11.6 us, 4096 17.0 / 12.4 / 11.6, 8192 20.5 / 12.6 / 14.9, 16384
// 20.9 / 20.0 / 25.7, 32768 32.9 / 33.8 / 46.3
constexpr int64_t kRouteSplit4T = 6144, kRouteSplit2T = 24576;

static int route_launch(const void* x, int64_t ldx, const void* wr, const float* bias, int64_t T, int64_t d, int E,
                        int k, int renorm, float scaling, float* logits, int32_t* topk_ids, float* topk_w,
                        hipStream_t s) {
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(wr);
  if (E <= 16) {
    // four waves per 16-token tile below kRouteSplit4T tokens, two below kRouteSplit2T, else one (four tiles per
    // workgroup)
    if (T < kRouteSplit4T) {
      hipLaunchKernelGGL(route_topk_direct_kernel<4>, dim3((unsigned)((T + 15) / 16)), dim3(256), 0, s, xp, ldx, wp,
                         bias, (int)T, (int)d, E, k, renorm, scaling, logits, topk_ids, topk_w);
    } else if (T < kRouteSplit2T) {
      hipLaunchKernelGGL(route_topk_direct_kernel<2>, dim3((unsigned)((T + 31) / 32)), dim3(256), 0, s, xp, ldx, wp,
                         bias, (int)T, (int)d, E, k, renorm, scaling, logits, topk_ids, topk_w);
    } else {
      hipLaunchKernelGGL(route_topk_direct_kernel<1>, dim3((unsigned)((T + 63) / 64)), dim3(256), 0, s, xp, ldx, wp,
                         bias, (int)T, (int)d, E, k, renorm, scaling, logits, topk_ids, topk_w);
    }
    HMOE_CHECK_LAUNCH();
    return HMOE_OK;
  }
  if (T * E <= kRouteBlockTE && logits)
    return block_route_launch<false>(s, xp, ldx, wp, bias, (int)T, (int)d, E, k, renorm, scaling, logits, topk_ids,
                                     topk_w, 1, 1);
#define HMOE_RT(NW, NB, TT)                                                                                      \
  return mfma_route_launch<NW, NB, TT, false>((int)((T + 16 * (TT) - 1) / (16 * (TT))), s, xp, ldx, wp, bias,    \
                                              (int)T, (int)d, E, k, renorm, scaling, logits, topk_ids, topk_w, 1, 1)
  // the experts split over the waves
  const int tt = T >= 8192 ? 2 : 1;
  if (E <= 64) {
    if (tt == 2) HMOE_RT(4, 1, 2);
    HMOE_RT(4, 1, 1);
  }
  if (E <= 128) {
    if (tt == 2) HMOE_RT(8, 1, 2);
    HMOE_RT(8, 1, 1);
  }
  if (tt == 2) HMOE_RT(8, 2, 2);
  HMOE_RT(8, 2, 1);
#undef HMOE_RT
}

static int route_check(const void* x, int64_t ldx, const void* wr, int64_t T, int64_t d, int E, int k,
                       const int32_t* topk_ids, const float* topk_w) {
  if (T < 0 || d <= 0 || E <= 0 || k <= 0) return HMOE_ERR_ARG;
  if (T == 0) return HMOE_OK;
  if (!x || !wr || !topk_ids || !topk_w) return HMOE_ERR_ARG;
  if (E > kRouteMaxE || k > kMaxK || k > E || T > INT32_MAX) return HMOE_ERR_SHAPE;
  if (d % 8 || ldx % 8 || ldx < d || !al16(x) || !al16(wr)) return HMOE_ERR_ARG;
  return HMOE_OK;
}

static size_t dispatch_ws_bytes(int64_t T, int k, int E) {
  const int64_t M = T * k;
  const int64_t nblk = (M + kFPB - 1) / kFPB;
  const size_t hist = (size_t)(nblk > 0 ? nblk : 1) * (size_t)E * 4;
  const size_t rank = (size_t)(M > 0 ? M : 1) * 4;
  const size_t gst = (size_t)(E + 1) * 4;  // row-group starts of the tiles
  return ((hist + 255) / 256) * 256 + ((rank + 255) / 256) * 256 + ((gst + 255) / 256) * 256;
}

// hmoe_dispatch with its workspace given: every argument is checked before the first launch, so an error leaves
// counts / starts untouched.  The workspace holds the per-block histograms (then their exclusive offsets) and the
// per-row ranks; each call writes every entry it later reads, so nothing in it has to start at zero.
static int dispatch_impl(const void* topk_ids, int ids_dtype, const void* topk_w, int w_dtype, int64_t T, int k, int E,
                         const void* x, int64_t ldx, int64_t d, void* xs, void* xs_tiles, int32_t* counts,
                         int64_t* counts64, int32_t* starts, int32_t* order, int32_t* a_idx, int32_t* inv_pos,
                         uint16_t* w_sorted, int32_t* n_invalid, void* workspace, size_t workspace_bytes,
                         int dtype, hipStream_t s) {
  if (T < 0 || k <= 0 || E <= 0) return HMOE_ERR_ARG;
  if (E > kMaxEDispatch || k > kMaxK) return HMOE_ERR_SHAPE;
  if (!counts || !starts) return HMOE_ERR_ARG;
  if (ids_dtype != HMOE_DT_I32 && ids_dtype != HMOE_DT_I64) return HMOE_ERR_DTYPE;
  if (topk_w && w_dtype != HMOE_DT_F32 && w_dtype != HMOE_DT_BF16 && w_dtype != HMOE_DT_F16) return HMOE_ERR_DTYPE;
  if (dtype != HMOE_DT_BF16 && dtype != HMOE_DT_F16) return HMOE_ERR_DTYPE;
  const bool f16 = dtype == HMOE_DT_F16;
  if (w_sorted && !topk_w) return HMOE_ERR_ARG;
  const int64_t M = T * k;
  if (M > INT32_MAX) return HMOE_ERR_SHAPE;
  if (M > 0 && (!topk_ids || !order)) return HMOE_ERR_ARG;
  // the row copies read x only when there are rows
  if (xs && M > 0 && (!x || d <= 0 || d % 8 || ldx % 8 || ldx < d || !al16(x) || !al16(xs))) return HMOE_ERR_ARG;
  if (xs_tiles && M > 0 && (!x || d <= 0 || d % 8 || ldx % 8 || ldx < d || !al16(x) || !al16(xs_tiles)))
    return HMOE_ERR_ARG;
  if (workspace_bytes < dispatch_ws_bytes(T, k, E) || !workspace) return HMOE_ERR_WORKSPACE;
  const int64_t nblk = (M + kFPB - 1) / kFPB;
  int32_t* hist = static_cast<int32_t*>(workspace);
  const size_t hist_bytes = (((size_t)(nblk > 0 ? nblk : 1) * (size_t)E * 4 + 255) / 256) * 256;
  int32_t* rank = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + hist_bytes);
  const size_t rank_bytes = (((size_t)(M > 0 ? M : 1) * 4 + 255) / 256) * 256;
  int32_t* gstart = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + hist_bytes + rank_bytes);
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  const int ids64 = ids_dtype == HMOE_DT_I64;
  // the one-workgroup pass up to 8192 rows with E <= 16, 4096 above (kernel time at 8192 rows and 64 or 128
  // experts: 16.3 and 18.9 us, the three passes about 14)
  if (!xs && !xs_tiles && M <= (E <= 16 ? kSmallM : kSmallM / 2) && E <= kSmallE) {
    hipLaunchKernelGGL(dispatch_small_kernel, dim3(1), dim3(1024), 0, s, topk_ids, ids64, topk_w, w_dtype, (int)f16,
                       M, k, E, nbits, counts, counts64, starts, order, a_idx, inv_pos, w_sorted, n_invalid);
    HMOE_CHECK_LAUNCH();
    return HMOE_OK;
  }
  if (M > 0) {
    hipLaunchKernelGGL(dispatch_hist_kernel, dim3((unsigned)nblk), dim3(64), 0, s, topk_ids, ids64, M, E, nbits,
                       hist, rank);
    HMOE_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(dispatch_scan_kernel, dim3(1), dim3(1024), 0, s, hist, (int)nblk, E, counts, counts64, starts,
                     gstart, M, n_invalid);
  HMOE_CHECK_LAUNCH();
  if (M > 0 && (xs || xs_tiles)) {
    const int grid = grid_for(T, 4, 8192);
#define HMOE_SCAT(KT)                                                                                              \
  hipLaunchKernelGGL(dispatch_scatter_kernel<KT>, dim3(grid), dim3(256), 0, s, topk_ids, ids64, topk_w, w_dtype,      \
                     (int)f16, T, k, E, hist, rank, static_cast<const uint16_t*>(x), ldx, d,                        \
                     static_cast<uint16_t*>(xs), order, a_idx, inv_pos, w_sorted, static_cast<char*>(xs_tiles),      \
                     starts, gstart)
    if (k == 1)
      HMOE_SCAT(1);
    else if (k == 2)
      HMOE_SCAT(2);
    else if (k == 4)
      HMOE_SCAT(4);
    else if (k == 8)
      HMOE_SCAT(8);
    else
      HMOE_SCAT(0);
#undef HMOE_SCAT
    HMOE_CHECK_LAUNCH();
  } else if (M > 0) {
    hipLaunchKernelGGL(dispatch_index_kernel, dim3(grid_for(M, 256, 8192)), dim3(256), 0, s, topk_ids, ids64, topk_w,
                       w_dtype, (int)f16, M, k, E, hist, rank, order, a_idx, inv_pos, w_sorted);
    HMOE_CHECK_LAUNCH();
  }
  return HMOE_OK;
}

// Device scratch of hmoe_dispatch_noalloc: the workspace hmoe_dispatch would take, as a file-scope device array (one
// copy per GPU, held until the process ends).  Host code never uses this name as an address: its device address is
// looked up once per device with hipGetSymbolAddress and kept in g_scratch_ptr.
constexpr size_t kDispatchScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[kDispatchScratchBytes];
static std::atomic<void*> g_scratch_ptr[64];

// The current device's address of `scratch` (nullptr with *rc set when the device or the lookup fails).
static void* dispatch_scratch(int* rc) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    *rc = HMOE_ERR_DEVICE;
    return nullptr;
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
      *rc = HMOE_ERR_DEVICE;
      return nullptr;
    }
    g_scratch_ptr[dev].store(p, std::memory_order_release);  // racing first calls store the same address
  }
  *rc = HMOE_OK;
  return p;
}

}  // namespace hmoe

using namespace hmoe;

extern "C" {

int hmoe_abi_version(void) { return HMOE_ABI_VERSION; }

const char* hmoe_error_string(int code) {
  switch (code) {
    case HMOE_OK: return "ok";
    case HMOE_ERR_ARG: return "invalid argument (null pointer, negative size or misaligned pointer / stride)";
    case HMOE_ERR_SHAPE: return "unsupported shape";
    case HMOE_ERR_DTYPE: return "unsupported element type";
    case HMOE_ERR_LAUNCH: return "kernel launch failed";
    case HMOE_ERR_WORKSPACE: return "workspace missing or too small";
    case HMOE_ERR_DEVICE: return "device query failed";
    case HMOE_ERR_TOO_LARGE:
      return "input too large for the fixed device scratch of an allocation-free entry point (use the workspace form)";
    default: return "unknown error";
  }
}

int hmoe_route_topk(const void* x, int64_t ldx, const void* wr, const float* bias, int64_t T, int64_t d, int E,
                    int k, int renorm, float scaling, float* logits, int32_t* topk_ids, float* topk_w,
                    hmoe_stream_t stream) {
  const int rc = route_check(x, ldx, wr, T, d, E, k, topk_ids, topk_w);
  if (rc || T == 0) return rc;
  return route_launch(x, ldx, wr, bias, T, d, E, k, renorm, scaling, logits, topk_ids, topk_w,
                      reinterpret_cast<hipStream_t>(stream));
}

int hmoe_route_sigmoid_group(const void* x, int64_t ldx, const void* wr, const float* expert_bias, int64_t T,
                             int64_t d, int E, int k, int n_group, int topk_group, float scaling, float* scores,
                             int32_t* topk_ids, float* topk_w, hmoe_stream_t stream) {
  const int rc = route_check(x, ldx, wr, T, d, E, k, topk_ids, topk_w);
  if (rc || T == 0) return rc;
  if (n_group < 1 || topk_group < 1 || topk_group > n_group || E % n_group) return HMOE_ERR_SHAPE;
  if (topk_group < n_group) {
    const int eg = E / n_group;  // experts per group: a power of two in [2, 64]
    if (eg < 2 || eg > 64 || (eg & (eg - 1))) return HMOE_ERR_SHAPE;
    if (k > topk_group * eg) return HMOE_ERR_SHAPE;  // the kept groups must hold k experts
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // waves x 16-expert blocks per wave cover E; two 16-token tiles per workgroup once that still gives a workgroup
  // per CU (8192 tokens), else one
  const int nw = E <= 64 ? 4 : 8, nb = E <= 128 ? 1 : 2, tt = T >= 8192 ? 2 : 1;
  const int grid = (int)((T + 16 * tt - 1) / (16 * tt));
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(wr);
  if (T * E <= kRouteBlockTE && scores)
    return block_route_launch<true>(s, xp, ldx, wp, expert_bias, (int)T, (int)d, E, k, 1, scaling, scores, topk_ids,
                                    topk_w, n_group, topk_group);
#define HMOE_SG(NW, NB, TT)                                                                                      \
  return mfma_route_launch<NW, NB, TT, true>(grid, s, xp, ldx, wp, expert_bias, (int)T, (int)d, E, k, 1,        \
                                                    scaling, scores, topk_ids, topk_w, n_group, topk_group)
  if (nw == 4 && tt == 2) HMOE_SG(4, 1, 2);
  if (nw == 4) HMOE_SG(4, 1, 1);
  if (nb == 1 && tt == 2) HMOE_SG(8, 1, 2);
  if (nb == 1) HMOE_SG(8, 1, 1);
  if (tt == 2) HMOE_SG(8, 2, 2);
  HMOE_SG(8, 2, 1);
#undef HMOE_SG
}

size_t hmoe_dispatch_workspace_size(int64_t T, int k, int E) { return dispatch_ws_bytes(T, k, E); }

int hmoe_dispatch(const void* topk_ids, int ids_dtype, const void* topk_w, int w_dtype, int64_t T, int k, int E,
                  const void* x, int64_t ldx, int64_t d, void* xs, int32_t* counts, int64_t* counts64,
                  int32_t* starts, int32_t* order, int32_t* a_idx, int32_t* inv_pos, uint16_t* w_sorted,
                  int32_t* n_invalid, void* workspace, size_t workspace_bytes, int dtype, hmoe_stream_t stream) {
  return dispatch_impl(topk_ids, ids_dtype, topk_w, w_dtype, T, k, E, x, ldx, d, xs, nullptr, counts, counts64, starts,
                       order, a_idx, inv_pos, w_sorted, n_invalid, workspace, workspace_bytes, dtype,
                       reinterpret_cast<hipStream_t>(stream));
}

size_t hmoe_xs_tiles_bytes(int64_t M, int E, int64_t d) {
  return (M < 0 || E <= 0 || d <= 0) ? 0 : (size_t)tiles_bytes(M, E, d);
}

int hmoe_dispatch_tiles(const void* topk_ids, int ids_dtype, const void* topk_w, int w_dtype, int64_t T, int k, int E,
                        const void* x, int64_t ldx, int64_t d, void* xs, void* xs_tiles, int32_t* counts,
                        int64_t* counts64, int32_t* starts, int32_t* order, int32_t* a_idx, int32_t* inv_pos,
                        uint16_t* w_sorted, int32_t* n_invalid, void* workspace, size_t workspace_bytes, int dtype,
                        hmoe_stream_t stream) {
  return dispatch_impl(topk_ids, ids_dtype, topk_w, w_dtype, T, k, E, x, ldx, d, xs, xs_tiles, counts, counts64,
                       starts, order, a_idx, inv_pos, w_sorted, n_invalid, workspace, workspace_bytes, dtype,
                       reinterpret_cast<hipStream_t>(stream));
}

int hmoe_dispatch_noalloc(const void* topk_ids, int ids_dtype, const void* topk_w, int w_dtype, int64_t T, int k,
                          int E, const void* x, int64_t ldx, int64_t d, void* xs, int32_t* counts, int64_t* counts64,
                          int32_t* starts, int32_t* order, int32_t* a_idx, int32_t* inv_pos, uint16_t* w_sorted,
                          int32_t* n_invalid, int dtype, hmoe_stream_t stream) {
  if (T < 0 || k <= 0 || E <= 0) return HMOE_ERR_ARG;
  if (E > kMaxEDispatch || k > kMaxK) return HMOE_ERR_SHAPE;
  if (T > INT32_MAX / k || dispatch_ws_bytes(T, k, E) > kDispatchScratchBytes) return HMOE_ERR_TOO_LARGE;
  int rc = HMOE_OK;
  void* ws = dispatch_scratch(&rc);
  if (rc) return rc;
  return dispatch_impl(topk_ids, ids_dtype, topk_w, w_dtype, T, k, E, x, ldx, d, xs, nullptr, counts, counts64, starts,
                       order, a_idx, inv_pos, w_sorted, n_invalid, ws, kDispatchScratchBytes, dtype,
                       reinterpret_cast<hipStream_t>(stream));
}

int hmoe_make_schedule(const void* counts, int counts_dtype, int E, int64_t M, int block_m, int32_t* block_e,
                       int32_t* block_row, int32_t* row_end, hmoe_stream_t stream) {
  if (!counts || !block_e || !block_row || !row_end || E <= 0 || M < 0 || block_m <= 0) return HMOE_ERR_ARG;
  if (E > kMaxEDispatch) return HMOE_ERR_SHAPE;
  if (counts_dtype != HMOE_DT_I32 && counts_dtype != HMOE_DT_I64) return HMOE_ERR_DTYPE;
  const int64_t nb = (M + block_m - 1) / block_m + E;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(make_schedule_kernel, dim3(grid_for(nb, 256, 1024)), dim3(256), 0, s, counts,
                     counts_dtype == HMOE_DT_I64, E, nb, block_m, block_e, block_row, row_end);
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

int hmoe_combine(const void* y, const int32_t* inv_pos, int64_t T, int k, int64_t d, void* out, int dtype,
                 hmoe_stream_t stream) {
  if (T < 0 || k <= 0 || d <= 0) return HMOE_ERR_ARG;
  if (dtype != HMOE_DT_BF16 && dtype != HMOE_DT_F16) return HMOE_ERR_DTYPE;
  if (T == 0) return HMOE_OK;
  if (!y || !out || d % 8 || !al16(y) || !al16(out)) return HMOE_ERR_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t work = T * (d / 8);
  if (dtype == HMOE_DT_F16)
    combine_launch<true>(static_cast<const uint16_t*>(y), inv_pos, T, k, d, nullptr, static_cast<uint16_t*>(out), work,
                         s);
  else
    combine_launch<false>(static_cast<const uint16_t*>(y), inv_pos, T, k, d, nullptr, static_cast<uint16_t*>(out), work,
                          s);
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

int hmoe_combine_add(const void* y, const int32_t* inv_pos, int64_t T, int k, int64_t d, const void* add, void* out,
                     int dtype, hmoe_stream_t stream) {
  if (T < 0 || k <= 0 || d <= 0) return HMOE_ERR_ARG;
  if (dtype != HMOE_DT_BF16 && dtype != HMOE_DT_F16) return HMOE_ERR_DTYPE;
  if (T == 0) return HMOE_OK;
  if (!y || !add || !out || d % 8 || !al16(y) || !al16(add) || !al16(out)) return HMOE_ERR_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t work = T * (d / 8);
  if (dtype == HMOE_DT_F16)
    combine_launch<true>(static_cast<const uint16_t*>(y), inv_pos, T, k, d, static_cast<const uint16_t*>(add),
                         static_cast<uint16_t*>(out), work, s);
  else
    combine_launch<false>(static_cast<const uint16_t*>(y), inv_pos, T, k, d, static_cast<const uint16_t*>(add),
                          static_cast<uint16_t*>(out), work, s);
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

int hmoe_combine_bwd(const void* dout, const void* yhat, const int32_t* order, const int32_t* a_idx,
                     const uint16_t* w_sorted, int64_t M, int k, int64_t d, void* dys, float* dtopk_w,
                     hmoe_stream_t stream) {
  if (M < 0 || k <= 0 || d <= 0) return HMOE_ERR_ARG;
  if (M == 0) return HMOE_OK;
  const bool dw = yhat != nullptr;  // without yhat: the scaled rows only (dtopk_w and order unused)
  if (!dout || !a_idx || !w_sorted || !dys || (dw && (!order || !dtopk_w))) return HMOE_ERR_ARG;
  if (d % 8 || !al16(dout) || !al16(yhat) || !al16(dys)) return HMOE_ERR_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define HMOE_CBWD(DW)                                                                                              \
  hipLaunchKernelGGL((combine_bwd_kernel<DW>), dim3(grid_for(M, 4, 16384)), dim3(256), 0, s,                        \
                     static_cast<const uint16_t*>(dout), static_cast<const uint16_t*>(yhat), order, a_idx, w_sorted, \
                     M, k, d, static_cast<uint16_t*>(dys), dtopk_w)
  if (dw)
    HMOE_CBWD(true);
  else
    HMOE_CBWD(false);
#undef HMOE_CBWD
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

size_t hmoe_router_bwd_workspace_size(int64_t T, int E, int64_t d) {
  const int64_t nchunk = (T + kDwrChunk - 1) / kDwrChunk;
  return (size_t)(nchunk > 0 ? nchunk : 1) * (size_t)E * (size_t)d * 4;
}

int hmoe_router_bwd(const float* logits, const int32_t* topk_ids, const float* dtopk_w, int64_t T, int E, int k,
                    int renorm, float scaling, const void* x, int64_t ldx, int64_t d, float* dlogits, void* dwr,
                    int dwr_dtype, void* workspace, size_t workspace_bytes, hmoe_stream_t stream) {
  if (T < 0 || E <= 0 || k <= 0 || d <= 0) return HMOE_ERR_ARG;
  if (E > kRouteMaxE || k > kMaxK) return HMOE_ERR_SHAPE;
  // T = 0 still writes dwr (zeros); nothing per token is read or written then, so those pointers may be NULL
  if (T > 0 && (!logits || !topk_ids || !dtopk_w || !dlogits)) return HMOE_ERR_ARG;
  if (dwr && dwr_dtype != HMOE_DT_F32 && dwr_dtype != HMOE_DT_BF16) return HMOE_ERR_DTYPE;
  if (dwr && ((T > 0 && !x) || d % 8 || ldx % 8 || ldx < d || !al16(x))) return HMOE_ERR_ARG;
  if (dwr && (!workspace || workspace_bytes < hmoe_router_bwd_workspace_size(T, E, d))) return HMOE_ERR_WORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (T > 0) {
    if (E <= 16)
      hipLaunchKernelGGL(router_dlogits16_kernel, dim3(grid_for(T, 16, 8192)), dim3(256), 0, s, logits, topk_ids,
                         dtopk_w, T, E, k, renorm, scaling, dlogits);
    else
      hipLaunchKernelGGL(router_dlogits_kernel, dim3(grid_for(T, 4, 8192)), dim3(256), 0, s, logits, topk_ids,
                         dtopk_w, T, E, k, renorm, scaling, dlogits);
    HMOE_CHECK_LAUNCH();
  }
  if (dwr) {
    const int nchunk = (int)((T + kDwrChunk - 1) / kDwrChunk);
    float* part = static_cast<float*>(workspace);
    if (nchunk > 0) {
      if (E <= 16)
        hipLaunchKernelGGL(router_dwr_mfma_kernel, dim3(nchunk, (unsigned)((d + 511) / 512)), dim3(256), 0, s,
                           dlogits, static_cast<const uint16_t*>(x), ldx, T, E, d, part);
      else
        hipLaunchKernelGGL(router_dwr_partial_kernel, dim3(nchunk, (unsigned)((d + 511) / 512)), dim3(256), 0, s,
                           dlogits, static_cast<const uint16_t*>(x), ldx, T, E, d, part);
      HMOE_CHECK_LAUNCH();
    }
    hipLaunchKernelGGL(router_dwr_reduce_kernel, dim3(grid_for((int64_t)E * d, 64, 4096)), dim3(1024), 0, s, part,
                       nchunk, E, d, dwr, dwr_dtype == HMOE_DT_BF16);
    HMOE_CHECK_LAUNCH();
  }
  return HMOE_OK;
}

int hmoe_unpermute_bwd(const void* dxs, int dxs_dtype, const int32_t* inv_pos, const float* dlogits, const void* wr,
                       int64_t T, int k, int64_t d, int E, void* dx, hmoe_stream_t stream) {
  if (T < 0 || k <= 0 || d <= 0) return HMOE_ERR_ARG;
  if (T == 0) return HMOE_OK;
  if (dxs_dtype != HMOE_DT_BF16 && dxs_dtype != HMOE_DT_F32) return HMOE_ERR_DTYPE;
  if (!dxs || !inv_pos || !dx || d % 8 || !al16(dxs) || !al16(dx)) return HMOE_ERR_ARG;
  if (dlogits && (!wr || E <= 0 || !al16(wr))) return HMOE_ERR_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // one thread per 8 columns, up to 256 threads per column slab; workgroups walk the tokens
  const int64_t vec = d / 8;
  const int threads = (int)(vec >= 256 ? 256 : ((vec + 63) / 64) * 64);
  const unsigned slabs = (unsigned)((vec + threads - 1) / threads);
  const unsigned tgrid = (unsigned)((T + 1) / 2 < 4096 ? (T + 1) / 2 : 4096);
  const uint16_t* wp = static_cast<const uint16_t*>(wr);
  uint16_t* dxp = static_cast<uint16_t*>(dx);
  const bool regs = dlogits == nullptr || E <= 16;
#define HMOE_UNPERM(F, EM)                                                                                         \
  hipLaunchKernelGGL((unpermute_bwd_kernel<F, EM>), dim3(tgrid, slabs), dim3(threads), 0, s, dxs, inv_pos, dlogits, \
                     wp, T, k, d, E, dxp)
  if (dxs_dtype == HMOE_DT_F32) {
    if (regs)
      HMOE_UNPERM(true, 16);
    else
      HMOE_UNPERM(true, 0);
  } else {
    if (regs)
      HMOE_UNPERM(false, 16);
    else
      HMOE_UNPERM(false, 0);
  }
#undef HMOE_UNPERM
  HMOE_CHECK_LAUNCH();
  return HMOE_OK;
}

}  // extern "C"
