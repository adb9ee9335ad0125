// fp32 MFMA contraction for the CROWN backward pass (gfx950).
//
//   C[M, N] = A'[M, K] x B[K, N]
//
// M = domains x specs (the coefficient rows), K = current-layer neurons,
// N = previous-layer neurons.  A' is either A itself or A after the ReLU
// relaxation of the layer (boundflow/runtime/crown_ibp.py:1211-1298), applied
// while the A tile is staged into LDS from a per-(domain, neuron) table of
// slopes/intercepts; the row reductions the relaxation needs (the bias terms
// sum_k A * beta_sel and sum_k A' * bias_k, and optionally a center term
// sum_k A' * c_k) are produced in the same pass.  The epilogue either stores C
// (optionally plus a rank-1 term) or reduces |C| (optionally weighted) along
// each row -- the Linf / box concretization norm
// (boundflow/runtime/perturbation.py:175-222, 327-359) fused so that the final
// [M, input] coefficient never reaches HBM.
//
// Tiling (template Tile<BM, BN, BK, NWM, NWN, OCC>): NWM x NWN wave64s per
// workgroup, each owning a (BM/NWM) x (BN/NWN) sub-tile of 32 x 32
// v_mfma_f32_32x32x2f32 blocks.  The two lane halves of a wave take the two
// halves of the K tile (a fixed permutation of the reduction order), so a
// lane's A (and transposed B) operands for four consecutive k-steps are one
// 128-bit LDS read.  Global tiles are read as float4 and double-buffered in LDS
// with one barrier per K tile.  Workgroups are mapped to tiles XCD-aware: each
// of the 8 XCDs receives a contiguous run of tiles, so the column tiles that
// share an A row-block share that XCD's L2.
//
// This header holds the kernel template and its launcher; each tile
// configuration is instantiated in its own translation unit (bf_gemm_tile_*.hip)
// so that the configurations compile in parallel.

#pragma once

#include <type_traits>

#include "bf_common.h"
#include "bf_gemm_args.h"

namespace bf {

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Partial-norm granularity of the |C| epilogue (columns per partial sum); every
// tile configuration used with EPI_ABSSUM has BN == NORM_BN.
constexpr int NORM_BN = 128;

// DL_ONLY_: the configuration is built for the direct-to-LDS loop alone (its
// occupancy needs that loop's LDS footprint); other operands are refused.
template <int BM_, int BN_, int BK_, int NWM_, int NWN_, int OCC_, bool DL_ONLY_ = false>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, NWM = NWM_, NWN = NWN_, OCC = OCC_;
  static constexpr bool DL_ONLY = DL_ONLY_;
  static constexpr int NT = 64 * NWM * NWN;          // threads (OCC: workgroups per CU, see gemm_waves_per_simd)
  static constexpr int WTM = BM / NWM;               // wave tile rows
  static constexpr int WTN = BN / NWN;               // wave tile cols
  static constexpr int FM = WTM / 32;                // 32x32 MFMA blocks per wave (rows)
  static constexpr int FN = WTN / 32;                // (cols)
  static constexpr int AP = BK + 4;                  // As row pitch (row-major along k)
  static constexpr int BPT = BK + 4;                 // Bs row pitch (n-major [n][k], for either B layout)
  static constexpr int KQ = BK / 4;                  // float4 per A row per K tile
  static constexpr int A_SLOTS = BM * BK / 4 / NT;
  static constexpr int B_QUADS = BN * BK / 4;         // float4 of a B tile
  static constexpr int B_SLOTS = (B_QUADS + NT - 1) / NT;
  static constexpr bool B_FULL = B_QUADS % NT == 0;   // else the last slot is partly idle
  static constexpr int RPP = NT / KQ;                // A rows covered per slot index
  static constexpr int BS_FLOATS = BN * BPT;
  // Relaxation operands staged in LDS per K tile: one (domain, k) entry per
  // thread of the first TAB_ENTRIES, so a tile whose rows span at most TAB_DOMS
  // domains reads them there (16 domains: every tile when S >= 9).
  static constexpr int TAB_ENTRIES = NT < 256 ? NT : 256;
  static constexpr int TAB_DOMS = TAB_ENTRIES / BK;
  // LDS stages of the direct-to-LDS loop: three, or two when four workgroups share a CU
  static constexpr int DL_STAGES = OCC >= 4 ? 2 : 3;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32");
  static_assert((BM * BK) % (4 * NT) == 0 && NT % KQ == 0, "tile/thread mismatch");
  static_assert((BK & (BK - 1)) == 0 && BK >= 8, "BK must be a power of two >= 8");
};

__device__ __forceinline__ float fsel(const float4& r, bool lower, bool nonneg, float* beta) {
  // upper: A >= 0 -> (alpha_u, beta_u) else (alpha_l, beta_l); lower: mirrored
  const bool use_u = lower ? !nonneg : nonneg;
  *beta = use_u ? r.y : r.w;
  return use_u ? r.x : r.z;
}

// Occupancy target of an instantiation, in waves per SIMD (the second argument
// of __launch_bounds__): OCC workgroups per CU for the plain prologue; the
// relaxation prologue keeps OCC waves per SIMD (a register budget of 512 / OCC),
// since binding its larger state to the plain kernel's budget spills.
template <int PRO, class T>
constexpr int gemm_waves_per_simd() {
  constexpr int per_simd = (T::OCC * T::NT + 255) / 256;   // OCC workgroups' waves, the busiest SIMD
  return (PRO == PRO_PLAIN && per_simd > T::OCC) ? per_simd : T::OCC;
}

// LDS-DMA waits and the workgroup barrier of the direct-to-LDS main loop, as
// inline assembly so that the compiler adds no wait of its own for the copies
// still in flight (a fence would wait for every one of them).
// One global_load_lds_dwordx4: lane l's 16 bytes at src land at lds_dst + 16 l
// (lds_dst wave-uniform).  Issued as inline assembly so that the compiler does
// not track the copy and adds no wait before the LDS reads of other stages; the
// loop orders it with wait_vmem and lds_barrier.  M0 holds the LDS address (no
// other code of the kernel uses M0).
typedef __attribute__((address_space(3))) float lds_float;
__device__ __forceinline__ void lds_copy16(const float* src, float* lds_dst) {
  const uint32_t off = (uint32_t)(uintptr_t)((lds_float*)lds_dst);
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(off) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Reduction of the 16 row values a lane holds in a 32 x 32 MFMA block (row index r of
// acc[..][r]) over the 32 lanes of its half-wave (the block's columns), by recursive
// halving: at the step across lane bit b (16, 8, 4, 2, 1) a lane keeps the half of its
// values whose row bit matches its own lane bit and joins the partner's copy of them.
// The pairs are those of the butterfly over lanes ^16, ^8, ^4, ^2, ^1, whose lanes all
// end with the same bits (join is commutative), so the result is the butterfly's bit for
// bit, with 16 exchanges per lane instead of 80.  Lane lrow ends with row index lrow >> 1.
struct AddJoin {
  __device__ float operator()(float a, float b) const { return a + b; }
};
template <class J>
__device__ __forceinline__ float halve_rows16(const float (&v)[16], int lrow, J join) {
  const bool b4 = (lrow >> 4) & 1, b3 = (lrow >> 3) & 1, b2 = (lrow >> 2) & 1, b1 = (lrow >> 1) & 1;
  float w8[8], w4[4], w2[2];
#pragma unroll
  for (int q = 0; q < 8; ++q) w8[q] = join(b4 ? v[q + 8] : v[q], __shfl_xor(b4 ? v[q] : v[q + 8], 16, 64));
#pragma unroll
  for (int q = 0; q < 4; ++q) w4[q] = join(b3 ? w8[q + 4] : w8[q], __shfl_xor(b3 ? w8[q] : w8[q + 4], 8, 64));
#pragma unroll
  for (int q = 0; q < 2; ++q) w2[q] = join(b2 ? w4[q + 2] : w4[q], __shfl_xor(b2 ? w4[q] : w4[q + 2], 4, 64));
  const float w1 = join(b1 ? w2[1] : w2[0], __shfl_xor(b1 ? w2[0] : w2[1], 2, 64));
  return join(w1, __shfl_xor(w1, 1, 64));
}

// Center (z = 0) or radius (z = 1) of an interval operand, of its ReLU when relu (the
// arithmetic of ibp_center_radius_kernel, so either way gives the same bits).
__device__ __forceinline__ float ivl_pick(float l, float u, bool center, bool relu) {
  if (relu) {
    l = fmaxf(l, 0.f);
    u = fmaxf(u, 0.f);
  }
  return center ? (l + u) / 2.0f : (u - l) / 2.0f;
}
__device__ __forceinline__ float4 ivl_pick4(float4 l, float4 u, bool center, bool relu) {
  return make_float4(ivl_pick(l.x, u.x, center, relu), ivl_pick(l.y, u.y, center, relu),
                     ivl_pick(l.z, u.z, center, relu), ivl_pick(l.w, u.w, center, relu));
}

// DL: the direct-to-LDS main loop (plain prologue, transposed B, BK 16, aligned
// float4 operands): three LDS stages filled by global_load_lds_dwordx4, two K
// tiles in flight while the third is multiplied, one barrier per K tile.  Each
// 1 KB stage chunk holds 16 rows x 4 float4 of k, float4 kq of row r at position
// 4 r + (kq ^ swz(r)), swz(r) = (r >> 1) & 3, so that the MFMA operand reads of
// 32 rows hit distinct banks.  The reduction order is that of the register-staged
// loop (lane half h takes k = 8 h + 4 jq + e of each K tile), so both give the
// same bits.
template <int PRO, int EPI, bool TRANS_B, class T, bool DL = false>
__global__ void __launch_bounds__(T::NT, (gemm_waves_per_simd<PRO, T>()))
gemm_kernel(GemmArgs p) {
  constexpr int GBM = T::BM, GBN = T::BN, GBK = T::BK, GNT = T::NT;
  constexpr int AP = T::AP, BPT = T::BPT, A_SLOTS = T::A_SLOTS, B_SLOTS = T::B_SLOTS;
  constexpr int KQ = T::KQ, RPP = T::RPP, FM = T::FM, FN = T::FN;
  static_assert(!DL || (PRO == PRO_PLAIN && TRANS_B && GBK == 16 && GBM % 16 == 0 && GBN % 16 == 0 &&
                        T::WTM % 8 == 0 && T::WTN % 8 == 0),
                "direct-to-LDS loop: plain prologue, transposed B, BK 16");
  constexpr int NSTAGE = DL ? T::DL_STAGES : 2;
  constexpr int A_STAGE = DL ? GBM * GBK : GBM * AP;
  constexpr int B_STAGE = DL ? GBN * GBK : T::BS_FLOATS;
  // the A and B stages, one array: the relaxation epilogue stages its operands over all of it
  __shared__ __attribute__((aligned(16))) float smem_ab[NSTAGE * (A_STAGE + B_STAGE)];
  float (*As)[A_STAGE] = reinterpret_cast<float (*)[A_STAGE]>(smem_ab);
  float (*Bs)[B_STAGE] = reinterpret_cast<float (*)[B_STAGE]>(smem_ab + NSTAGE * A_STAGE);
  __shared__ float red[T::NWN][GBM];
  constexpr int TE = (PRO == PRO_RELAX) ? T::TAB_ENTRIES : 1;
  constexpr int TK = (PRO == PRO_RELAX) ? GBK : 1;
  __shared__ float4 Ts[2][TE];   // relaxation table slice of a K tile, double-buffered
  __shared__ float As_add[2][TE];  // beta split coefficient slice (lower bound)
  constexpr int TC = (PRO == PRO_RELAX && EPI == EPI_ABSSUM) ? T::TAB_ENTRIES : 1;
  __shared__ float Cs[2][TC];      // center-vector slice (concretization)
  __shared__ float Kb[2][TK];    // affine bias slice

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = t >> 6;
  const int wm = wave / T::NWN;
  const int wn = wave % T::NWN;
  // blockIdx.y = z * ksplit + (K chunk index) when split, else z
  const bool split = (PRO == PRO_PLAIN && EPI == EPI_STORE) && p.ksplit > 1;   // uniform
  const int z = split ? (int)blockIdx.y / p.ksplit : (int)blockIdx.y;
  const int kc = split ? (int)blockIdx.y - z * p.ksplit : 0;
  const bool lower = p.z_lower_first ? (z == 0) : (z == 1);
  const bool abs_b = (p.abs_b >> z) & 1;
  const float* __restrict__ A = p.A[z];
  // K range of this workgroup: [kbase, K) (the whole contraction unless split)
  const int64_t kbase = split ? (int64_t)kc * p.kchunk : 0;
  const int64_t M = p.M, N = p.N;
  const int64_t K = split ? (kbase + p.kchunk < p.K ? kbase + p.kchunk : p.K) : p.K;
  // XCD-aware tile order: workgroups are dealt round-robin to the 8 XCDs, so
  // give each XCD a contiguous run of tiles in row-major (n fastest) order.
  const int64_t ntn = ceil_div(N, GBN);
  const int64_t ntiles = ceil_div(M, GBM) * ntn;
  const int64_t per_xcd = ceil_div(ntiles, 8);
  const int64_t tile = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (tile >= ntiles) return;
  const int64_t tile_n = tile % ntn;
  const int64_t m0 = (tile / ntn) * GBM;
  const int64_t n0 = tile_n * GBN;
  const bool row_reduce = (PRO == PRO_RELAX) && (tile_n == 0);
  const bool vec_a = ((K & 3) == 0) && ((p.lda & 3) == 0) && ((p.lda_d & 3) == 0) && (((uintptr_t)A & 15) == 0) &&
                     (((uintptr_t)p.ivl_hi & 15) == 0);
  const bool ivl = PRO == PRO_PLAIN && !DL && p.ivl_hi != nullptr;   // uniform
  const bool vec_b = TRANS_B ? (((K & 3) == 0) && ((p.ldb & 3) == 0) && (((uintptr_t)p.B & 15) == 0))
                             : (((N & 3) == 0) && ((p.ldb & 3) == 0) && (((uintptr_t)p.B & 15) == 0));

  // A-tile ownership: float4 slot q = t + GNT*j -> row (t / KQ) + RPP*j, k quad (t % KQ)
  const int a_kq = t % KQ;
  const int a_r0 = t / KQ;
  int64_t a_base[A_SLOTS];
  int a_dom[A_SLOTS];   // domain of the row (D < 2^31)
  float s_beta[A_SLOTS], s_bias[A_SLOTS], s_cen[A_SLOTS];
#pragma unroll
  for (int j = 0; j < A_SLOTS; ++j) {
    const int64_t m = m0 + a_r0 + RPP * j;
    const int64_t mm = m < M ? m : 0;
    const int64_t d = mm / p.S;
    a_dom[j] = (int)d;
    a_base[j] = d * p.lda_d + (mm - d * p.S) * p.lda;
    s_beta[j] = 0.f;
    s_bias[j] = 0.f;
    s_cen[j] = 0.f;
  }

  float4 a_reg[A_SLOTS];
  float4 b_reg[B_SLOTS];

  // B-tile ownership (transposed B): float4 slot q = t + GNT*j -> column n0 + q / KQ,
  // k quad q % KQ.  On the unchecked path a column past N reads column N - 1 and a
  // row past M reads row 0: their products land in rows / columns no epilogue keeps.
  uint32_t b_off[B_SLOTS];
#pragma unroll
  for (int j = 0; j < B_SLOTS; ++j) {
    const int q = t + GNT * j;
    const int64_t gn = n0 + q / KQ;
    b_off[j] = (uint32_t)((gn < N ? gn : N - 1) * p.ldb + 4 * (q % KQ));
  }
  const bool unchecked = PRO == PRO_PLAIN && TRANS_B && vec_a && vec_b && ((K - kbase) % GBK == 0);

  // unchk: every K tile of this workgroup is whole and every operand row is
  // float4-aligned (uniform), so the loads need no bounds checks
  auto load_tiles = [&](int64_t k0, auto unchk_c) {
    if constexpr (TRANS_B && decltype(unchk_c)::value) {
#pragma unroll
      for (int j = 0; j < A_SLOTS; ++j)
        a_reg[j] = *reinterpret_cast<const float4*>(A + a_base[j] + k0 + 4 * a_kq);
      if (PRO == PRO_PLAIN && ivl) {
#pragma unroll
        for (int j = 0; j < A_SLOTS; ++j)
          a_reg[j] = ivl_pick4(a_reg[j], *reinterpret_cast<const float4*>(p.ivl_hi + a_base[j] + k0 + 4 * a_kq),
                               z == 0, p.ivl_relu != 0);
      }
#pragma unroll
      for (int j = 0; j < B_SLOTS; ++j) {
        if (!T::B_FULL && t + GNT * j >= T::B_QUADS) {
          b_reg[j] = make_float4(0.f, 0.f, 0.f, 0.f);
          continue;
        }
        float4 v = *reinterpret_cast<const float4*>(p.B + b_off[j] + (uint32_t)k0);
        if (abs_b) {
          v.x = fabsf(v.x); v.y = fabsf(v.y); v.z = fabsf(v.z); v.w = fabsf(v.w);
        }
        b_reg[j] = v;
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < A_SLOTS; ++j) {
      const int64_t m = m0 + a_r0 + RPP * j;
      const int64_t k = k0 + 4 * a_kq;
      auto load_a = [&](const float* base) {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (m < M) {
          const float* src = base + a_base[j] + k;
          if (vec_a) {
            if (k < K) v = *reinterpret_cast<const float4*>(src);
          } else {
            if (k + 0 < K) v.x = src[0];
            if (k + 1 < K) v.y = src[1];
            if (k + 2 < K) v.z = src[2];
            if (k + 3 < K) v.w = src[3];
          }
        }
        return v;
      };
      float4 v = load_a(A);
      // padding (zero bounds) gives a zero center and radius
      if (PRO == PRO_PLAIN && ivl) v = ivl_pick4(v, load_a(p.ivl_hi), z == 0, p.ivl_relu != 0);
      a_reg[j] = v;
    }
#pragma unroll
    for (int j = 0; j < B_SLOTS; ++j) {
      const int q = t + GNT * j;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (!T::B_FULL && q >= T::B_QUADS) {
        b_reg[j] = v;
        continue;
      }
      if (TRANS_B) {
        const int n = q / KQ, kq = q % KQ;
        const int64_t gn = n0 + n, gk = k0 + 4 * kq;
        if (gn < N) {
          // B offsets fit in 32 bits (checked at launch): uniform base + 32-bit offset
          const float* src = p.B + (uint32_t)(gn * p.ldb + gk);
          if (vec_b) {
            if (gk < K) v = *reinterpret_cast<const float4*>(src);
          } else {
            if (gk + 0 < K) v.x = src[0];
            if (gk + 1 < K) v.y = src[1];
            if (gk + 2 < K) v.z = src[2];
            if (gk + 3 < K) v.w = src[3];
          }
        }
      } else {
        // B given as [K, N]: thread reads 4 consecutive k of one column n (each of
        // the 4 loads is coalesced across the wave), stored as one n-major float4.
        const int n = q % GBN, kq = q / GBN;
        const int64_t gn = n0 + n, gk = k0 + 4 * kq;
        if (gn < N) {
          const uint32_t o = (uint32_t)(gk * p.ldb + gn), ld = (uint32_t)p.ldb;
          if (gk + 0 < K) v.x = p.B[o];
          if (gk + 1 < K) v.y = p.B[o + ld];
          if (gk + 2 < K) v.z = p.B[o + 2 * ld];
          if (gk + 3 < K) v.w = p.B[o + 3 * ld];
        }
      }
      if (abs_b) {
        v.x = fabsf(v.x); v.y = fabsf(v.y); v.z = fabsf(v.z); v.w = fabsf(v.w);
      }
      b_reg[j] = v;
    }
  };

  const bool use_add = (PRO == PRO_RELAX) && lower && (p.add_l != nullptr);

  // The rows of this tile span domains d_first .. d_first + ndom - 1.  When that
  // fits TAB_DOMS, the relaxation operands of a K tile are loaded once per
  // (domain, k) -- one entry per thread, coalesced -- and staged in LDS one K
  // tile ahead (slot (kt & 1)), so every coefficient reads them from LDS.
  int d_first = 0;
  int ndom = 0;
  bool tab_lds = false;
  if (PRO == PRO_RELAX && p.relax && (EPI != EPI_ABSSUM || p.cvec)) {
    const int64_t m_last = (m0 + GBM < M ? m0 + GBM : M) - 1;
    d_first = (int)(m0 / p.S);
    const int64_t nd = m_last / p.S - d_first + 1;
    tab_lds = nd <= T::TAB_DOMS;
    ndom = tab_lds ? (int)nd : 0;
  }
  const int e_dom = t / GBK, e_k = t % GBK;   // this thread's table entry
  // LDS entry of this thread's first coefficient of slot j (loop invariant);
  // rows past M read their first domain's entries, their results are discarded
  int e_base[A_SLOTS];
#pragma unroll
  for (int j = 0; j < A_SLOTS; ++j)
    e_base[j] = ((m0 + a_r0 + RPP * j < M ? a_dom[j] : d_first) - d_first) * GBK + 4 * a_kq;

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int64_t nk = ceil_div(K - kbase, GBK);
  const int lrow = lane & 31;
  const int h = lane >> 5;   // lane half -> k half of the tile

  // The main loop, instantiated per combination of the uniform relaxation
  // options so that the loop body carries no branches on them.  FAST: operands
  // from the LDS slices; ADD: beta split term; KB: affine bias; RR: row sums
  // (first column tile only); the center sums follow EPI == EPI_ABSSUM.
  // FULL: every 32-column MFMA block of this wave lies inside N; otherwise the
  // blocks past N (the last column tile of a ragged N) skip their MFMAs.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int64_t wcol0 = n0 + (int64_t)(wave_u % T::NWN) * T::WTN;
  const int fn_act = wcol0 >= N ? 0 : (int)(ceil_div(N - wcol0, 32) < FN ? ceil_div(N - wcol0, 32) : FN);
  auto main_loop = [&](auto fast_c, auto add_c, auto kb_c, auto rr_c, auto full_c, auto unchk_c) {
    constexpr bool FAST = decltype(fast_c)::value;
    constexpr bool ADD = decltype(add_c)::value;
    constexpr bool KB = decltype(kb_c)::value;
    constexpr bool RR = decltype(rr_c)::value;
    constexpr bool FULL = decltype(full_c)::value;
    constexpr bool CV = (EPI == EPI_ABSSUM);
    float4 tab_reg = make_float4(1.f, 0.f, 1.f, 0.f);
    float add_reg = 0.f, kb_reg = 0.f, cv_reg = 0.f;

    auto load_tab = [&](int64_t k0) {
      if constexpr (PRO == PRO_RELAX && FAST) {
        const int64_t k = k0 + e_k;
        const bool ok = e_dom < ndom && k < K;
        const int64_t d = (int64_t)d_first + e_dom;
        tab_reg = ok ? p.relax[d * K + k] : make_float4(1.f, 0.f, 1.f, 0.f);
        if constexpr (ADD) add_reg = ok ? p.add_l[d * p.add_ld + k] : 0.f;
        if constexpr (CV && RR) cv_reg = ok ? p.cvec[d * p.cvec_ld + k] : 0.f;
        if constexpr (KB && RR)
          if (t < GBK) kb_reg = (k0 + t < K) ? p.kbias[k0 + t] : 0.f;
      }
    };
    auto store_tab = [&](int slot) {
      if constexpr (PRO == PRO_RELAX && FAST) {
        if (t < T::TAB_ENTRIES) {
          Ts[slot][t] = tab_reg;
          if constexpr (ADD) As_add[slot][t] = add_reg;
          if constexpr (CV && RR) Cs[slot][t] = cv_reg;
        }
        if constexpr (KB && RR)
          if (t < GBK) Kb[slot][t] = kb_reg;
      }
    };

    // ReLU relaxation of one coefficient (crown_ibp.py:1261-1296), applied as
    // the A tile is written to LDS.  Fast path: padding coefficients (k >= K)
    // are zero and meet identity / zero entries, so they contribute nothing.
    auto relax_one = [&](float a, int j, int e, int64_t k, int slot) -> float {
      float4 r;
      float add = 0.f, kb = 0.f, cv = 0.f;
      if constexpr (FAST) {
        r = Ts[slot][e_base[j] + e];
        if constexpr (ADD) add = As_add[slot][e_base[j] + e];
        if constexpr (KB && RR) kb = Kb[slot][4 * a_kq + e];
        if constexpr (CV && RR) cv = Cs[slot][e_base[j] + e];
      } else {
        if (k >= K) return a;
        const int64_t d = a_dom[j];
        r = p.relax ? p.relax[d * K + k] : make_float4(1.f, 0.f, 1.f, 0.f);
        if (use_add) add = p.add_l[d * p.add_ld + k];
        if (p.kbias) kb = p.kbias[k];
        if (p.cvec) cv = p.cvec[d * p.cvec_ld + k];
      }
      float be;
      float out = a * fsel(r, lower, a >= 0.f, &be);
      if constexpr (FAST) {
        if constexpr (ADD) out = out + add;
        if constexpr (RR) {
          s_beta[j] += a * be;
          if constexpr (KB) s_bias[j] += out * kb;
          if constexpr (CV) s_cen[j] += out * cv;
        }
      } else {
        if (use_add) out = out + add;
        if (row_reduce) {
          s_beta[j] += a * be;
          if (p.kbias) s_bias[j] += out * kb;
          if (p.cvec) s_cen[j] += out * cv;
        }
      }
      return out;
    };

    // kt: index of the K tile being stored (its relaxation slice is in slot kt & 1)
    auto store_tiles = [&](int buf, int64_t k0, int64_t kt) {
      const int slot = (int)(kt & 1);
#pragma unroll
      for (int j = 0; j < A_SLOTS; ++j) {
        const int r = a_r0 + RPP * j;
        float4 v = a_reg[j];
        if constexpr (PRO == PRO_RELAX) {
          if (FAST || m0 + r < M) {
            const int64_t k = k0 + 4 * a_kq;
            v.x = relax_one(v.x, j, 0, k + 0, slot);
            v.y = relax_one(v.y, j, 1, k + 1, slot);
            v.z = relax_one(v.z, j, 2, k + 2, slot);
            v.w = relax_one(v.w, j, 3, k + 3, slot);
          }
        }
        *reinterpret_cast<float4*>(&As[buf][r * AP + 4 * a_kq]) = v;
      }
#pragma unroll
      for (int j = 0; j < B_SLOTS; ++j) {
        const int q = t + GNT * j;
        if (!T::B_FULL && q >= T::B_QUADS) continue;
        const int n = TRANS_B ? q / KQ : q % GBN;
        const int kq = TRANS_B ? q % KQ : q / GBN;
        *reinterpret_cast<float4*>(&Bs[buf][n * BPT + 4 * kq]) = b_reg[j];
      }
    };

    // The 32 MFMAs of one K tile of this wave, operands from LDS buffer buf.
    auto mfma_tile = [&](int buf) {
      const float* __restrict__ as = As[buf];
      const float* __restrict__ bs = Bs[buf];
      // waves with MFMAs to issue go first: the loads and LDS stores of the others fit around them
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int jb = 0; jb < GBK / 2; jb += 4) {
        float av[FM][4];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const float4 a4 = *reinterpret_cast<const float4*>(
              &as[(wm * T::WTM + i * 32 + lrow) * AP + h * (GBK / 2) + jb]);
          av[i][0] = a4.x; av[i][1] = a4.y; av[i][2] = a4.z; av[i][3] = a4.w;
        }
        float bv[FN][4];
#pragma unroll
        for (int jj = 0; jj < FN; ++jj) {
          const float4 b4 = *reinterpret_cast<const float4*>(
              &bs[(wn * T::WTN + jj * 32 + lrow) * BPT + h * (GBK / 2) + jb]);
          bv[jj][0] = b4.x; bv[jj][1] = b4.y; bv[jj][2] = b4.z; bv[jj][3] = b4.w;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int jj = 0; jj < FN; ++jj)
              if (FULL || jj < fn_act)
                acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[jj][e], acc[i][jj], 0, 0, 0);
      }
      __builtin_amdgcn_s_setprio(0);
    };

    // Prologue: relaxation slices of K tiles 0 and 1, then tile 0 itself.
    load_tab(0);
    store_tab(0);
    if (nk > 1) {
      load_tab(GBK);
      store_tab(1);
    }
    load_tiles(kbase, unchk_c);
    __syncthreads();
    store_tiles(0, kbase, 0);
    __syncthreads();
    int buf = 0;
    for (int64_t kt = 0; kt < nk; ++kt) {
      const bool more = kt + 1 < nk;
      const bool more2 = kt + 2 < nk;
      if (more) load_tiles(kbase + (kt + 1) * GBK, unchk_c);
      if (more2) load_tab((kt + 2) * GBK);
      mfma_tile(buf);
      if (more) store_tiles(buf ^ 1, kbase + (kt + 1) * GBK, kt + 1);
      // slot kt & 1 held tile kt's slice, consumed one iteration ago
      if (more2) store_tab((int)(kt & 1));
      __syncthreads();
      buf ^= 1;
    }
  };

  using TT = std::true_type;
  using FF = std::false_type;
  const bool full = fn_act == FN;   // wave-uniform
  auto run = [&](auto fast_c, auto add_c, auto kb_c, auto rr_c) {
    if constexpr (PRO != PRO_PLAIN || !TRANS_B) {
      if (full) main_loop(fast_c, add_c, kb_c, rr_c, TT{}, FF{});
      else main_loop(fast_c, add_c, kb_c, rr_c, FF{}, FF{});
    } else if (unchecked) {
      if (full) main_loop(fast_c, add_c, kb_c, rr_c, TT{}, TT{});
      else main_loop(fast_c, add_c, kb_c, rr_c, FF{}, TT{});
    } else {
      if (full) main_loop(fast_c, add_c, kb_c, rr_c, TT{}, FF{});
      else main_loop(fast_c, add_c, kb_c, rr_c, FF{}, FF{});
    }
  };
  if constexpr (DL) {
    // ---- direct-to-LDS main loop ----
    constexpr int A_CHUNKS = GBM / 16, B_CHUNKS = GBN / 16, NW = GNT / 64;
    constexpr int A_PW = (A_CHUNKS + NW - 1) / NW, B_PW = (B_CHUNKS + NW - 1) / NW;
    const int wave_s = __builtin_amdgcn_readfirstlane(wave);
    // this lane's copy slots: chunk c = wave + NW j, row 16 c + lane / 4, stored float4
    // lane % 4 holding k quad (lane % 4) ^ swz(row); rows past M / N read row M-1 / N-1
    const int sl_q = lane & 3;
    int64_t a_row[A_PW];
    int a_kq[A_PW];
#pragma unroll
    for (int j = 0; j < A_PW; ++j) {
      const int r = 16 * (wave_s + NW * j) + (lane >> 2);
      const int64_t m = m0 + r < M ? m0 + r : M - 1;
      const int64_t d = m / p.S;
      a_row[j] = d * p.lda_d + (m - d * p.S) * p.lda;
      a_kq[j] = sl_q ^ ((r >> 1) & 3);
    }
    uint32_t b_row[B_PW];
    int b_kq[B_PW];
#pragma unroll
    for (int j = 0; j < B_PW; ++j) {
      const int r = 16 * (wave_s + NW * j) + (lane >> 2);
      const int64_t n = n0 + r < N ? n0 + r : N - 1;
      b_row[j] = (uint32_t)(n * p.ldb);
      b_kq[j] = sl_q ^ ((r >> 1) & 3);
    }
    constexpr int PER_STAGE_A = A_CHUNKS % NW == 0 ? A_PW : -1;
    constexpr int PER_STAGE_B = B_CHUNKS % NW == 0 ? B_PW : -1;
    static_assert(PER_STAGE_A > 0 && PER_STAGE_B > 0, "every wave issues the same copies per stage");
    constexpr int COPIES = PER_STAGE_A + PER_STAGE_B;   // vmem operations per stage and wave
    // copy K tile [k0, k0 + 16) into a stage; quads at or past K read the row start
    // and are zeroed by fix_tail once they have landed
    auto issue = [&](int st, int64_t k0) {
#pragma unroll
      for (int j = 0; j < A_PW; ++j) {
        const int64_t k = k0 + 4 * a_kq[j];
        const float* src = A + a_row[j] + (k < K ? k : 0);
        lds_copy16(src, &As[st][(wave_s + NW * j) * 256]);
      }
#pragma unroll
      for (int j = 0; j < B_PW; ++j) {
        const int64_t k = k0 + 4 * b_kq[j];
        const float* src = p.B + b_row[j] + (uint32_t)(k < K ? k : 0);
        lds_copy16(src, &Bs[st][(wave_s + NW * j) * 256]);
      }
    };
    auto fix_tail = [&](int st, int64_t k0) {
#pragma unroll
      for (int j = 0; j < A_PW; ++j)
        if (k0 + 4 * a_kq[j] >= K)
          *reinterpret_cast<float4*>(&As[st][(wave_s + NW * j) * 256 + 4 * lane]) = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int j = 0; j < B_PW; ++j)
        if (k0 + 4 * b_kq[j] >= K)
          *reinterpret_cast<float4*>(&Bs[st][(wave_s + NW * j) * 256 + 4 * lane]) = make_float4(0.f, 0.f, 0.f, 0.f);
    };
    // operand positions (floats) of this lane: row wm WTM + 32 i + lrow (n: wn WTN + 32 jj + lrow),
    // k quad 2 h + jq; swz of the row is (lrow >> 1) & 3 since the block offsets are multiples of 8
    const int swz = (lrow >> 1) & 3;
    int a_pos[FM][2], b_pos[FN][2];
#pragma unroll
    for (int jq = 0; jq < 2; ++jq) {
#pragma unroll
      for (int i = 0; i < FM; ++i) a_pos[i][jq] = 4 * (4 * (wm * T::WTM + 32 * i + lrow) + ((2 * h + jq) ^ swz));
#pragma unroll
      for (int jj = 0; jj < FN; ++jj) b_pos[jj][jq] = 4 * (4 * (wn * T::WTN + 32 * jj + lrow) + ((2 * h + jq) ^ swz));
    }
    auto dl_loop = [&](auto full_c) {
      constexpr bool FULL = decltype(full_c)::value;
      const bool tail = (K - kbase) % GBK != 0;
      const int nki = (int)nk;   // K tiles of this workgroup (K < 2^31)
      constexpr int AHEAD = NSTAGE - 1;   // K tiles in flight beyond the one being multiplied
      issue(0, kbase);
      if (AHEAD > 1 && nki > 1) issue(1, kbase + GBK);
      int st = 0, st2 = AHEAD;   // stage of tile kt, stage refilled with tile kt + AHEAD
      for (int kt = 0; kt < nki; ++kt) {
        if (AHEAD > 1 && kt + 1 < nki) wait_vmem<(AHEAD - 1) * COPIES>(); else wait_vmem<0>();
        if (tail && kt + 1 == nki) fix_tail(st, kbase + (int64_t)kt * GBK);
        lds_barrier();   // tile kt visible; every wave is done with the stage refilled next
        if (kt + AHEAD < nki) issue(st2, kbase + (int64_t)(kt + AHEAD) * GBK);
        const float* __restrict__ as = As[st];
        const float* __restrict__ bs = Bs[st];
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int jq = 0; jq < 2; ++jq) {
          float av[FM][4];
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            const float4 a4 = *reinterpret_cast<const float4*>(&as[a_pos[i][jq]]);
            av[i][0] = a4.x; av[i][1] = a4.y; av[i][2] = a4.z; av[i][3] = a4.w;
          }
          float bv[FN][4];
#pragma unroll
          for (int jj = 0; jj < FN; ++jj) {
            float4 b4 = *reinterpret_cast<const float4*>(&bs[b_pos[jj][jq]]);
            if (abs_b) {
              b4.x = fabsf(b4.x); b4.y = fabsf(b4.y); b4.z = fabsf(b4.z); b4.w = fabsf(b4.w);
            }
            bv[jj][0] = b4.x; bv[jj][1] = b4.y; bv[jj][2] = b4.z; bv[jj][3] = b4.w;
          }
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
              for (int jj = 0; jj < FN; ++jj)
                if (FULL || jj < fn_act)
                  acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[jj][e], acc[i][jj], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
        st = st == NSTAGE - 1 ? 0 : st + 1;
        st2 = st2 == NSTAGE - 1 ? 0 : st2 + 1;
      }
      lds_barrier();   // every wave is done with the stages before an epilogue reuses them
    };
    if (full) dl_loop(TT{});
    else dl_loop(FF{});
  } else if constexpr (PRO == PRO_PLAIN) {
    run(FF{}, FF{}, FF{}, FF{});
  } else {
    const bool kb = p.kbias != nullptr;
    if (!tab_lds) run(FF{}, FF{}, FF{}, FF{});
    else if (row_reduce) {
      if (use_add) { if (kb) run(TT{}, TT{}, TT{}, TT{}); else run(TT{}, TT{}, FF{}, TT{}); }
      else { if (kb) run(TT{}, FF{}, TT{}, TT{}); else run(TT{}, FF{}, FF{}, TT{}); }
    } else {
      if (use_add) run(TT{}, TT{}, FF{}, FF{});
      else run(TT{}, FF{}, FF{}, FF{});
    }
  }

  // Row reductions of the relaxation prologue: the KQ threads holding one row
  // are KQ consecutive lanes; reduce with xor shuffles in a fixed order.
  if (row_reduce) {
#pragma unroll
    for (int j = 0; j < A_SLOTS; ++j) {
      float sb = s_beta[j], sk = s_bias[j], sc = s_cen[j];
#pragma unroll
      for (int off = KQ / 2; off >= 1; off >>= 1) {
        sb += __shfl_xor(sb, off, 64);
        sk += __shfl_xor(sk, off, 64);
        sc += __shfl_xor(sc, off, 64);
      }
      const int64_t m = m0 + a_r0 + RPP * j;
      if (a_kq == 0 && m < M) {
        const float b0 = p.b_in[z] ? p.b_in[z][m] : 0.f;
        if (p.b_out[z]) p.b_out[z][m] = (b0 + sb) + sk;
        if (p.c_out[z]) p.c_out[z][m] = sc;
      }
    }
  }

  if constexpr (EPI == EPI_STORE) {
    float* __restrict__ C = split ? p.part + (int64_t)blockIdx.y * M * N : p.C[z];   // partial (z, kc)
    const int64_t ldc = split ? N : p.ldc;
    const bool r1 = !split && p.r1_row;
    const bool fits32 = M < (1LL << 31);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row >= M) continue;
        // the row's rank-1 factor and vector, once per row (no division when the vector is shared)
        float rf = 0.f;
        const float* __restrict__ vrow = p.r1_col;
        if (r1) {
          rf = p.r1_row[row];
          if (p.r1_ld) vrow += div_rows(row, p.S, fits32) * p.r1_ld;
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t col = n0 + wn * T::WTN + j * 32 + lrow;
          if (col < N) {
            float v = acc[i][j][r];
            if (r1) v = v + rf * vrow[col];
            C[row * ldc + col] = v;
          }
        }
      }
  } else if constexpr (EPI == EPI_ABSSUM) {
    static_assert(GBN == NORM_BN || GBN == NORM_BN / 2, "the |C| epilogue takes 128- or 64-column tiles");
    // sum_n |C[m, n]| * w[d, n] over this block's columns, fixed order (norm kind 0);
    // max_n |C[m, n]| (1) or sum_n C[m, n]^2 (2) for the L1 and L2 balls.  The kind
    // is uniform over the launch: one specialisation of the epilogue per kind.
    const bool fits32 = M < (1LL << 31);
    auto norm_epilogue = [&](auto kind) {
      constexpr int NK = decltype(kind)::value;
      auto join = [](float a, float b) { return NK == 1 ? fmaxf(a, b) : a + b; };
      float rs[FM][16];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = m0 + wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          const int64_t d = (p.wvec && row < M) ? div_rows(row, p.S, fits32) : 0;
          float s = 0.f;
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            const int64_t col = n0 + wn * T::WTN + j * 32 + lrow;
            const float a = acc[i][j][r];
            float v = col < N ? (NK == 2 ? a * a : fabsf(a)) : 0.f;   // columns past N hold products no one keeps
            float wgt = 1.f;
            if (NK == 0 && p.wvec) {
              wgt = (row < M && col < N) ? p.wvec[d * p.w_ld + col] : 0.f;
              v = v * wgt;
            }
            s = join(s, v);
            if (lower && p.h_out && row < M && col < N) {
              if (NK != 0) {
                p.h_out[row * N + col] = a;   // the L1/L2 seeds need the whole row's norm: made from C afterwards
              } else {
                const float sg = (a > 0.f) ? 1.f : ((a < 0.f) ? -1.f : 0.f);
                const float hs = p.h_scale[row];
                p.h_out[row * N + col] = p.wvec ? hs * sg * wgt : hs * sg;
              }
            }
          }
          rs[i][r] = s;
        }
      float rsum[FM];
#pragma unroll
      for (int i = 0; i < FM; ++i) rsum[i] = halve_rows16(rs[i], lrow, join);
      if ((lrow & 1) == 0) {
        const int r = lrow >> 1;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int rloc = wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          red[wn][rloc] = rsum[i];
        }
      }
      __syncthreads();
      for (int rr = t; rr < GBM; rr += GNT) {
        const int64_t row = m0 + rr;
        if (row < M) {
          float s = 0.f;
#pragma unroll
          for (int q = 0; q < T::NWN; ++q) s = join(s, red[q][rr]);
          p.partial[z][tile_n * M + row] = s;
        }
      }
    };
    if (p.norm_kind == 0) norm_epilogue(std::integral_constant<int, 0>{});
    else if (p.norm_kind == 1) norm_epilogue(std::integral_constant<int, 1>{});
    else norm_epilogue(std::integral_constant<int, 2>{});
  } else {
    // Relaxation of the next ReLU (crown_ibp.py:1261-1296) applied to C before
    // it is stored, so the next contraction reads A' directly; every coefficient
    // is relaxed once here instead of once per column tile of its consumer.
    static_assert(GBN == NORM_BN, "the relaxation epilogue needs BN == NORM_BN");
    // As / Bs are free once every wave has left the main loop: As holds the
    // relaxation entries of the tile's domains x columns, Bs the split term,
    // the center vector, the bias and the domain of each row.
    // per (domain, column) entry: the float4 relaxation, the split term and the center
    constexpr int E_DOMS = (NSTAGE * (A_STAGE + B_STAGE)) / (6 * GBN);
    __shared__ float Ke[GBN];
    __shared__ int Re[GBM];
    __syncthreads();
    float4* Te = reinterpret_cast<float4*>(smem_ab);
    float* Ae = smem_ab + 4 * E_DOMS * GBN;
    float* Ce = Ae + E_DOMS * GBN;
    const int64_t m_last = (m0 + GBM < M ? m0 + GBM : M) - 1;
    const int e_first = (int)(m0 / p.S);
    const int endom = (int)(m_last / p.S) - e_first + 1;
    const bool staged = endom <= E_DOMS;   // uniform; otherwise entries are read from global memory
    const bool add_e = lower && (p.e_add != nullptr);
    const bool kb_e = p.e_kbias != nullptr;
    const bool cv_e = p.e_cvec != nullptr;
    if (staged) {
      for (int q = t; q < endom * GBN; q += GNT) {
        const int dd = q / GBN, c = q % GBN;
        const int64_t n = n0 + c, d = (int64_t)e_first + dd;
        const bool ok = n < N;
        Te[q] = ok ? p.e_relax[d * N + n] : make_float4(1.f, 0.f, 1.f, 0.f);
        if (add_e) Ae[q] = ok ? p.e_add[d * p.e_add_ld + n] : 0.f;
        if (cv_e) Ce[q] = ok ? p.e_cvec[d * p.e_cvec_ld + n] : 0.f;
      }
      for (int c = t; c < GBN; c += GNT) Ke[c] = (kb_e && n0 + c < N) ? p.e_kbias[n0 + c] : 0.f;
      for (int rl = t; rl < GBM; rl += GNT) {
        const int64_t m = m0 + rl;
        Re[rl] = (m < M ? (int)(m / p.S) : e_first) - e_first;
      }
    }
    __syncthreads();
    float* __restrict__ C = p.C[z];
    float* __restrict__ Cpre = p.C_pre[z];
    float pb[FM][16], pc[FM][16];
    const bool fits32 = M < (1LL << 31);
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rloc = wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        const int64_t row = m0 + rloc;
        float sb = 0.f, sc = 0.f;
        // the row's domain, once per row: its LDS entry block, or its rows of the global operands
        int eq = 0;
        const float4* __restrict__ erow = p.e_relax;
        const float* __restrict__ arow = p.e_add;
        const float* __restrict__ crow = p.e_cvec;
        if (staged) {
          eq = Re[rloc] * GBN;
        } else if (row < M) {
          const int64_t d = div_rows(row, p.S, fits32);
          erow += d * N;
          if (add_e) arow += d * p.e_add_ld;
          if (cv_e) crow += d * p.e_cvec_ld;
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int cloc = wn * T::WTN + j * 32 + lrow;
          const int64_t col = n0 + cloc;
          if (row < M && col < N) {
            const float a = acc[i][j][r];
            float4 e;
            float add = 0.f, cv = 0.f, kb = 0.f;
            if (staged) {
              const int q = eq + cloc;
              e = Te[q];
              if (add_e) add = Ae[q];
              if (cv_e) cv = Ce[q];
              kb = Ke[cloc];
            } else {
              e = erow[col];
              if (add_e) add = arow[col];
              if (cv_e) cv = crow[col];
              if (kb_e) kb = p.e_kbias[col];
            }
            if (Cpre) Cpre[row * p.ldc + col] = a;
            float be;
            float out = a * fsel(e, lower, a >= 0.f, &be);
            if (add_e) out = out + add;
            sb += a * be;
            if (kb_e) sb += out * kb;
            if (cv_e) sc += out * cv;
            C[row * p.ldc + col] = out;
          }
        }
        pb[i][r] = sb;
        pc[i][r] = sc;
      }
    // fixed-order reduction over the tile's columns: 32 lanes (halve_rows16), then the NWN waves
    const AddJoin add_f;
    float rb[FM], rc[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      rb[i] = halve_rows16(pb[i], lrow, add_f);
      rc[i] = cv_e ? halve_rows16(pc[i], lrow, add_f) : 0.f;
    }
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      if (pass == 1 && !cv_e) break;   // uniform
      if ((lrow & 1) == 0) {
        const int r = lrow >> 1;
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const int rloc = wm * T::WTM + i * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          red[wn][rloc] = pass == 0 ? rb[i] : rc[i];
        }
      }
      __syncthreads();
      float* __restrict__ dst = pass == 0 ? p.partial[z] : p.partial_c[z];
      for (int rr = t; rr < GBM; rr += GNT) {
        const int64_t row = m0 + rr;
        if (row < M) {
          float v = 0.f;
#pragma unroll
          for (int q = 0; q < T::NWN; ++q) v += red[q][rr];
          dst[tile_n * M + row] = v;
        }
      }
      __syncthreads();
    }
  }
}

// Tile configurations (selected per call by gemm_dispatch).
using TileG = Tile<128, 128, 16, 4, 2, 3>;   // 8 waves of 32x64, 3 workgroups per CU
using TileH = Tile<128, 128, 32, 4, 4, 2>;   // 16 waves of 32x32, BK 32, 2 workgroups per CU (64 VGPRs)
using TileQ = Tile<64, 128, 16, 2, 2, 6, true>;   // 4 waves of 32x64, 6 workgroups per CU (two LDS stages)
using TileS = Tile<64, 64, 32, 2, 2, 4>;          // 4 waves of 32x32, 4 workgroups per CU, store epilogues only

// Operands the direct-to-LDS loop takes: transposed B and whole aligned float4 rows.
inline bool gemm_dl_operands(const GemmArgs& a, int nz) {
  bool dl = a.trans_b && (a.K & 3) == 0 && (a.lda & 3) == 0 && (a.lda_d & 3) == 0 && (a.ldb & 3) == 0 &&
            ((uintptr_t)a.B & 15) == 0 && a.ivl_hi == nullptr;
  for (int z = 0; z < nz; ++z) dl = dl && ((uintptr_t)a.A[z] & 15) == 0;
  return dl;
}

template <int PRO, int EPI, class T>
static int launch_gemm_staged(const GemmArgs& a, dim3 grid, hipStream_t stream);

template <int PRO, int EPI, class T>
static int launch_gemm_t(const GemmArgs& a, int nz, hipStream_t stream) {
  const int64_t b_extent = a.trans_b ? (a.N - 1) * a.ldb + a.K : (a.K - 1) * a.ldb + a.N;
  BF_REQUIRE(b_extent < (1LL << 31), "gemm: B operand too large for 32-bit offsets (%lld elements)",
             (long long)b_extent);
  const int64_t ntiles = ceil_div(a.M, T::BM) * ceil_div(a.N, T::BN);
  BF_REQUIRE(ntiles + 8 < (1LL << 31), "gemm grid too large (M=%lld N=%lld)", (long long)a.M, (long long)a.N);
  const unsigned gy = (PRO == PRO_PLAIN && EPI == EPI_STORE && a.ksplit > 1) ? (unsigned)(a.ksplit * nz) : (unsigned)nz;
  dim3 grid((unsigned)(ceil_div(ntiles, 8) * 8), gy);
  if constexpr (PRO == PRO_PLAIN && T::BK == 16) {
    if (gemm_dl_operands(a, nz)) {
      hipLaunchKernelGGL((gemm_kernel<PRO, EPI, true, T, true>), grid, dim3(T::NT), 0, stream, a);
      BF_LAUNCH_CHECK("gemm_kernel");
      return BF_OK;
    }
  }
  if constexpr (T::DL_ONLY) {
    set_error("gemm: this tile configuration takes only the direct-to-LDS operands (plain prologue, "
              "transposed B, 16-byte aligned float4 rows)");
    return BF_EINVAL;
  } else {
    return launch_gemm_staged<PRO, EPI, T>(a, grid, stream);
  }
}

template <int PRO, int EPI, class T>
static int launch_gemm_staged(const GemmArgs& a, dim3 grid, hipStream_t stream) {
  if (a.trans_b) {
    hipLaunchKernelGGL((gemm_kernel<PRO, EPI, true, T>), grid, dim3(T::NT), 0, stream, a);
  } else {
    if constexpr (EPI == EPI_RELAX) {
      set_error("gemm: the relaxation epilogue takes the transposed weight");
      return BF_EINVAL;
    } else {
      hipLaunchKernelGGL((gemm_kernel<PRO, EPI, false, T>), grid, dim3(T::NT), 0, stream, a);
    }
  }
  BF_LAUNCH_CHECK("gemm_kernel");
  return BF_OK;
}

// Launcher of one tile configuration for a (prologue, epilogue) pair, defined
// in that configuration's translation unit.  EPI_ABSSUM needs BN == NORM_BN.
template <class T>
int launch_tile(const GemmArgs& a, int pro, int epi, int nz, hipStream_t stream);

#define BF_DEFINE_LAUNCH_TILE(T)                                                             \
  template <>                                                                                \
  int launch_tile<T>(const GemmArgs& a, int pro, int epi, int nz, hipStream_t stream) {      \
    if (pro == PRO_PLAIN && epi == EPI_STORE) return launch_gemm_t<PRO_PLAIN, EPI_STORE, T>(a, nz, stream);   \
    if (pro == PRO_RELAX && epi == EPI_STORE) return launch_gemm_t<PRO_RELAX, EPI_STORE, T>(a, nz, stream);   \
    if constexpr (T::BN == NORM_BN && T::BM <= 128) {                                        \
      if (pro == PRO_PLAIN && epi == EPI_ABSSUM) return launch_gemm_t<PRO_PLAIN, EPI_ABSSUM, T>(a, nz, stream); \
      if (pro == PRO_RELAX && epi == EPI_ABSSUM) return launch_gemm_t<PRO_RELAX, EPI_ABSSUM, T>(a, nz, stream); \
    }                                                                                        \
    if constexpr (T::BN == NORM_BN / 2 && T::BM <= 128) {                                    \
      if (pro == PRO_PLAIN && epi == EPI_ABSSUM) return launch_gemm_t<PRO_PLAIN, EPI_ABSSUM, T>(a, nz, stream); \
    }                                                                                        \
    if constexpr (T::BN == NORM_BN && T::BM <= 128) {                                        \
      if (pro == PRO_PLAIN && epi == EPI_RELAX) return launch_gemm_t<PRO_PLAIN, EPI_RELAX, T>(a, nz, stream);   \
      if (pro == PRO_RELAX && epi == EPI_RELAX) return launch_gemm_t<PRO_RELAX, EPI_RELAX, T>(a, nz, stream);   \
    }                                                                                        \
    set_error("gemm: tile configuration does not support pro=%d epi=%d", pro, epi);          \
    return BF_EINVAL;                                                                        \
  }

template <> int launch_tile<TileG>(const GemmArgs&, int, int, int, hipStream_t);
template <> int launch_tile<TileH>(const GemmArgs&, int, int, int, hipStream_t);
template <> int launch_tile<TileQ>(const GemmArgs&, int, int, int, hipStream_t);
template <> int launch_tile<TileS>(const GemmArgs&, int, int, int, hipStream_t);

}  // namespace bf
