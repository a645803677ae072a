// sta_score6.hip -- pass 2 of the shared score passes (threshold + byte votes) with one bf16
// product plus an fp6 correction per score.
//
// Reference: shared_selection_triton_exact_2.py:105-140 (pass 2 of _select_vote_kernel).  The
// keep test is the reference's, s >= m - tau on the scaled score (exact_2.py:121), compared on
// the raw dot against x0 = the smallest float with fl(x0 * sm_scale) >= m - tau; the votes are
// the kept rows of each (tile, key) (exact_2.py:123).  The row maxima m come from the screened
// pass 1 (score_kernel MODE 1, exact fp32 dots).  Each score is
//   hi(q).hi(k)                                  v_mfma_f32_32x32x16_bf16, D/16 products
// + Q6(q_hi).Q6(k - k_hi) + Q6(q - q_hi).Q6(k_hi)  v_mfma_scale_f32_32x32x64_f8f6f4 (e2m3), D/32
// in one fp32 accumulator, the small terms first (sta_fp6.h: the error is ~1e-4 on unit-scale
// scores; heads whose error estimate exceeds a quarter of the 1e-3 band are left to the
// three-product kernel, as are the workgroups whose screen fell back to the exact sweep).
//
// Work split as in the plain pass 2 of score_kernel: one workgroup = one head and 512 query rows
// in eight waves of 64 rows (two per SIMD), the head's workgroups on one XCD, heaviest first.
// 64-key chunks of K -- the bf16 hi fragments, the fp6 planes and the scales -- are copied from
// global memory straight into LDS, four buffers deep, and read by all eight waves.  Within a
// wave, each K operand read from LDS feeds the products of both 32-row blocks, and the vote
// epilogue of 32-key block n runs between the products of block n + 1.
#include "sta_device.h"
#include "sta_fp6.h"
#include "sta_kernels.h"

#include <float.h>

#include <type_traits>

namespace sta {

namespace {

typedef int v8i32 __attribute__((ext_vector_type(8)));

// one lane's fp6 operand of a 32x32x64 product: 32 e2m3 elements in three 8-byte planes
struct F6 {
  uint64_t p[3];
};

__device__ __forceinline__ v8i32 f6_operand(const F6& x) {
  return v8i32{(int)(uint32_t)x.p[0], (int)(uint32_t)(x.p[0] >> 32), (int)(uint32_t)x.p[1],
               (int)(uint32_t)(x.p[1] >> 32), (int)(uint32_t)x.p[2], (int)(uint32_t)(x.p[2] >> 32), 0, 0};
}

// e2m3 x e2m3, scale bytes SA of sa (A rows) and SB of sb (B columns)
template <int SA, int SB>
__device__ __forceinline__ floatx16 mfma6(const F6& a, uint32_t sa, const F6& b, uint32_t sb, floatx16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f6_operand(a), f6_operand(b), c, 2, 2, SA, (int)sa, SB,
                                                         (int)sb);
}

// f(integral_constant<I>) for I = B .. E - 1
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

}  // namespace

template <int D, int T>
__global__ __launch_bounds__(512, 1) void score6_kernel(ScoreArgs a) {
#pragma clang fp contract(off)
  constexpr int NW = 8, RB = 2, S = D / 16, NU = D / 32, CK = 64, SBC = CK / 32, NBUF = 4;
  constexpr int WG_ROWS = NW * 32 * RB;          // 512 query rows
  constexpr int NTW = 32 * RB / T;               // tiles per wave
  constexpr int HI_U = SBC * S * 64;             // u32x4 units of a chunk's bf16 hi fragments
  constexpr int F6_U = SBC * NU * 3 * 64 / 2;    // ... of its fp6 planes
  constexpr int SC_U = SBC * 64 / 4;             // ... of its scale dwords (half a wave's copy)
  constexpr int BUF_U = HI_U + F6_U + SC_U;
  constexpr int NHI = HI_U / 64, NF6 = F6_U / 64;
  constexpr int NCP = NHI + NF6 + 1;             // 1 KB copies per chunk (the last one 512 bytes)
  constexpr int CMAX = (NCP + NW - 1) / NW;      // copies per wave and chunk: CMAX or CMAX - 1
  constexpr int NSTEP = NU + S;                  // operand steps of a 32-key block
  static_assert(SC_U == 32, "the scales are one half-wave copy");
  static_assert(2 * CMAX < 16, "vmcnt range");
  __shared__ u32x4 lds[NBUF][BUF_U];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rows_total = a.nt * T;
  const int ngroups = (rows_total + WG_ROWS - 1) / WG_ROWS;
  int h, g;
  {
    const int bid = blockIdx.x;
    if ((a.H & 7) == 0) {  // XCD-aware: workgroup i runs on XCD i % 8; keep a head on one XCD
      const int hpx = a.H >> 3;
      const int r = bid >> 3;
      h = (bid & 7) * hpx + r % hpx;
      g = ngroups - 1 - r / hpx;
    } else {
      h = bid % a.H;
      g = ngroups - 1 - bid / a.H;
    }
  }
  if (!fast6_serves(a, h, g, D, WG_ROWS)) return;   // the three-product kernel takes it
  const int kvh = h / (a.H / a.Hkv);
  const int wrow0 = g * WG_ROWS + wave * 32 * RB;
  const bool active = wrow0 < rows_total;
  const int hi_max = a.q_pos_base + min(g * WG_ROWS + WG_ROWS, rows_total);
  const int qpos0 = a.q_pos_base + wrow0;
  const int hi_w = qpos0 + 32 * RB;
  const int nchunks = (hi_max + CK - 1) / CK;
  const int nfull = min(min(nchunks, (a.q_pos_base + g * WG_ROWS + 1) / CK), a.N / CK);
  const float tau = a.tau[h];
  uint8_t* vrow = a.votes + ((int64_t)h * a.nt + wrow0 / T) * a.votes_stride;
  auto tile_ok = [&](int j) { return wrow0 + j * T < rows_total; };

  // ---- Q operands: bf16 hi fragments (AGPRs), fp6 units and their scale dwords ----
  const int64_t qrb0 = (int64_t)h * (a.q_rows_pad >> 5) + wrow0 / 32;
  u32x4 qhi[RB][S];
  F6 q6[RB][NU];
  uint32_t qsc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const bool ok = wrow0 + 32 * rb < rows_total;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      qhi[rb][s] = ok ? a.qfrag[((qrb0 + rb) * S + s) * 128 + lane] : u32x4{0, 0, 0, 0};
      asm volatile("" : "+a"(qhi[rb][s]));
    }
#pragma unroll
    for (int m = 0; m < NU; ++m)
#pragma unroll
      for (int j = 0; j < 3; ++j) q6[rb][m].p[j] = ok ? a.q6[((qrb0 + rb) * NU + m) * 192 + j * 64 + lane] : 0ull;
    qsc[rb] = ok ? a.q6sc[(qrb0 + rb) * 64 + lane] : 0x7f7f7f7fu;
  }

  // ---- keep thresholds x0 on the raw dot from the screen's exact row maxima.  For tau >= 0 the
  // threshold is capped at max - delta (delta bounds the fp6 score's distance from the screen's
  // exact dot, sta_fp6.h: fast6_delta), so a row's best key keeps its vote, as in the reference
  // whose two passes share one dot.  Row block 0's accumulators start from -x0 (held in the
  // AGPRs beside the Q operands), so its products accumulate s - x0 and the keep test is the
  // accumulator's sign (that rounding, ~1e-6 of the score, is far inside the correction's error);
  // row block 1 keeps x0 in VGPRs and subtracts it (the register file holds one set of each).
  floatx16 nx0[RB];
  {
    const float2 knm = a.knorm_max[kvh], kd = a.k6dmax[kvh];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = wrow0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        const bool ok = active && row < a.N;   // padded rows never vote (exact_2.py:121)
        const int64_t ri = (int64_t)h * a.q_rows_pad + (row < rows_total ? row : 0);
        const float v = a.srmax[ri];
        const float m = v * a.sm_scale;          // fl(max * c) == max of fl(s * c) for c > 0
        float x = ok ? min_arg_for(m - tau, a.sm_scale) : INFINITY;
        if (ok && tau >= 0.0f) {
          const float2 qn = a.qnorm[ri], qd = a.q6dn[ri];
          x = fminf(x, v - fast6_delta(qn.x, qn.y, qd.x, qd.y, knm.x, knm.y, kd.x, kd.y));
        }
        nx0[rb][i] = -x;
        if (a.row_max && (lane & 31) == 0 && ok) a.row_max[(int64_t)h * a.N + row] = m;
      }
    asm volatile("" : "+a"(nx0[0]));
  }
  // the accumulator's start and the kept test of row block rb
  auto acc0 = [&](int rb) { return rb == 0 ? nx0[0] : floatx16{}; };
  auto dropped = [&](float v, int rb, int i) {
    return (int)(__float_as_uint(rb == 0 ? v : v + nx0[rb][i]) >> 31);
  };

  // ---- K chunk copies: copy i of a chunk is issued by wave i % NW (wave-uniform bases in
  // SGPRs, one lane offset) ----
  const u32x4* khi = a.kfrag + (int64_t)kvh * (a.k_rows_pad >> 5) * S * 128;
  const u32x4* k6u = (const u32x4*)(a.k6 + (int64_t)kvh * (a.k_rows_pad >> 5) * NU * 192);
  const u32x4* k6s = (const u32x4*)(a.k6sc + (int64_t)kvh * (a.k_rows_pad >> 5) * 64);
  const uint32_t loff = (uint32_t)lane * 16u;
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  auto issue = [&](int c, u32x4* dst) {
#pragma unroll
    for (int j = 0; j < CMAX; ++j) {
      const int i = j * NW + wave_s;
      if (i < NHI) {   // (32-key block, k step) i: its 1 KB of hi units, packed
        copy16_to_lds_s(khi + (int64_t)c * SBC * S * 128 + 128 * i, loff, lds_addr(dst + 64 * i));
      } else if (i < NHI + NF6) {
        copy16_to_lds_s(k6u + (int64_t)c * F6_U + 64 * (i - NHI), loff, lds_addr(dst + HI_U + 64 * (i - NHI)));
      } else if (i == NHI + NF6 && lane < 32) {
        copy16_to_lds_s(k6s + (int64_t)c * SC_U, loff, lds_addr(dst + HI_U + F6_U));
      }
    }
  };
  // this wave's copies per chunk; wait until at most n chunks of them are in flight (vector
  // memory operations complete in order; vote stores in between only make the wait stricter)
  const bool many = (NCP - wave_s + NW - 1) / NW == CMAX;
  auto wait_copies = [&](int n) {
    constexpr int E = (7 << 4) | (15 << 8);   // expcnt / lgkmcnt: no wait
    constexpr int A1 = CMAX, A2 = 2 * CMAX, B1 = CMAX - 1, B2 = 2 * (CMAX - 1);
    if (n <= 0) __builtin_amdgcn_s_waitcnt(E);
    else if (many) {
      if (n == 1) __builtin_amdgcn_s_waitcnt(E | (A1 & 15) | ((A1 >> 4) << 14));
      else __builtin_amdgcn_s_waitcnt(E | (A2 & 15) | ((A2 >> 4) << 14));
    } else {
      if (n == 1) __builtin_amdgcn_s_waitcnt(E | (B1 & 15) | ((B1 >> 4) << 14));
      else __builtin_amdgcn_s_waitcnt(E | (B2 & 15) | ((B2 >> 4) << 14));
    }
  };
  static_assert(NBUF == 4, "wait_copies covers up to two newer chunks");

  // ---- LDS operand reads of 32-key block sb ----
  auto ldh = [&](const u32x4* buf, int sb, int s) { return buf[(sb * S + s) * 64 + lane]; };
  auto ld6 = [&](const u32x4* buf, int sb, int m) {
    const uint64_t* p = (const uint64_t*)(buf + HI_U) + (sb * NU + m) * 192 + lane;
    F6 r;
    r.p[0] = p[0];
    r.p[1] = p[64];
    r.p[2] = p[128];
    return r;
  };
  auto ldsc = [&](const u32x4* buf, int sb) { return ((const uint32_t*)(buf + HI_U + F6_U))[sb * 64 + lane]; };

  // the votes of key `key` from the dropped-row counts of this wave's row blocks (16 rows per
  // lane each; lanes l and l + 32 hold complementary rows of the same key)
  auto store_votes = [&](int key, bool check, const int* drop) {
    const bool key_ok = !check || key < a.N;
    int tot[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      int c = 0;
#pragma unroll
      for (int rb = j * T / 32; rb < (j + 1) * T / 32; ++rb) c += 16 - drop[rb];
      tot[j] = c + __shfl_xor(c, 32, 64);
    }
    if constexpr (NTW == 1) {
      if (lane < 32 && active && key_ok) vrow[key] = (uint8_t)tot[0];
    } else {
      const int j = lane >> 5;
      if (tile_ok(j) && key_ok) vrow[j * a.votes_stride + key] = (uint8_t)(lane < 32 ? tot[0] : tot[1]);
    }
  };

  // fp6 product of Q unit M with the K unit holding the other half of the [hi | x - hi] vector
  auto unit6 = [&](auto mc, const F6& b, uint32_t bsc, floatx16* acc) {
    constexpr int M = decltype(mc)::value, MB = (M + NU / 2) % NU;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma6<M, MB>(q6[rb][M], qsc[rb], b, bsc, acc[rb]);
  };
  // epilogue scores of step k (of NSTEP): the 32 scores of the previous block spread evenly
  auto epi_step = [&](auto kc, const floatx16* accO, int* drop) {
    constexpr int K = decltype(kc)::value;
    constexpr int LO = K * 16 * RB / NSTEP, HI = (K + 1) * 16 * RB / NSTEP;
#pragma unroll
    for (int idx = LO; idx < HI; ++idx) {
      const int rb = idx / 16, i = idx % 16;
      drop[rb] += dropped(accO[rb][i], rb, i);
    }
  };
  // all products of block sb into accN (fp6 units, then the bf16 k steps), the K operands read
  // one step ahead; with PREV, the previous unmasked block accO (keys keyO..) is finished between
  // the products and its votes stored
  auto block = [&](auto prevc, const u32x4* buf, int sb, floatx16* accN, const floatx16* accO, int keyO) {
    constexpr bool PREV = decltype(prevc)::value;
    int drop[RB] = {};
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) accN[rb] = acc0(rb);
    const uint32_t bsc = ldsc(buf, sb);
    F6 b6 = ld6(buf, sb, NU / 2);
    u32x4 bh{};
    static_for<0, NU>([&](auto mc) {
      constexpr int M = decltype(mc)::value;
      F6 nb6 = b6;
      if constexpr (M + 1 < NU) nb6 = ld6(buf, sb, (M + 1 + NU / 2) % NU);
      else bh = ldh(buf, sb, 0);
      unit6(mc, b6, bsc, accN);
      if constexpr (PREV) epi_step(mc, accO, drop);
      b6 = nb6;
    });
    static_for<0, S>([&](auto kc) {
      constexpr int K = decltype(kc)::value;
      u32x4 nh = bh;
      if constexpr (K + 1 < S) nh = ldh(buf, sb, K + 1);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) accN[rb] = mfma32(qhi[rb][K], bh, accN[rb]);
      if constexpr (PREV) epi_step(std::integral_constant<int, NU + K>{}, accO, drop);
      bh = nh;
    });
    if constexpr (PREV) store_votes(keyO + (lane & 31), false, drop);
    // schedule: per step, its two products with a share of the epilogue between them, the next
    // step's operand reads after the first product
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);   // scale + first fp6 unit
#pragma unroll
    for (int k = 0; k < NSTEP; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (k + 1 < NU) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
      else if (k + 1 < NSTEP) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if constexpr (PREV) __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (PREV) __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
    }
  };
  auto flush = [&](const floatx16* acc, int key0) {
    int drop[RB] = {};
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) drop[rb] += dropped(acc[rb][i], rb, i);
    store_votes(key0 + (lane & 31), false, drop);
  };

  // ---- the sweep ----
  __builtin_amdgcn_s_waitcnt(0);   // nothing the compiler tracks stays in flight into the sweep
  for (int c = 0; c < NBUF - 1 && c < nchunks; ++c) issue(c, lds[c]);
  wait_copies(min(nchunks, NBUF - 1) - 1);
  __syncthreads();
  auto chunk_begin = [&](int c) {
    if (c + NBUF - 1 < nchunks) issue(c + NBUF - 1, lds[(c + NBUF - 1) % NBUF]);
  };
  auto chunk_end = [&](int c) {   // chunk c + 1's copies have landed, every wave is done with c
    if (c + 1 < nchunks) wait_copies(min(nchunks - 1, c + NBUF - 1) - (c + 1));
    __syncthreads();
  };
  constexpr std::integral_constant<bool, true> kPrev{};
  constexpr std::integral_constant<bool, false> kNoPrev{};
  floatx16 accA[RB], accB[RB];
  int c = 0;
  for (; c < nfull; ++c) {
    chunk_begin(c);
    const u32x4* buf = lds[c % NBUF];
    if (active) {
      if (c == 0) block(kNoPrev, buf, 0, accA, accB, 0);
      else block(kPrev, buf, 0, accA, accB, c * CK - 32);
      block(kPrev, buf, 1, accB, accA, c * CK);
    }
    chunk_end(c);
  }
  if (active && nfull > 0) flush(accB, nfull * CK - 32);
  for (; c < nchunks; ++c) {   // chunks on the diagonal or past N: masked, one block at a time
    chunk_begin(c);
    const u32x4* buf = lds[c % NBUF];
    if (active) {
      for (int sb = 0; sb < SBC; ++sb) {
        const int key0 = c * CK + sb * 32;
        if (key0 >= hi_w) break;
        floatx16 acc[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb] = acc0(rb);
        const uint32_t bsc = ldsc(buf, sb);
        static_for<0, NU>([&](auto mc) {
          constexpr int M = decltype(mc)::value;
          unit6(mc, ld6(buf, sb, (M + NU / 2) % NU), bsc, acc);
        });
#pragma unroll
        for (int s = 0; s < S; ++s) {
          const u32x4 bh = ldh(buf, sb, s);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) acc[rb] = mfma32(qhi[rb][s], bh, acc[rb]);
        }
        const int key = key0 + (lane & 31);
        const int dk = key - qpos0 - (lane >> 5) * 4;   // causal: dk <= the slot's row constant
        const bool diag = key0 + 31 > qpos0;
        int drop[RB] = {};
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const bool causal = !diag || dk <= rb * 32 + (i >> 2) * 8 + (i & 3);   // exact_2.py:119
            drop[rb] += causal ? dropped(acc[rb][i], rb, i) : 1;
          }
        store_votes(key, true, drop);
      }
    }
    chunk_end(c);
  }
}

template <int D, int T>
static hipError_t launch_score6_t(const ScoreArgs& a, hipStream_t st) {
  const int rows = a.nt * T;
  const int ng = (rows + 511) / 512;
  hipLaunchKernelGGL((score6_kernel<D, T>), dim3(a.H * ng), dim3(512), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_score6(int D, int tile, const ScoreArgs& a, hipStream_t st) {
  if (D == 64 && tile == 32) return launch_score6_t<64, 32>(a, st);
  if (D == 64 && tile == 64) return launch_score6_t<64, 64>(a, st);
  if (D == 128 && tile == 32) return launch_score6_t<128, 32>(a, st);
  if (D == 128 && tile == 64) return launch_score6_t<128, 64>(a, st);
  return hipErrorInvalidValue;
}

}  // namespace sta
