// sta_dca_sel.hip -- exact-max threshold votes over the inter-chunk keys of dual chunk attention.
//
// Config 4 combines DCA's positions (dca_kernel.py:166-231, 372-489) with the shared-selection
// rule (shared_selection_triton_exact_2.py:50-140, 277-426): the keys older than the previous
// chunk -- the ones DCA's inter block attends at the constant query position (:481-487) -- are
// thresholded and top-X% selected per 64-query tile; the keys of a query's own and previous chunk
// stay dense.  Query i of chunk c = i / L sees the inter keys [0, (c - 1) L), the same range for
// every query of the chunk, so the score block of a tile is a rectangle.
//
// Scores are the DCA inter-block scores: the query rotated at the inter position and the key at
// j mod L, both already rounded to the model dtype by the rotation pre-kernel, so one bf16 (or
// fp16) product per score is exact and only the fp32 accumulation rounds (fp32 inputs keep their
// hi / lo planes: three products).
//   pass 0: raw row maxima over the inter keys (rmax)
//   pass 1: votes[t][j] = #{ i in tile t : fl(dot_ij * scale) >= fl(fl(max_i * scale) - tau) },
//           compared on the raw dot against x0 = min_arg_for(m - tau, scale), as Kernel A does
// One workgroup = one head and 256 consecutive queries in four waves of 64 (two 32-row blocks,
// Q fragments in registers); 32-key chunks are staged once in LDS for the four waves.  L is a
// multiple of 64, so a wave's 64 rows lie in one chunk and its inter range ends on a multiple of
// 64: a key chunk is entirely inside or outside it.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

template <int DT, int D, int PASS>
__global__ __launch_bounds__(256) void dca_vote_kernel(DcaVoteArgs a) {
#pragma clang fp contract(off)
  constexpr bool X3 = DT == DT_F32;
  constexpr int P = X3 ? 2 : 1;
  constexpr int S = D / 16;
  constexpr int KSTR = D + 8;                // padded LDS row (elements)
  constexpr int UNITS = P * 32 * D / 8;      // 16-byte units of one 32-key chunk
  constexpr int PER = (UNITS + 255) / 256;
  __shared__ __align__(16) uint16_t lds[2][P * 32 * KSTR];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ngroups = (a.N + 255) / 256;
  const int g = ngroups - 1 - (int)(blockIdx.x / a.H);      // longest inter ranges first
  const int h = blockIdx.x % a.H;
  const int kvh = h / (a.H / a.Hkv);
  const int wrow0 = g * 256 + wave * 64;
  const bool wave_ok = wrow0 < a.N;
  const int cq = wrow0 / a.L;
  const int ext = wave_ok && cq >= 2 ? (cq - 1) * a.L : 0;  // the wave's inter keys [0, ext)
  int ext_wg;
  {
    const int last = min(g * 256 + 255, a.N - 1);
    const int cl = last / a.L;
    ext_wg = cl >= 2 ? (cl - 1) * a.L : 0;                  // the workgroup's widest range
  }
  const int nchunks = ext_wg / 32;

  // query fragments at the inter position: A operand rows wrow0 + 32 rb + (lane & 31)
  u32x4 qh[2][S], ql[2][S];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int row = min(wrow0 + rb * 32 + (lane & 31), a.Npad - 1);
    const uint16_t* src = a.qrot + (((int64_t)(2 * a.H + h) * a.Npad + row) * P) * D + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      qh[rb][s] = *(const u32x4*)(src + s * 16);
      if constexpr (X3) ql[rb][s] = *(const u32x4*)(src + D + s * 16);
    }
  }

  // per row slot: pass 0 the running raw max, pass 1 the threshold x0 on the raw dot
  float st[2][16];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = wrow0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      if constexpr (PASS == 0) {
        st[rb][i] = -INFINITY;
      } else {
        float x0 = INFINITY;                                  // rows past N never vote
        if (row < a.N && ext > 0) {
          const float m = a.rmax[(int64_t)h * a.Npad + row] * a.scale;
          x0 = min_arg_for(m - a.tau[h], a.scale);
        }
        st[rb][i] = x0;
      }
    }

  const uint16_t* kt = a.krot + (int64_t)kvh * a.Npad * P * D;
  u32x4 pre[PER];
  auto load_chunk = [&](int c) {
    const uint16_t* src = kt + (int64_t)c * 32 * P * D;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + u * 256;
      if (e < UNITS) pre[u] = *(const u32x4*)(src + e * 8);
    }
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int e = tid + u * 256;
      if (e >= UNITS) continue;
      const int r = e / (P * D / 8), rem = e % (P * D / 8);
      const int pl = rem / (D / 8), dc = rem % (D / 8);
      *(u32x4*)(&lds[buf][(pl * 32 + r) * KSTR + dc * 8]) = pre[u];
    }
  };
  if (nchunks > 0) {
    load_chunk(0);
    store_chunk(0);
  }
  __syncthreads();
  const int tile = wrow0 / 64;
  uint8_t* vrow = a.votes + ((int64_t)h * a.nt + tile) * a.votes_stride;
  for (int c = 0; c < nchunks; ++c) {
    const int buf = c & 1;
    if (c + 1 < nchunks) load_chunk(c + 1);
    const int key0 = c * 32;
    if (key0 < ext) {                                         // wave-uniform
      floatx16 acc[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[rb][i] = 0.0f;
      const uint16_t* kr = &lds[buf][(lane & 31) * KSTR + 8 * (lane >> 5)];
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const u32x4 bh = *(const u32x4*)(kr + s * 16);
        if constexpr (X3) {
          const u32x4 bl = *(const u32x4*)(kr + 32 * KSTR + s * 16);
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) {
            acc[rb] = mfma32(ql[rb][s], bh, acc[rb]);
            acc[rb] = mfma32(qh[rb][s], bl, acc[rb]);
            acc[rb] = mfma32(qh[rb][s], bh, acc[rb]);
          }
        } else if constexpr (DT == DT_F16) {
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) acc[rb] = mfma32_f16(qh[rb][s], bh, acc[rb]);
        } else {
#pragma unroll
          for (int rb = 0; rb < 2; ++rb) acc[rb] = mfma32(qh[rb][s], bh, acc[rb]);
        }
      }
      if constexpr (PASS == 0) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int i = 0; i < 16; ++i) st[rb][i] = fmaxf(st[rb][i], acc[rb][i]);
      } else {
        int cnt = 0;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
          for (int i = 0; i < 16; ++i) cnt += acc[rb][i] >= st[rb][i] ? 1 : 0;
        cnt += __shfl_xor(cnt, 32, 64);                       // the other 32 rows of the tile
        if (lane < 32) vrow[key0 + lane] = (uint8_t)cnt;
      }
    }
    if (c + 1 < nchunks) store_chunk(buf ^ 1);
    __syncthreads();
  }

  if constexpr (PASS == 0) {
    // row maxima over the 32 lanes holding a row's keys
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float v = st[rb][i];
        v = fmaxf(v, __shfl_xor(v, 1, 64));
        v = fmaxf(v, __shfl_xor(v, 2, 64));
        v = fmaxf(v, __shfl_xor(v, 4, 64));
        v = fmaxf(v, __shfl_xor(v, 8, 64));
        v = fmaxf(v, __shfl_xor(v, 16, 64));
        const int row = wrow0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        if ((lane & 31) == 0 && row < a.N) {
          a.rmax[(int64_t)h * a.Npad + row] = v;
          if (a.row_max) a.row_max[(int64_t)h * a.N + row] = ext > 0 ? v * a.scale : -INFINITY;
        }
      }
  }
}

// The 16-bit instances: 64-key chunks of the rotated keys copied from global memory straight
// into LDS (global_load_lds_dwordx4, three chunks in flight) instead of through registers, two
// 32-key blocks per barrier.  A copy lane's 16 bytes land at a fixed LDS position, so the
// swizzle is applied on the source side: LDS granule x of key row r holds the row's granule
// x ^ (r mod G) (G granules of 8 elements per row), and the MFMA operand read of granule j of row
// r (lane r, half j & 1) finds it at position j ^ (r mod G): the 32 rows of a read fall in
// distinct bank groups.
constexpr int DV_NW = 4;                    // waves per workgroup: 256 query rows share each chunk

template <int DT, int D, int PASS>
__global__ __launch_bounds__(64 * DV_NW, 3) void dca_vote16_kernel(DcaVoteArgs a) {
#pragma clang fp contract(off)
  static_assert(DT == DT_BF16 || DT == DT_F16, "16-bit key tables");
  // +inf hidden from the optimiser: med3(x, y, pinf) = max(x, y) stays one v_med3_f32
  float pinf = INFINITY;
  asm volatile("" : "+s"(pinf));
  constexpr int S = D / 16;
  constexpr int G = D / 8;                   // 16-byte granules per key row
  constexpr int CK = 64;                     // keys per chunk
  constexpr int NBUF = 3;
  constexpr int CHUNK_G = CK * G;            // granules per chunk
  constexpr int CPW = CHUNK_G / 64 / DV_NW;  // 1 KB copies per wave and chunk
  static_assert(CPW * 64 * DV_NW == CHUNK_G, "whole copies per wave");
  __shared__ __align__(16) u32x4 lds[NBUF][CHUNK_G];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int WG_ROWS = 64 * DV_NW;
  const int ngroups = (a.N + WG_ROWS - 1) / WG_ROWS;
  const int g = ngroups - 1 - (int)(blockIdx.x / a.H);      // longest inter ranges first
  const int h = blockIdx.x % a.H;
  const int kvh = h / (a.H / a.Hkv);
  const int wrow0 = g * WG_ROWS + wave * 64;
  const bool wave_ok = wrow0 < a.N;
  const int cq = wrow0 / a.L;
  const int ext = wave_ok && cq >= 2 ? (cq - 1) * a.L : 0;  // the wave's inter keys [0, ext)
  int ext_wg;
  {
    const int last = min(g * WG_ROWS + WG_ROWS - 1, a.N - 1);
    const int cl = last / a.L;
    ext_wg = cl >= 2 ? (cl - 1) * a.L : 0;                  // the workgroup's widest range
  }
  const int nchunks = ext_wg / CK;                           // L is a multiple of 64

  u32x4 qh[2][S];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int row = min(wrow0 + rb * 32 + (lane & 31), a.Npad - 1);
    const uint16_t* src = a.qrot + ((int64_t)(2 * a.H + h) * a.Npad + row) * D + 8 * (lane >> 5);
#pragma unroll
    for (int s = 0; s < S; ++s) qh[rb][s] = *(const u32x4*)(src + s * 16);
  }
  float st[2][16];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = wrow0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      if constexpr (PASS == 0) {
        st[rb][i] = -INFINITY;
      } else {
        float x0 = INFINITY;                                  // rows past N never vote
        if (row < a.N && ext > 0) {
          const float m = a.rmax[(int64_t)h * a.Npad + row] * a.scale;
          x0 = min_arg_for(m - a.tau[h], a.scale);
        }
        st[rb][i] = x0;
      }
    }
  if (nchunks > 0) {                                        // workgroup-uniform
    // copies: wave w's e-th copy of chunk c fills LDS granules [64 u, 64 u + 64), u = e * NW + w;
    // lane L's granule p = 64 u + L is key row p / G, slot p % G, fed from the row's granule
    // (p % G) ^ (row % G)
    const uint16_t* kt = a.krot + (int64_t)kvh * a.Npad * D;
    const uint16_t* csrc[CPW];
#pragma unroll
    for (int e = 0; e < CPW; ++e) {
      const int p = (e * DV_NW + wave) * 64 + lane;
      const int r = p / G, x = p % G;
      csrc[e] = kt + (int64_t)r * D + 8 * (x ^ (r % G));
    }
    auto issue = [&](int c) {
      u32x4* dst = lds[c % NBUF];
      const int64_t off = (int64_t)c * CK * D;
#pragma unroll
      for (int e = 0; e < CPW; ++e) copy16_to_lds(csrc[e] + off, lds_addr(dst + (e * DV_NW + wave) * 64));
    };
    auto wait_copies = [&](int chunks) {     // at most `chunks` chunks of this wave's copies in flight
      constexpr int E = (7 << 4) | (15 << 8);
      if (chunks <= 0) __builtin_amdgcn_s_waitcnt(E);
      else {
        constexpr int n1 = CPW;
        if (chunks == 1) __builtin_amdgcn_s_waitcnt(E | (n1 & 15) | ((n1 >> 4) << 14));
        else {
          constexpr int n2 = 2 * CPW;
          __builtin_amdgcn_s_waitcnt(E | (n2 & 15) | ((n2 >> 4) << 14));
        }
      }
    };
    // nothing the compiler tracks may be in flight past here: its own waits then stay out of the
    // loop, whose copies it does not see
    __builtin_amdgcn_s_waitcnt(0);
    for (int c = 0; c < NBUF - 1; ++c) issue(min(c, nchunks - 1));
    wait_copies(NBUF - 2);
    __syncthreads();
    // the MFMA operand read: lane (r = lane & 31, half) reads granule 2 s + half of row r
    const int rr = lane & 31, hf = lane >> 5;
    const int tile = wrow0 / 64;
    uint8_t* vrow = a.votes + ((int64_t)h * a.nt + tile) * a.votes_stride;
    for (int c = 0; c < nchunks; ++c) {
      // chunk c + NBUF - 1 into the buffer chunk c - 1 used (every wave left it at the last
      // barrier); past the last chunk the last one is copied again into that free buffer, which
      // keeps the waits fixed
      issue(min(c + NBUF - 1, nchunks - 1));
      const u32x4* buf = lds[c % NBUF];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const int key0 = c * CK + sb * 32;
        if (key0 < ext) {                                     // wave-uniform
          floatx16 acc[2];
#pragma unroll
          for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rb][i] = 0.0f;
          const int rowp = (sb * 32 + rr) * G;
          // the K fragment of step s + 1 is read while step s's two products run
          u32x4 bh = buf[rowp + (hf ^ (rr % G))];
#pragma unroll
          for (int s = 0; s < S; ++s) {
            u32x4 nh = bh;
            if (s + 1 < S) nh = buf[rowp + ((2 * (s + 1) + hf) ^ (rr % G))];
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
              if constexpr (DT == DT_F16) acc[rb] = mfma32_f16(qh[rb][s], bh, acc[rb]);
              else acc[rb] = mfma32(qh[rb][s], bh, acc[rb]);
            }
            bh = nh;
          }
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // reads of steps 0 and 1
#pragma unroll
          for (int s = 0; s < S; ++s) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0); // step s's products
            if (s + 2 < S) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // step s + 2's read
          }
          if constexpr (PASS == 0) {
            // max(st, acc) as one v_med3_f32 (scores are finite; fmaxf canonicalises both inputs)
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
              for (int i = 0; i < 16; ++i) st[rb][i] = __builtin_amdgcn_fmed3f(acc[rb][i], st[rb][i], pinf);
          } else {
            int cnt = 0;
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
              for (int i = 0; i < 16; ++i) cnt += acc[rb][i] >= st[rb][i] ? 1 : 0;
            cnt += __shfl_xor(cnt, 32, 64);                   // the other 32 rows of the tile
            if (lane < 32) vrow[key0 + lane] = (uint8_t)cnt;
          }
        }
      }
      wait_copies(NBUF - 2);                                  // chunk c + 1 has landed
      __syncthreads();                                        // and every wave is done with c
    }
    wait_copies(0);                                           // the stray copies drain
  }
  if constexpr (PASS == 0) {
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float v = st[rb][i];
        v = fmaxf(v, __shfl_xor(v, 1, 64));
        v = fmaxf(v, __shfl_xor(v, 2, 64));
        v = fmaxf(v, __shfl_xor(v, 4, 64));
        v = fmaxf(v, __shfl_xor(v, 8, 64));
        v = fmaxf(v, __shfl_xor(v, 16, 64));
        const int row = wrow0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        if ((lane & 31) == 0 && row < a.N) {
          a.rmax[(int64_t)h * a.Npad + row] = v;
          if (a.row_max) a.row_max[(int64_t)h * a.N + row] = ext > 0 ? v * a.scale : -INFINITY;
        }
      }
  }
}

template <int DT, int D>
static hipError_t launch_dca_votes_t(const DcaVoteArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)(((a.N + 255) / 256) * a.H));
  if constexpr (DT == DT_F32) {
    hipLaunchKernelGGL((dca_vote_kernel<DT, D, 0>), grid, dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((dca_vote_kernel<DT, D, 1>), grid, dim3(256), 0, st, a);
  } else {
    if (a.L % 64 != 0) return hipErrorInvalidValue;
    const dim3 grid16((unsigned)(((a.N + 64 * DV_NW - 1) / (64 * DV_NW)) * a.H));
    hipLaunchKernelGGL((dca_vote16_kernel<DT, D, 0>), grid16, dim3(64 * DV_NW), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((dca_vote16_kernel<DT, D, 1>), grid16, dim3(64 * DV_NW), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_dca_votes(int dtype, int D, const DcaVoteArgs& a, hipStream_t st) {
#define STA_DV(DT_, D_) if (dtype == DT_ && D == D_) return launch_dca_votes_t<DT_, D_>(a, st);
  STA_DV(DT_F32, 64) STA_DV(DT_F32, 128) STA_DV(DT_BF16, 64) STA_DV(DT_BF16, 128)
  STA_DV(DT_F16, 64) STA_DV(DT_F16, 128)
#undef STA_DV
  return hipErrorInvalidValue;
}

}  // namespace sta
