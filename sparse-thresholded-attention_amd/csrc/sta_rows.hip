// sta_rows.hip -- per-key scores of a batch of queries on the matrix cores.
//
// The per-query selection rules (shared_selection_triton_exact_2.py:527-604,
// shared_selection_triton_perquery.py:651-720) take each query's full row of scores
// fl(dot(rot(q), rot(k)) * sm_scale) over the keys it sees.  For one or a few decode queries the
// decode score kernel computes them with fp32 dots; for a batch of queries -- the per-query
// prefill (every prompt position, perquery.py:905-924) -- this kernel computes them as a
// matrix product on the rotated hi / lo bf16 fragments of the RoPE pre-kernel:
//   dot = lo(q) . hi(k) + hi(q) . lo(k) + hi(q) . hi(k)
// with fp32 accumulation in v_mfma_f32_32x32x16_bf16, the score kernel's pass-2 product (error
// <= 3 * 2^-16 * sum |q_i k_i|, about 1e-6 on unit-scale rows).
//
// One workgroup = one head, 256 consecutive queries in four waves of 64 (two 32-row blocks,
// whose Q fragments stay in registers) and one piece of at most ROWS_PIECE 32-key chunks of the
// keys those queries see: a group's key range is split so that a launch over a few heads still
// has thousands of equal workgroups (a group per workgroup gave one head pair 128 workgroups of
// 1 to 64 units of work).  Every wave reads the chunks from LDS: the next chunk's fragments are
// loaded into registers while the current chunk's products run, then stored into the other LDS
// buffer.  Query i sees the keys [0, M - (Q - 1 - i)) (its cache prefix: [0, q_pos0 + i] when the
// batch ends at the cache's last key); scores past that are not written.
// Each wave's 64 x 32 block of scores goes out through a per-wave LDS tile: written in the matrix
// cores' output layout, read back as four consecutive keys per lane, so that a row's 32 scores
// leave in 16-byte stores (8 lanes per row) rather than 4-byte ones (the store data path moves
// about as many bytes per instruction at 16 bytes per lane as at 4).  Row-major (H, Q, M) rows
// put each row's 128 bytes of a block 4M bytes from the next row's; in the tiled layout
// (score_tile_row, for scores that only the selection reads) the block's rows lie 512 bytes
// apart inside one 32 KB tile, which the memory writes at a higher rate.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

constexpr int ROWS_PIECE = 32;               // 32-key chunks per workgroup
constexpr int ROWS_TS = 40;                  // tile row stride in floats: 16-byte rows, and the
                                             // two row groups of one write 32 banks apart

template <int D>
__global__ __launch_bounds__(256) void score_rows_kernel(RowsArgs a, int npieces) {
  constexpr int S = D / 16;                  // k steps of 16
  constexpr int CH = S * 2 * 64;             // 16-byte units of one 32-key block (hi, lo)
  constexpr int PER = CH / 256;              // units per thread and chunk
  __shared__ u32x4 lds[2][CH];
  __shared__ __align__(16) float tile[4][64 * ROWS_TS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = (int)blockIdx.x / npieces, piece = (int)blockIdx.x % npieces;
  const int h = blockIdx.y;
  const int kvh = h / (a.H / a.Hkv);
  const int r0 = g * 256;
  const int wrow0 = r0 + wave * 64;
  const int last_row = min(r0 + 256, a.Q) - 1;
  // row i sees the keys [0, m_i), m_i = M - (Q - 1 - i): the cache prefix of the decode contract
  const int kend = a.M - (a.Q - 1 - last_row);            // keys any row of the group sees
  const int c0 = piece * ROWS_PIECE;
  const int c1 = min((kend + 31) / 32, c0 + ROWS_PIECE);  // this piece's chunks [c0, c1)
  if (c0 >= c1) return;                                   // uniform: the group's keys end earlier
  const int wlast = min(wrow0 + 63, a.Q - 1);
  const int wkend = wrow0 < a.Q ? a.M - (a.Q - 1 - wlast) : 0;

  // the wave's Q fragments: two 32-row blocks x S steps x (hi, lo)
  u32x4 qh[2][S], ql[2][S];
  const int qblocks = a.q_rows_pad >> 5;
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int blk = (wrow0 >> 5) + rb;
    const u32x4* src = a.qfrag + ((int64_t)h * qblocks + blk) * S * 128 + lane;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (blk < qblocks) {
        qh[rb][s] = src[s * 128];
        ql[rb][s] = src[s * 128 + 64];
      } else {
        qh[rb][s] = u32x4{0, 0, 0, 0};
        ql[rb][s] = u32x4{0, 0, 0, 0};
      }
    }
  }

  const u32x4* kf = a.kfrag + (int64_t)kvh * (a.k_rows_pad >> 5) * CH;
  u32x4 pre[PER];
  auto load_chunk = [&](int c) {
#pragma unroll
    for (int e = 0; e < PER; ++e) pre[e] = kf[(int64_t)c * CH + e * 256 + tid];
  };
  auto store_chunk = [&](int buf) {
#pragma unroll
    for (int e = 0; e < PER; ++e) lds[buf][e * 256 + tid] = pre[e];
  };
  load_chunk(c0);
  store_chunk(0);
  __syncthreads();
  // 16-byte stores need every row start 16-byte aligned (tiles: 128-byte rows)
  const bool vec = (a.tiles || (a.M & 3) == 0) && ((uintptr_t)a.scores & 15) == 0;
  for (int c = c0; c < c1; ++c) {
    const int buf = (c - c0) & 1;
    if (c + 1 < c1) load_chunk(c + 1);
    const int key0 = c * 32;
    if (key0 < wkend) {                      // wave-uniform: some row of the wave sees the chunk
      floatx16 acc[2];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[rb][i] = 0.0f;
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const u32x4 bh = lds[buf][s * 128 + lane];
        const u32x4 bl = lds[buf][s * 128 + 64 + lane];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
          acc[rb] = mfma32(ql[rb][s], bh, acc[rb]);
          acc[rb] = mfma32(qh[rb][s], bl, acc[rb]);
          acc[rb] = mfma32(qh[rb][s], bh, acc[rb]);
        }
      }
      float* t = tile[wave];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          t[(rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3)) * ROWS_TS + (lane & 31)] = acc[rb][i] * a.sm_scale;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // lane: row k * 8 + lane / 8 of the wave's 64, keys key0 + 4 (lane % 8) .. + 3
      const int kq = key0 + 4 * (lane & 7);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int r = k * 8 + (lane >> 3);
        const float4 v = *(const float4*)&t[r * ROWS_TS + 4 * (lane & 7)];
        const int row = wrow0 + r;
        const int mrow = a.M - (a.Q - 1 - row);  // the keys this row sees
        if (row < a.Q && kq < mrow) {
          float* dst = a.tiles ? a.scores + score_tile_row(h, row, a.Q, a.M) +
                                     ((int64_t)(kq >> SCORE_TW_LG) << (6 + SCORE_TW_LG)) + (kq & (SCORE_TW - 1))
                               : a.scores + ((int64_t)h * a.Q + row) * a.M + kq;
          if (vec && kq + 3 < mrow) {
            // written once, read once by the selection: non-temporal, past the caches' allocation
            __builtin_nontemporal_store(floatx4{v.x, v.y, v.z, v.w}, (floatx4*)dst);
          } else {
            dst[0] = v.x;
            if (kq + 1 < mrow) dst[1] = v.y;
            if (kq + 2 < mrow) dst[2] = v.z;
            if (kq + 3 < mrow) dst[3] = v.w;
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");   // the reads before the next writes
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (c + 1 < c1) store_chunk(buf ^ 1);   // that buffer was last read before the barrier
    __syncthreads();
  }
}

hipError_t launch_score_rows(int D, const RowsArgs& a, hipStream_t st) {
  // pieces of the longest group (its last row sees all M keys); shorter groups leave the tail of
  // their pieces empty
  const int npieces = ((a.M + 31) / 32 + ROWS_PIECE - 1) / ROWS_PIECE;
  const dim3 grid((unsigned)((a.Q + 255) / 256 * npieces), (unsigned)a.H);
  if (D == 64) hipLaunchKernelGGL(score_rows_kernel<64>, grid, dim3(256), 0, st, a, npieces);
  else if (D == 128) hipLaunchKernelGGL(score_rows_kernel<128>, grid, dim3(256), 0, st, a, npieces);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace sta
