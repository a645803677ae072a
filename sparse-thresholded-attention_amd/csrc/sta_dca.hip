// sta_dca.hip -- dual chunk attention (DCA) prefill: dense causal attention whose RoPE positions
// are remapped by chunk distance so no relative distance exceeds the pretraining window.
//
// Reference: dca_kernel.py.  Keys sit at j mod L (L = chunk_size - local_window); a query i
// scores keys of its own chunk at i mod L (intra), keys of the previous chunk at
// min(i mod L + L, chunk_size) (succ) and older keys at min(2L - 1, chunk_size) (inter); the
// tables are cos / sin of fl(t * inv_freq) times mscale, cast to the model dtype (:166-231), and
// the rotation x*cos + rotate_half(x)*sin runs in the model dtype (:278-286).  The reference runs
// three attention blocks per query chunk and merges them by log-sum-exp (:453-489), which is one
// softmax over all causal keys: here one online-softmax sweep over the keys, switching the
// query's position variant as the sweep crosses chunk boundaries.
//
// Launches: dca_rope_kernel (keys once, queries in their three variants, table semantics and
// rounding of the reference), then dca_attn_kernel: one workgroup = one head and G consecutive
// 32-query tiles (wave w owns rows 32 (g G + w) .. +31), 64-key blocks staged once in LDS
// (double-buffered, V transposed) and read by all G waves.  S^T = K . Q^T (32x32x16 MFMA, lane =
// query), so the softmax weights are already the B operand of O^T += V^T . P^T.
// Requires L % 64 == 0: every 32-query tile and every 64-key block then lies in one chunk.
#include "sta_dca_rot.h"
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

// ------------------------------------------------------------------------------------------
// Rotated keys (variant -1) and queries (variants 0 intra, 1 succ, 2 inter).  out layout:
// keys (Hkv, Npad, P, D), queries (3, H, Npad, P, D); P = 2 (bf16 hi / lo) for fp32 inputs,
// else the model dtype.  Rows >= N are zero.
// ------------------------------------------------------------------------------------------
// The table of every position the remap produces, t = 0 .. chunk_size (keys t < L, queries up
// to the succ / inter clamps): entry (t, f) = (cos, sin) of fl(t * inv_freq[f]) times mscale in
// the model dtype (dca_table_entry).  One sin / cos per (t, f) instead of one per (head, row, f).
template <int DT, int D>
__global__ __launch_bounds__(256) void dca_table_kernel(const float* __restrict__ inv_freq, float mscale,
                                                        int chunk_size, float2* __restrict__ table) {
  const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (x >= (int64_t)(chunk_size + 1) * (D / 2)) return;
  const int t = (int)(x / (D / 2)), f = (int)(x % (D / 2));
  float cs, sn;
  dca_table_entry<DT>(t, inv_freq[f], mscale, cs, sn);
  table[x] = make_float2(cs, sn);
}

template <int DT, int D>
__global__ __launch_bounds__(256) void dca_rope_kernel(const void* __restrict__ x, int64_t head_stride,
                                                       int64_t tok_stride, int heads, int N, int Npad,
                                                       int L, int chunk_size, int is_key,
                                                       const float2* __restrict__ table,
                                                       uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
  constexpr int C = D / 8;
  constexpr int P = DT == DT_F32 ? 2 : 1;
  // one thread per (head, row, 8-dim group): the row's input is read once and rotated at the key
  // position, or at the three query positions
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)heads * Npad * C) return;
  const int c = (int)(gid % C);
  const int64_t r = gid / C;
  const int row = (int)(r % Npad);
  const int head = (int)(r / Npad);
  const int d0 = c * 8;
  const bool first = d0 < D / 2;
  const int i0 = first ? d0 : d0 - D / 2;
  float a[8], b[8];
  if (row < N) {
    const int64_t base = (int64_t)head * head_stride + (int64_t)row * tok_stride;
    load8<DT>(x, base + i0, a);
    load8<DT>(x, base + D / 2 + i0, b);
  }
  const int variants = is_key ? 1 : 3;
  for (int var = 0; var < variants; ++var) {
    float o[8];
    if (row < N) {
      int t;
      if (is_key) {
        t = row % L;                                               // dca_kernel.py:187-190
      } else {
        const int pid = row % L;
        if (var == 0) t = pid;                                     // :181-182
        else if (var == 1) t = min(pid + L, chunk_size);           // :185-186
        else t = min(2 * L - 1, chunk_size);                       // the clamped index L-1, :464-467
      }
      float cs[8], sn[8];
      const float4* tr = (const float4*)(table + (int64_t)t * (D / 2) + i0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float4 v = tr[e];
        cs[2 * e] = v.x;
        sn[2 * e] = v.y;
        cs[2 * e + 1] = v.z;
        sn[2 * e + 1] = v.w;
      }
      dca_rot8_cs<DT>(a, b, cs, sn, first, o);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = 0.0f;
    }
    uint16_t* dst = out + ((((int64_t)var * heads + head) * Npad + row) * P) * D + d0;
    if constexpr (DT == DT_F32) {
      u32x4 hi, lo;
      split_bf16x8(o, hi, lo);
      *(u32x4*)dst = hi;
      *(u32x4*)(dst + D) = lo;
    } else if constexpr (DT == DT_F16) {
      *(u32x4*)dst = pack_f16x8(o);
    } else {
      *(u32x4*)dst = pack_bf16x8(o);
    }
  }
}

// ------------------------------------------------------------------------------------------
// the attention sweep
// ------------------------------------------------------------------------------------------
template <int DT, int D, int G, int BNV = 64>
struct DcaCfg {
  static constexpr int BN = BNV;                    // keys per block
  static constexpr bool X3 = DT == DT_F32;
  static constexpr int P = X3 ? 2 : 1;
  static constexpr int NTH = G * 64;
  static constexpr int KSTR = D + 8;
  using VL = VtLayout<BN>;   // V^T LDS layout (swizzled)
  static constexpr int VSTR = VL::STR;
  static constexpr int KBUF = P * BN * KSTR;
  static constexpr int VBUF = P * D * VSTR;
  static constexpr int KUNITS = P * BN * D / 8;
  static constexpr int KU = (KUNITS + NTH - 1) / NTH;
  static constexpr int VUNITS = (BN / 4) * (D / 8);
  static constexpr int VU = (VUNITS + NTH - 1) / NTH;
  static constexpr size_t lds_bytes = (size_t)2 * (KBUF + VBUF) * 2;
};

// MODE 0: dense DCA attention (every causal key).
// MODE 1 (config 4, selected inter keys): one workgroup = one 64-query selection tile (G = 2);
//   the sweep runs over the tile's selected inter keys idx[h][t][0 .. min(kept, k_max)), gathered
//   block by block, with the inter query variant, and leaves each row's unnormalised softmax
//   state (o, m, l) in a.state.
// MODE 2 (config 4, local keys): as MODE 0 over the keys of the query's own and previous chunk
//   only ([max(0, (c - 1) L), i]), starting from the MODE 1 state of each row.
// keys per block: 64, or 32 for the selected instance, whose two waves stage each block alone
// (half the staging registers; its workgroups hold one wave per SIMD at 64)
constexpr int dca_block_keys(int mode) { return mode == 1 ? 32 : 64; }

template <int DT, int D, int G, int MODE = 0>
__global__ __launch_bounds__(G * 64, (MODE == 1 && DT != DT_F32) ? 2 : 1) void dca_attn_kernel(DcaArgs a) {
#pragma clang fp contract(off)
  using Cfg = DcaCfg<DT, D, G, dca_block_keys(MODE)>;
  constexpr int BN = Cfg::BN;
  constexpr bool X3 = Cfg::X3;
  constexpr int P = Cfg::P, NTH = Cfg::NTH, KSTR = Cfg::KSTR, VSTR = Cfg::VSTR;
  constexpr int KS = D / 16;
  constexpr int NSB = BN / 32;
  constexpr int RBS = D / 32;
  constexpr int KU = Cfg::KU, VU = Cfg::VU;
  extern __shared__ __align__(16) uint16_t sm[];
  auto kbuf = [&](int p) { return sm + p * (Cfg::KBUF + Cfg::VBUF); };
  auto vbuf = [&](int p) { return sm + p * (Cfg::KBUF + Cfg::VBUF) + Cfg::KBUF; };

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hf = lane >> 5, q = lane & 31;
  const int nt = (a.N + 31) / 32;
  const int ngroups = (nt + G - 1) / G;
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
  const int kvh = h / (a.H / a.Hkv);
  const int N = a.N, L = a.L;
  const int t = g * G + wave;
  const bool tile_ok = t < nt;
  const int r0 = t * 32;
  const int row = r0 + q;
  const bool row_ok = tile_ok && row < N;
  const int cq = r0 / L;                                          // the tile's chunk
  // MODE 1: the selection tile's valid slots; MODE 2: the first local key
  const int nsel = MODE == 1 ? min(a.kept_size[(int64_t)h * a.nt64 + g], a.k_max) : 0;
  const int kstart = MODE == 2 && cq >= 2 ? (cq - 1) * L : 0;
  const int nblk = MODE == 1 ? (nsel + BN - 1) / BN
                             : (tile_ok ? min(r0 + 31, N - 1) / BN + 1 : 0);   // keys 0 .. last row
  const int t_last = min(g * G + G - 1, nt - 1);
  const int nb_wg = MODE == 1 ? nblk : min(t_last * 32 + 31, N - 1) / BN + 1;
  // MODE 2: the workgroup's sweep starts at its first tile's first local key (a multiple of 64)
  const int b_begin = MODE == 2 ? ((g * G * 32) / L >= 2 ? ((g * G * 32) / L - 1) * L / BN : 0) : 0;
  const int32_t* sel = MODE == 1 ? a.idx + ((int64_t)h * a.nt64 + g) * a.k_max : nullptr;

  // ---- query fragments of the current position variant (B operand, dims 16s + 8hf + e) ----
  u32x4 qf[KS], qfl[KS];
  int cur_var = -1;
  auto load_q = [&](int var) {
    const uint16_t* src = a.qrot + ((((int64_t)var * a.H + h) * a.Npad + (row_ok ? row : 0)) * P) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qf[s] = *(const u32x4*)(src + s * 16 + 8 * hf);
      if constexpr (X3) qfl[s] = *(const u32x4*)(src + D + s * 16 + 8 * hf);
    }
  };

  // ---- staging of K / V blocks into LDS (all threads) ----
  const uint16_t* kt = a.krot + (int64_t)kvh * a.Npad * P * D;
  const int64_t vhb = (int64_t)kvh * a.v_head_stride;
  u32x4 kreg[KU];
  Raw8<DT> vreg[VU][4];
  // the key of block b's slot r: contiguous keys, or (MODE 1) the selected inter keys, with
  // -1 past the tile's valid slots
  auto key_of = [&](int b, int r) -> int {
    if constexpr (MODE == 1) {
      const int s = b * BN + r;
      return s < nsel ? sel[s] : -1;
    } else {
      const int j = b * BN + r;
      return j < N ? j : -1;
    }
  };
  auto load_block = [&](int b) {
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int e = tid + u * NTH;
      if (e < Cfg::KUNITS) {
        if constexpr (MODE == 1) {
          const int r = e / (P * D / 8), rem = e % (P * D / 8);
          const int j = key_of(b, r);
          kreg[u] = j >= 0 ? *(const u32x4*)(kt + (int64_t)j * P * D + rem * 8) : u32x4{0, 0, 0, 0};
        } else {
          kreg[u] = *(const u32x4*)(kt + (int64_t)b * BN * P * D + e * 8);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int e = tid + u * NTH;
      const int sg = e / (D / 8), dc = e % (D / 8);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = e < Cfg::VUNITS ? key_of(b, sg * 4 + k) : -1;
        if (j >= 0) vreg[u][k].load(a.v, vhb + (int64_t)j * a.v_tok_stride + dc * 8);
        else vreg[u][k].zero();
      }
    }
  };
  auto store_block = [&](int p) {
    uint16_t* kd = kbuf(p);
    uint16_t* vd = vbuf(p);
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int e = tid + u * NTH;
      if (e >= Cfg::KUNITS) continue;
      const int r = e / (P * D / 8), rem = e % (P * D / 8);
      const int pl = rem / (D / 8), dc = rem % (D / 8);
      *(u32x4*)(kd + pl * BN * KSTR + r * KSTR + dc * 8) = kreg[u];
    }
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int e = tid + u * NTH;
      if (e >= Cfg::VUNITS) continue;
      const int sg = e / (D / 8), dc = e % (D / 8);
      if constexpr (!X3) {   // 16-bit storage: transpose the raw bits
        u32x2 cols[8];
        transpose4x8_16(vreg[u][0].w, vreg[u][1].w, vreg[u][2].w, vreg[u][3].w, cols);
#pragma unroll
        for (int e8 = 0; e8 < 8; ++e8) *(u32x2*)(vd + Cfg::VL::off(dc * 8 + e8, sg)) = cols[e8];
      } else {              // fp32: bf16 hi and lo planes
        float vv[4][8];
#pragma unroll
        for (int k = 0; k < 4; ++k) vreg[u][k].to_f32(vv[k]);
#pragma unroll
        for (int e8 = 0; e8 < 8; ++e8) {
          u32x2 w, wl;
          w[0] = pack2_bf16(vv[0][e8], vv[1][e8]);
          w[1] = pack2_bf16(vv[2][e8], vv[3][e8]);
          float lo[4];
#pragma unroll
          for (int k = 0; k < 4; ++k) lo[k] = vv[k][e8] - bf16_bits_to_f32(f32_to_bf16_bits(vv[k][e8]));
          wl[0] = pack2_bf16(lo[0], lo[1]);
          wl[1] = pack2_bf16(lo[2], lo[3]);
          *(u32x2*)(vd + Cfg::VL::off(dc * 8 + e8, sg)) = w;
          *(u32x2*)(vd + D * VSTR + Cfg::VL::off(dc * 8 + e8, sg)) = wl;
        }
      }
    }
  };

  floatx16 oacc[RBS];
#pragma unroll
  for (int rb = 0; rb < RBS; ++rb) oacc[rb] = floatx16{};
  float mR = -INFINITY, l_i = 0.0f;
  // state row of this lane's query (D + 4 floats, 16-byte rows): o (unnormalised), m, l
  float* srow = (MODE != 0 && row_ok) ? a.state + ((int64_t)h * a.Npad + row) * (D + 4) : nullptr;
  if constexpr (MODE == 2) {
    if (srow) {
#pragma unroll
      for (int rb = 0; rb < RBS; ++rb)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const float4 o = *(const float4*)(srow + rb * 32 + g4 * 8 + 4 * hf);
          oacc[rb][g4 * 4 + 0] = o.x;
          oacc[rb][g4 * 4 + 1] = o.y;
          oacc[rb][g4 * 4 + 2] = o.z;
          oacc[rb][g4 * 4 + 3] = o.w;
        }
      mR = srow[D];
      l_i = srow[D + 1];
    }
  }

  if (b_begin < nb_wg) {
    load_block(b_begin);
    store_block(b_begin & 1);
  }
  __syncthreads();

  for (int b = b_begin; b < nb_wg; ++b) {
    const int p = b & 1;
    const bool more = b + 1 < nb_wg;
    if (more) load_block(b + 1);
    if (tile_ok && b < nblk && b * BN >= kstart) {
      const int start = b * BN;
      const int di = cq - start / L;                               // chunk distance of the block
      const int var = MODE == 1 ? 2 : (di == 0 ? 0 : (di == 1 ? 1 : 2));
      if (var != cur_var) {                                        // inter -> succ -> intra
        load_q(var);
        cur_var = var;
      }
      const uint16_t* kr = kbuf(p);
      floatx16 sacc[NSB];
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb) {
        sacc[sb] = floatx16{};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int off = (sb * 32 + q) * KSTR + s * 16 + 8 * hf;
          const u32x4 kh = *(const u32x4*)(kr + off);
          if constexpr (X3) {
            const u32x4 kl = *(const u32x4*)(kr + BN * KSTR + off);
            sacc[sb] = mfma32(kl, qf[s], sacc[sb]);
            sacc[sb] = mfma32(kh, qfl[s], sacc[sb]);
            sacc[sb] = mfma32(kh, qf[s], sacc[sb]);
          } else if constexpr (DT == DT_F16) {
            sacc[sb] = mfma32_f16(kh, qf[s], sacc[sb]);
          } else {
            sacc[sb] = mfma32(kh, qf[s], sacc[sb]);
          }
        }
      }
      // causal mask only where the block reaches the tile's rows (intra chunk, :411-413); the
      // selected inter keys all precede the tile, only slots past the valid ones are masked.
      // The running max mR stays in raw dot units and the weights are exp2((s - mR) * c2) with
      // c2 = scale * log2(e): one FMA and one exp2 per score (scale > 0, so the raw max orders as
      // the scaled one).
      const bool diag = MODE == 1 ? start + BN > nsel : start + BN - 1 > r0;   // wave-uniform
      float bmax = -INFINITY;
      if (diag) {
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = start + sb * 32 + (i >> 2) * 8 + 4 * hf + (i & 3);
            const bool ok = MODE == 1 ? key < nsel : key <= row;
            const float v = ok ? sacc[sb][i] : -INFINITY;
            sacc[sb][i] = v;
            bmax = fmaxf(bmax, v);
          }
      } else {
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) bmax = fmaxf(bmax, sacc[sb][i]);
      }
      bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
      const float c2 = a.scale * 1.4426950408889634f;
      const float mnew = fmaxf(mR, bmax);
      const float mc = (mnew == -INFINITY) ? 0.0f : mnew * c2;   // exponent origin
      const float alpha = __builtin_amdgcn_exp2f(mR * c2 - mc);  // mR = -inf: 0
      float psum = 0.0f;
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[sb][i], c2, -mc));
          sacc[sb][i] = pv;
          psum += pv;
        }
      psum += __shfl_xor(psum, 32, 64);
      l_i = l_i * alpha + psum;
      mR = mnew;
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int rb = 0; rb < RBS; ++rb) oacc[rb] *= alpha;
      }
      const uint16_t* vt = vbuf(p);
#pragma unroll
      for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          float pv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) pv[e] = sacc[sb][kk * 8 + e];
          u32x4 pb, pbl;
          if constexpr (DT == DT_F16) pb = pack_f16x8(pv);
          else if constexpr (X3) split_bf16x8(pv, pb, pbl);
          else pb = pack_bf16x8(pv);
          const int c0 = sb * 32 + kk * 16 + 4 * hf, c1 = c0 + 8;
#pragma unroll
          for (int rb = 0; rb < RBS; ++rb) {
            const int r = rb * 32 + q;
            const int o0 = Cfg::VL::off(r, c0 >> 2), o1 = Cfg::VL::off(r, c1 >> 2);
              const u32x2 a0 = *(const u32x2*)(vt + o0);
            const u32x2 a1 = *(const u32x2*)(vt + o1);
            const u32x4 va = u32x4{a0[0], a0[1], a1[0], a1[1]};
            if constexpr (DT == DT_F16) {
              oacc[rb] = mfma32_f16(va, pb, oacc[rb]);
            } else if constexpr (X3) {
              const u32x2 b0 = *(const u32x2*)(vt + D * VSTR + o0);
              const u32x2 b1 = *(const u32x2*)(vt + D * VSTR + o1);
              const u32x4 vl = u32x4{b0[0], b0[1], b1[0], b1[1]};
              oacc[rb] = mfma32(vl, pb, oacc[rb]);
              oacc[rb] = mfma32(va, pbl, oacc[rb]);
              oacc[rb] = mfma32(va, pb, oacc[rb]);
            } else {
              oacc[rb] = mfma32(va, pb, oacc[rb]);
            }
          }
        }
    }
    if (more) store_block(p ^ 1);
    __syncthreads();
  }

  if constexpr (MODE == 1) {
    if (srow) {
#pragma unroll
      for (int rb = 0; rb < RBS; ++rb)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4)
          *(float4*)(srow + rb * 32 + g4 * 8 + 4 * hf) =
              make_float4(oacc[rb][g4 * 4], oacc[rb][g4 * 4 + 1], oacc[rb][g4 * 4 + 2], oacc[rb][g4 * 4 + 3]);
      if (hf == 0) {
        srow[D] = mR;
        srow[D + 1] = l_i;
      }
    }
    return;
  }
  if (row_ok) {
    const int64_t ob = ((int64_t)h * N + row) * D;
#pragma unroll
    for (int rb = 0; rb < RBS; ++rb)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int d0 = rb * 32 + g4 * 8 + 4 * hf;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = oacc[rb][g4 * 4 + e] / l_i;
        if constexpr (DT == DT_F32) {
          *(float4*)((float*)a.out + ob + d0) = make_float4(o[0], o[1], o[2], o[3]);
        } else if constexpr (DT == DT_BF16) {
          u32x2 w;
          w[0] = pack2_bf16(o[0], o[1]);
          w[1] = pack2_bf16(o[2], o[3]);
          *(u32x2*)((uint16_t*)a.out + ob + d0) = w;
        } else {
          u32x2 w;
          w[0] = pack2_f16(o[0], o[1]);
          w[1] = pack2_f16(o[2], o[3]);
          *(u32x2*)((uint16_t*)a.out + ob + d0) = w;
        }
      }
  }
}

// ------------------------------------------------------------------------------------------
// host launchers
// ------------------------------------------------------------------------------------------
size_t dca_table_bytes(int D, int chunk_size) { return (size_t)(chunk_size + 1) * (D / 2) * sizeof(float2); }

template <int DT, int D>
static hipError_t launch_dca_table_t(const float* inv_freq, float mscale, int chunk_size, float2* table,
                                     hipStream_t st) {
  const int64_t total = (int64_t)(chunk_size + 1) * (D / 2);
  hipLaunchKernelGGL((dca_table_kernel<DT, D>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, inv_freq,
                     mscale, chunk_size, table);
  return hipGetLastError();
}

hipError_t launch_dca_table(int dtype, int D, const float* inv_freq, float mscale, int chunk_size, float2* table,
                            hipStream_t st) {
#define STA_DT(DT_, D_) \
  if (dtype == DT_ && D == D_) return launch_dca_table_t<DT_, D_>(inv_freq, mscale, chunk_size, table, st);
  STA_DT(DT_F32, 64) STA_DT(DT_F32, 128) STA_DT(DT_BF16, 64) STA_DT(DT_BF16, 128)
  STA_DT(DT_F16, 64) STA_DT(DT_F16, 128)
#undef STA_DT
  return hipErrorInvalidValue;
}

template <int DT, int D>
static hipError_t launch_dca_rope_t(const void* x, int64_t hs, int64_t ts, int heads, int N, int Npad, int L,
                                    int chunk_size, int is_key, const float2* table, uint16_t* out,
                                    hipStream_t st) {
  const int64_t total = (int64_t)heads * Npad * (D / 8);
  hipLaunchKernelGGL((dca_rope_kernel<DT, D>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, hs,
                     ts, heads, N, Npad, L, chunk_size, is_key, table, out);
  return hipGetLastError();
}

hipError_t launch_dca_rope(int dtype, int D, const void* x, int64_t hs, int64_t ts, int heads, int N, int Npad,
                           int L, int chunk_size, int is_key, const float2* table, uint16_t* out,
                           hipStream_t st) {
#define STA_DR(DT_, D_) \
  if (dtype == DT_ && D == D_) \
    return launch_dca_rope_t<DT_, D_>(x, hs, ts, heads, N, Npad, L, chunk_size, is_key, table, out, st);
  STA_DR(DT_F32, 64) STA_DR(DT_F32, 128) STA_DR(DT_BF16, 64) STA_DR(DT_BF16, 128)
  STA_DR(DT_F16, 64) STA_DR(DT_F16, 128)
#undef STA_DR
  return hipErrorInvalidValue;
}

constexpr int kDcaTiles = 8;   // 32-query tiles (waves) per workgroup

size_t dca_lds_bytes(int dtype, int D) {
#define STA_DL(DT_, D_) if (dtype == DT_ && D == D_) return DcaCfg<DT_, D_, kDcaTiles>::lds_bytes;
  STA_DL(DT_F32, 64) STA_DL(DT_F32, 128) STA_DL(DT_BF16, 64) STA_DL(DT_BF16, 128)
  STA_DL(DT_F16, 64) STA_DL(DT_F16, 128)
#undef STA_DL
  return 0;
}

template <int DT, int D, int G, int MODE>
static hipError_t launch_dca_attn_g(const DcaArgs& a, hipStream_t st) {
  using Cfg = DcaCfg<DT, D, G, dca_block_keys(MODE)>;
  hipError_t e = hipFuncSetAttribute((const void*)dca_attn_kernel<DT, D, G, MODE>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cfg::lds_bytes);
  if (e != hipSuccess) return e;
  const int nt = (a.N + 31) / 32;
  const int ngroups = (nt + G - 1) / G;
  hipLaunchKernelGGL((dca_attn_kernel<DT, D, G, MODE>), dim3(a.H * ngroups), dim3(Cfg::NTH), Cfg::lds_bytes,
                     st, a);
  return hipGetLastError();
}

// dense (a.state == null), or config 4's two sweeps: the selected inter keys of each 64-query
// tile (two waves per workgroup), then the local keys from the partial states
template <int DT, int D>
static hipError_t launch_dca_attn_t(const DcaArgs& a, hipStream_t st) {
  if (!a.state) return launch_dca_attn_g<DT, D, kDcaTiles, 0>(a, st);
  hipError_t e = launch_dca_attn_g<DT, D, 2, 1>(a, st);
  if (e != hipSuccess) return e;
  return launch_dca_attn_g<DT, D, kDcaTiles, 2>(a, st);
}

hipError_t launch_dca_attn(int dtype, int D, const DcaArgs& a, hipStream_t st) {
#define STA_DA(DT_, D_) if (dtype == DT_ && D == D_) return launch_dca_attn_t<DT_, D_>(a, st);
  STA_DA(DT_F32, 64) STA_DA(DT_F32, 128) STA_DA(DT_BF16, 64) STA_DA(DT_BF16, 128)
  STA_DA(DT_F16, 64) STA_DA(DT_F16, 128)
#undef STA_DA
  return hipErrorInvalidValue;
}

}  // namespace sta
