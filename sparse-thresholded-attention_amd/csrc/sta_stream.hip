// sta_stream.hip -- PQ Stream: per-query keep sets with streamed tile positions, attended in one
// sweep over aligned key blocks, newest first.
//
// Reference: pqstream_kernel.py:174-368 (_pqstream_kernel).  Per (head, 32-query tile), with
// P_top = min(last row, N-1) and key blocks of BN aligned keys visited from the tile's diagonal
// down to key 0:
//   keep(i, j) = (s_ij >= m_i - tau  or  j forced) and j <= qpos_i and row i < N      (:285-286)
//   adv = max_i #keep(i, block)   (or the slots the block occupies, advance="full")   (:303-306)
//   npk_j = -(d + hi_t - j),  npq_i = qpos_i - P_top,  base RoPE at those positions   (:270-332)
//   -inf-safe online softmax over the kept keys, P cast to the input dtype, d += adv  (:334-348)
// Blocks where no query keeps a key are skipped (adv == 0), leaving d unchanged.
//
// Fused sweep (the default): pass 1 of the score kernel leaves each query's keep threshold x0 on
// the raw dot; the sweep stages each block's selection-geometry K fragments beside K~ and V and
// computes the tile's selection scores itself -- S_a^T = K_a . Q_a^T as hi.lo + lo.hi + hi.hi
// bf16 MFMAs in the score kernel's order, so each keep bit equals the one the score kernel's
// pass 2 would write -- then keeps s >= x0 (causal, rows < N), so no keep-bit buffer exists.
// The unfused sweep reads those bits from the score kernel's pass 2 instead; it serves the
// configurations whose LDS the fused staging would overflow (fp32 inputs with block_n 64).
// The position rule is applied by rotation
// algebra instead of per-slot trigonometry: with K~_j = R(j) k_j (keys rotated once at their
// absolute positions by the pre-kernel below), R(npk_j) k_j = R(-w) K~_j for w = d + hi_t, so
//   q_att_i . R(npk_j) k_j = (R(w) q_att_i) . K~_j .
// Each block rotates the tile's 32 queries once (one sin/cos pair per frequency, shared by the
// wave) and runs plain MFMA products against K~; the reference evaluates 32 x D/2 sin/cos per
// block.  Angles are the fp32 products of the integer positions with inv_freq (w*f, j*f and
// npq*f, each rounded once), where the reference rounds (j - w)*f once: the difference is a few
// fp32 ulps of the angle.
//
// One workgroup = one head and G consecutive tiles (wave w owns tile g*G + w); each K~ / V block
// is staged once in LDS (double-buffered, V transposed) and read by all G waves.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

// ------------------------------------------------------------------------------------------
// K~: keys rotated at their absolute positions under the attend geometry (base RoPE, scale 1).
// Layout (Hkv, Npad, P, D) in 16-bit storage: bf16 for bf16 inputs, fp16 for fp16 inputs, and
// bf16 hi / lo planes (P = 2) for fp32 inputs.  Rows N .. Npad-1 are zero.
// ------------------------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(256) void abs_rope_kernel(const void* __restrict__ x, int64_t head_stride,
                                                       int64_t tok_stride, int heads, int N, int Npad,
                                                       const float* __restrict__ inv_freq,
                                                       uint16_t* __restrict__ out) {
#pragma clang fp contract(off)
  constexpr int C = D / 8;
  constexpr int P = DT == DT_F32 ? 2 : 1;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)heads * Npad * C) return;
  const int c = (int)(gid % C);
  const int64_t hr = gid / C;
  const int row = (int)(hr % Npad);
  const int head = (int)(hr / Npad);
  const int d0 = c * 8;
  float o[8];
  if (row < N) {
    const bool first = d0 < D / 2;
    const int i0 = first ? d0 : d0 - D / 2;
    float a[8], b[8];
    const int64_t base = (int64_t)head * head_stride + (int64_t)row * tok_stride;
    load8<DT>(x, base + i0, a);
    load8<DT>(x, base + D / 2 + i0, b);
    const float pf = (float)row;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ang = pf * inv_freq[i0 + e];
      float sn, cs;
      sincosf(ang, &sn, &cs);
      if (first) {
        const float p = a[e] * cs, q = b[e] * sn;
        o[e] = p - q;
      } else {
        const float p = b[e] * cs, q = a[e] * sn;
        o[e] = p + q;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0f;
  }
  uint16_t* dst = out + (((int64_t)head * Npad + row) * P) * D + d0;
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

// ------------------------------------------------------------------------------------------
// the stream kernel
// ------------------------------------------------------------------------------------------
template <int DT, int D, int BN, int G, bool FUSED = false>
struct StreamCfg {
  static constexpr bool X3 = DT == DT_F32;          // fp32 inputs: three-term bf16 products
  static constexpr int P = X3 ? 2 : 1;              // planes (hi, lo)
  static constexpr int NTH = G * 64;
  static constexpr int KSTR = D + 8;                // K~ LDS row stride (elements)
  using VL = VtLayout<BN, false>;   // V^T LDS layout (padded rows: measured faster than the
                                    // swizzled layout in this kernel)
  static constexpr int VSTR = VL::STR;               // V^T LDS row stride (elements)
  static constexpr int KBUF = P * BN * KSTR;        // elements of one K~ buffer
  static constexpr int VBUF = P * D * VSTR;         // elements of one V^T buffer
  static constexpr int KUNITS = P * BN * D / 8;     // 16-byte units of a K~ block
  static constexpr int KU = (KUNITS + NTH - 1) / NTH;
  static constexpr int VUNITS = (BN / 4) * (D / 8); // (4 keys x 8 dims) units of a V block
  static constexpr int VU = (VUNITS + NTH - 1) / NTH;
  static constexpr int S = D / 16;                  // k steps of a selection-geometry fragment
  static constexpr int KAUNITS = FUSED ? (BN / 32) * S * 2 * 64 : 0;   // 16-byte units of a K_a block
  static constexpr int KAU = FUSED ? (KAUNITS + NTH - 1) / NTH : 0;
  static constexpr size_t lds_bytes =
      (size_t)2 * (KBUF + VBUF) * 2 + (size_t)2 * KAUNITS * 16 + (size_t)G * (D / 2) * 8;
};

template <int DT, int D, int BN, int G, bool FUSED>
__global__ __launch_bounds__(G * 64, 1) void stream_kernel(StreamArgs a) {
#pragma clang fp contract(off)
  using Cfg = StreamCfg<DT, D, BN, G, FUSED>;
  constexpr bool X3 = Cfg::X3;
  constexpr int P = Cfg::P, NTH = Cfg::NTH, KSTR = Cfg::KSTR, VSTR = Cfg::VSTR;
  constexpr int KS = D / 16;          // k steps of the 32x32x16 score product
  constexpr int NSB = BN / 32;        // 32-key sub-blocks of a block
  constexpr int RBS = D / 32;         // 32-dim row blocks of the output
  constexpr int KU = Cfg::KU, VU = Cfg::VU;
  extern __shared__ __align__(16) uint16_t sm[];
  auto kbuf = [&](int p) { return sm + p * (Cfg::KBUF + Cfg::VBUF); };
  auto vbuf = [&](int p) { return sm + p * (Cfg::KBUF + Cfg::VBUF) + Cfg::KBUF; };
  u32x4* kabuf_all = (u32x4*)(sm + 2 * (Cfg::KBUF + Cfg::VBUF));      // 2 x KAUNITS (fused)
  auto kabuf = [&](int p) { return kabuf_all + p * Cfg::KAUNITS; };
  float* cstab_all = (float*)(kabuf_all + 2 * Cfg::KAUNITS);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hf = lane >> 5, q = lane & 31;
  const int ngroups = (a.nt + G - 1) / G;
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
  const int N = a.N;
  const int t = g * G + wave;
  const bool tile_ok = t < a.nt;
  const int P_top = min(t * 32 + 31, N - 1);                        // pqstream_kernel.py:203-204
  const int nblk = tile_ok ? (P_top + BN) / BN : 0;                 // :206
  const int t_last = min(g * G + G - 1, a.nt - 1);
  const int nb_wg = (min(t_last * 32 + 31, N - 1) + BN) / BN;
  const int row = t * 32 + q;                                       // this lane's query
  const bool row_ok = tile_ok && row < N;
  float* cstab = cstab_all + wave * (D / 2) * 2;
  const float* invf = a.inv_freq;

  // ---- the lane's query rotated at npq = qpos - P_top (:218-224), dims 16s + 8hf + e ----
  float qa[KS][8];
  {
    const float npq = (float)(row - P_top);
    const int64_t qb = (int64_t)h * a.q_head_stride + (int64_t)row * a.q_tok_stride;
#pragma unroll
    for (int s = 0; s < KS / 2; ++s) {
      const int d0 = s * 16 + 8 * hf;
      float x1[8], x2[8];
      if (row_ok) {
        load8<DT>(a.q, qb + d0, x1);
        load8<DT>(a.q, qb + d0 + D / 2, x2);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) { x1[e] = 0.0f; x2[e] = 0.0f; }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float sn, cs;
        fast_sincos(npq * invf[d0 + e], sn, cs);
        const float p1 = x1[e] * cs, p2 = x2[e] * sn;
        const float p3 = x2[e] * cs, p4 = x1[e] * sn;
        qa[s][e] = p1 - p2;
        qa[s + KS / 2][e] = p3 + p4;
      }
    }
  }

  // ---- fused: the tile's selection-geometry Q fragments (B operand: column = query, lane q)
  //      and the lane's query threshold x0 on the raw dot ----
  constexpr int S = Cfg::S;
  u32x4 qsel[FUSED ? S : 1][2];
  float x0q = INFINITY;
  if constexpr (FUSED) {
    const u32x4* qf = a.qfrag + ((int64_t)h * (a.q_rows_pad / 32) + (tile_ok ? t : 0)) * S * 128;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl) qsel[s][hl] = tile_ok ? qf[s * 128 + hl * 64 + lane] : u32x4{0u, 0u, 0u, 0u};
    if (tile_ok) x0q = a.xthr[(int64_t)h * a.q_rows_pad + row];
  }

  // ---- staging of K~ / V blocks into LDS (all threads) ----
  const uint16_t* kt = a.ktil + (int64_t)kvh * a.Npad * P * D;
  const int64_t vhb = (int64_t)kvh * a.v_head_stride;
  u32x4 kreg[KU];
  u32x4 kareg[FUSED ? Cfg::KAU : 1];
  Raw8<DT> vreg[VU][4];
  const u32x4* kaf = FUSED ? a.kfrag + (int64_t)kvh * (a.k_rows_pad / 32) * S * 128 : nullptr;
  auto load_block = [&](int b) {
    const uint16_t* src = kt + (int64_t)b * BN * P * D;   // rows b*BN .. +BN-1 are < Npad
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int e = tid + u * NTH;
      if (e < Cfg::KUNITS) kreg[u] = *(const u32x4*)(src + e * 8);
    }
    if constexpr (FUSED) {
      // the block's 32-key fragment blocks b*BN/32 .. are contiguous (rows < k_rows_pad)
      const u32x4* ksrc = kaf + (int64_t)b * (BN / 32) * S * 128;
#pragma unroll
      for (int u = 0; u < Cfg::KAU; ++u) {
        const int e = tid + u * NTH;
        if (e < Cfg::KAUNITS) kareg[u] = ksrc[e];
      }
    }
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int e = tid + u * NTH;
      const int sg = e / (D / 8), dc = e % (D / 8);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int j = b * BN + sg * 4 + k;
        if (e < Cfg::VUNITS && j < N) vreg[u][k].load(a.v, vhb + (int64_t)j * a.v_tok_stride + dc * 8);
        else vreg[u][k].zero();
      }
    }
  };
  auto store_block = [&](int p) {
    uint16_t* kd = kbuf(p);
    uint16_t* vd = vbuf(p);
    if constexpr (FUSED) {
      u32x4* kad = kabuf(p);
#pragma unroll
      for (int u = 0; u < Cfg::KAU; ++u) {
        const int e = tid + u * NTH;
        if (e < Cfg::KAUNITS) kad[e] = kareg[u];
      }
    }
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

  // ---- the tile's keep bits of one block: lane l < BN holds key start + l ----
  const uint32_t* brow = FUSED ? nullptr : a.bits + ((int64_t)h * a.nt + (tile_ok ? t : 0)) * a.bits_stride;
  const int64_t loc_lo = (int64_t)t * 32 - a.n_local + 1, loc_hi = (int64_t)t * 32 + 31;   // :260-261
  const int rows_hi = min(32, N - t * 32);                        // rows < N
  auto load_bits = [&](int b) -> uint32_t {
    if constexpr (FUSED) return 0u;
    const int j = b * BN + lane;
    return (tile_ok && lane < BN && b >= 0 && j <= P_top) ? brow[j] : 0u;
  };

  floatx16 oacc[RBS];
#pragma unroll
  for (int rb = 0; rb < RBS; ++rb) oacc[rb] = floatx16{};
  float mR = -INFINITY, l_i = 0.0f;   // running max of the raw dots, running sum
  const float c2 = a.sm_scale * 1.44269504088896341f;
  float d = 0.0f;                 // running base (:252)
  int kept_q = 0, n_used = 0;

  if (nb_wg > 0) {
    load_block(nb_wg - 1);
    store_block(0);
  }
  uint32_t bits_cur = load_bits(nb_wg - 1);
  __syncthreads();

  for (int it = 0; it < nb_wg; ++it) {
    const int b = nb_wg - 1 - it;                                 // descending (:266)
    const int p = it & 1;
    const bool more = it + 1 < nb_wg;
    if (more) load_block(b - 1);
    const uint32_t bits_next = load_bits(b - 1);
    if (tile_ok && b < nblk) {
      const int start = b * BN;
      const int hi_t = min(P_top, start + BN - 1);                  // :271
      // this lane's mask bits: query q, keys 32 sb + (i/4)*8 + 4 hf + i%4
      uint32_t mbits[NSB];
      int cnt = 0;
      if constexpr (FUSED) {
        // S_a^T = K_a . Q_a^T (key rows, query columns), hi.lo terms first as in the score
        // kernel's pass 2; keep = s >= x0 (rows < N through x0 = +inf), causal, or forced (:285-286)
        const u32x4* ka = kabuf(p);
        floatx16 sel[NSB];
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) sel[sb] = floatx16{};
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
          for (int sb = 0; sb < NSB; ++sb) {
            const u32x4 kh = ka[(sb * S + s) * 128 + lane];
            const u32x4 kl = ka[(sb * S + s) * 128 + 64 + lane];
            sel[sb] = mfma32(kh, qsel[s][1], sel[sb]);
            sel[sb] = mfma32(kl, qsel[s][0], sel[sb]);
            sel[sb] = mfma32(kh, qsel[s][0], sel[sb]);
          }
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) {
          uint32_t tb = 0, fb = 0;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int j = start + sb * 32 + (i >> 2) * 8 + 4 * hf + (i & 3);
            const bool causal = row_ok && j <= row;
            const bool forced = j < a.n_global || (j >= loc_lo && j <= loc_hi);   // :284
            tb |= (uint32_t)(causal && sel[sb][i] >= x0q) << i;
            fb |= (uint32_t)(causal && forced) << i;
          }
          mbits[sb] = tb | fb;
          cnt += __popc(mbits[sb]);
          if (a.bits_out) {
            // the threshold bits as the score kernel lays them out: one word per key, bit = row
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const uint64_t w = __ballot((tb >> i) & 1u);
              const int j = start + sb * 32 + (i >> 2) * 8 + (i & 3);
              uint32_t* bo = a.bits_out + ((int64_t)h * a.nt + t) * a.bits_stride;
              if (lane == 0 && j <= P_top) bo[j] = (uint32_t)w;
              if (lane == 0 && j + 4 <= P_top) bo[j + 4] = (uint32_t)(w >> 32);
            }
          }
        }
      } else {
        // keep word of key start + lane: threshold bits, or every causal row when forced
        uint32_t kw = 0;
        {
          const int j = start + lane;
          if (lane < BN && j <= P_top) {
            kw = bits_cur;
            const bool forced = j < a.n_global || (j >= loc_lo && j <= loc_hi);   // :284
            if (forced) {
              const int lo_r = max(0, j - t * 32);                  // causal: qpos_i >= j
              const uint32_t hi_mask = rows_hi >= 32 ? 0xffffffffu : ((1u << rows_hi) - 1u);
              kw |= hi_mask & ~((1u << lo_r) - 1u);
            }
          }
        }
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) {
          mbits[sb] = 0;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = sb * 32 + (i >> 2) * 8 + 4 * hf + (i & 3);
            const uint32_t w = (uint32_t)__shfl((int)kw, key, 64);
            mbits[sb] |= ((w >> q) & 1u) << i;
          }
          cnt += __popc(mbits[sb]);
        }
      }
      const int c_q = cnt + __shfl_xor(cnt, 32, 64);               // keys of query q (:288)
      int adv_i;
      if (a.adv_full) {
        adv_i = hi_t - start + 1;                                  // :303-304
      } else {
        int m = c_q;                                               // :305-306
        m = max(m, __shfl_xor(m, 1, 64));
        m = max(m, __shfl_xor(m, 2, 64));
        m = max(m, __shfl_xor(m, 4, 64));
        m = max(m, __shfl_xor(m, 8, 64));
        m = max(m, __shfl_xor(m, 16, 64));
        adv_i = m;
      }
      if (!(a.use_skip && adv_i <= 0)) {                            // :319-322
        // ---- rotate the tile's queries by w = d + hi_t (one sin/cos per frequency) ----
        const float wpos = d + (float)hi_t;
        if (lane < D / 2) {
          float sn, cs;
          fast_sincos(wpos * invf[lane], sn, cs);
          cstab[2 * lane] = cs;
          cstab[2 * lane + 1] = sn;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // ---- S^T = K~ . Q_w^T, 32 keys x 32 queries per sub-block; the rotated query is packed
        //      one k-step pair (dims d, d + D/2) at a time, right before its products ----
        const uint16_t* kr = kbuf(p);
        floatx16 sacc[NSB];
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb) sacc[sb] = floatx16{};
#pragma unroll
        for (int s = 0; s < KS / 2; ++s) {
          float y1[8], y2[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int f = s * 16 + 8 * hf + e;
            const float cs = cstab[2 * f], sn = cstab[2 * f + 1];
            if constexpr (X3) {   // fp32 inputs: every product rounded, as the reference rotates
              const float p1 = qa[s][e] * cs, p2 = qa[s + KS / 2][e] * sn;
              const float p3 = qa[s + KS / 2][e] * cs, p4 = qa[s][e] * sn;
              y1[e] = p1 - p2;
              y2[e] = p3 + p4;
            } else {              // 16-bit operands: one product and one FMA per coordinate, the
                                  // result rounded to the operand type right after
              y1[e] = fmaf(qa[s][e], cs, -(qa[s + KS / 2][e] * sn));
              y2[e] = fmaf(qa[s + KS / 2][e], cs, qa[s][e] * sn);
            }
          }
          u32x4 qh[2], ql[2];
          if constexpr (X3) {
            split_bf16x8(y1, qh[0], ql[0]);
            split_bf16x8(y2, qh[1], ql[1]);
          } else if constexpr (DT == DT_F16) {
            qh[0] = pack_f16x8(y1);
            qh[1] = pack_f16x8(y2);
          } else {
            qh[0] = pack_bf16x8(y1);
            qh[1] = pack_bf16x8(y2);
          }
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int ks = s + half * (KS / 2);
#pragma unroll
            for (int sb = 0; sb < NSB; ++sb) {
              const int off = (sb * 32 + q) * KSTR + ks * 16 + 8 * hf;
              const u32x4 kh = *(const u32x4*)(kr + off);
              if constexpr (X3) {
                const u32x4 kl = *(const u32x4*)(kr + BN * KSTR + off);
                sacc[sb] = mfma32(kl, qh[half], sacc[sb]);
                sacc[sb] = mfma32(kh, ql[half], sacc[sb]);
                sacc[sb] = mfma32(kh, qh[half], sacc[sb]);
              } else if constexpr (DT == DT_F16) {
                sacc[sb] = mfma32_f16(kh, qh[half], sacc[sb]);
              } else {
                sacc[sb] = mfma32(kh, qh[half], sacc[sb]);
              }
            }
          }
        }
        // ---- mask + online softmax (:334-344).  The running max stays on the raw dots (the
        //      scale is positive, so they order as the scaled scores) and each weight is
        //      exp2(raw * c2 - max * c2) with c2 = scale * log2(e): one FMA and one exp per score ----
        float bmax = -INFINITY;
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float v = ((mbits[sb] >> i) & 1u) ? sacc[sb][i] : -INFINITY;
            sacc[sb][i] = v;
            bmax = fmaxf(bmax, v);
          }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
        const float mnew = fmaxf(mR, bmax);
        const float msafe = (mnew == -INFINITY) ? 0.0f : mnew;
        const float alpha = __builtin_amdgcn_exp2f((mR - msafe) * c2);
        const float moff = -msafe * c2;
        float psum = 0.0f;
#pragma unroll
        for (int sb = 0; sb < NSB; ++sb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float pv = __builtin_amdgcn_exp2f(fmaf(sacc[sb][i], c2, moff));
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
        // ---- O^T += V^T . P^T (:345), contraction over keys in the score-slot order ----
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
        kept_q += c_q;                                            // :347
        d = d + (float)adv_i;                                     // :348
        n_used += 1;
      }
    }
    bits_cur = bits_next;
    if (more) store_block(p ^ 1);
    __syncthreads();
  }

  // ---- out = acc / l (:360-362) and the per-tile diagnostics (:363-366) ----
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
    if (hf == 0) a.kept[(int64_t)h * N + row] = kept_q;
  }
  if (tile_ok && lane == 0) {
    const int64_t o = (int64_t)h * a.nt + t;
    a.span[o] = d;
    a.blocks[o] = (float)nblk;
    a.skipped[o] = (float)(nblk - n_used);
  }
}

// ------------------------------------------------------------------------------------------
// host launchers
// ------------------------------------------------------------------------------------------
template <int DT, int D>
static hipError_t launch_abs_rope_t(const void* x, int64_t hs, int64_t ts, int heads, int N, int Npad,
                                    const float* inv_freq, uint16_t* out, hipStream_t st) {
  const int64_t total = (int64_t)heads * Npad * (D / 8);
  hipLaunchKernelGGL((abs_rope_kernel<DT, D>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, hs,
                     ts, heads, N, Npad, inv_freq, out);
  return hipGetLastError();
}

hipError_t launch_abs_rope(int dtype, int D, const void* x, int64_t hs, int64_t ts, int heads, int N, int Npad,
                           const float* inv_freq, uint16_t* out, hipStream_t st) {
#define STA_AR(DT_, D_) \
  if (dtype == DT_ && D == D_) return launch_abs_rope_t<DT_, D_>(x, hs, ts, heads, N, Npad, inv_freq, out, st);
  STA_AR(DT_F32, 64) STA_AR(DT_F32, 128) STA_AR(DT_BF16, 64) STA_AR(DT_BF16, 128)
  STA_AR(DT_F16, 64) STA_AR(DT_F16, 128)
#undef STA_AR
  return hipErrorInvalidValue;
}

constexpr int kStreamTiles = 8;        // tiles (waves) per workgroup, unfused sweep
constexpr int kStreamTilesFused = 4;   // fused sweep: one wave per SIMD, the register room the
                                       // selection fragments need

// the fused sweep exists where its staging fits the LDS (everything but fp32 inputs with block_n 64)
template <int DT, int D, int BN>
constexpr bool stream_fused() { return StreamCfg<DT, D, BN, kStreamTilesFused, true>::lds_bytes <= 160 * 1024; }

bool stream_can_fuse(int dtype, int D, int BN) {
#define STA_SF(DT_, D_, BN_) if (dtype == DT_ && D == D_ && BN == BN_) return stream_fused<DT_, D_, BN_>();
  STA_SF(DT_F32, 64, 32) STA_SF(DT_F32, 64, 64) STA_SF(DT_F32, 128, 32) STA_SF(DT_F32, 128, 64)
  STA_SF(DT_BF16, 64, 32) STA_SF(DT_BF16, 64, 64) STA_SF(DT_BF16, 128, 32) STA_SF(DT_BF16, 128, 64)
  STA_SF(DT_F16, 64, 32) STA_SF(DT_F16, 64, 64) STA_SF(DT_F16, 128, 32) STA_SF(DT_F16, 128, 64)
#undef STA_SF
  return false;
}

template <int DT, int D, int BN>
constexpr size_t stream_lds_t(bool fused) {
  if constexpr (stream_fused<DT, D, BN>()) {
    if (fused) return StreamCfg<DT, D, BN, kStreamTilesFused, true>::lds_bytes;
  }
  return StreamCfg<DT, D, BN, kStreamTiles, false>::lds_bytes;
}

size_t stream_lds_bytes(int dtype, int D, int BN, bool fused) {
#define STA_SL(DT_, D_, BN_) if (dtype == DT_ && D == D_ && BN == BN_) return stream_lds_t<DT_, D_, BN_>(fused);
  STA_SL(DT_F32, 64, 32) STA_SL(DT_F32, 64, 64) STA_SL(DT_F32, 128, 32) STA_SL(DT_F32, 128, 64)
  STA_SL(DT_BF16, 64, 32) STA_SL(DT_BF16, 64, 64) STA_SL(DT_BF16, 128, 32) STA_SL(DT_BF16, 128, 64)
  STA_SL(DT_F16, 64, 32) STA_SL(DT_F16, 64, 64) STA_SL(DT_F16, 128, 32) STA_SL(DT_F16, 128, 64)
#undef STA_SL
  return 0;
}

template <int DT, int D, int BN, int G, bool FUSED>
static hipError_t launch_stream_g(const StreamArgs& a, hipStream_t st) {
  using Cfg = StreamCfg<DT, D, BN, G, FUSED>;
  hipError_t e = hipFuncSetAttribute((const void*)stream_kernel<DT, D, BN, G, FUSED>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)Cfg::lds_bytes);
  if (e != hipSuccess) return e;
  const int ngroups = (a.nt + G - 1) / G;
  hipLaunchKernelGGL((stream_kernel<DT, D, BN, G, FUSED>), dim3(a.H * ngroups), dim3(Cfg::NTH), Cfg::lds_bytes,
                     st, a);
  return hipGetLastError();
}

template <int DT, int D, int BN>
static hipError_t launch_stream_t(const StreamArgs& a, hipStream_t st) {
  if constexpr (stream_fused<DT, D, BN>()) {
    if (a.qfrag) return launch_stream_g<DT, D, BN, kStreamTilesFused, true>(a, st);
  }
  if (!a.bits) return hipErrorInvalidValue;
  return launch_stream_g<DT, D, BN, kStreamTiles, false>(a, st);
}

hipError_t launch_stream(int dtype, int D, int BN, const StreamArgs& a, hipStream_t st) {
#define STA_ST(DT_, D_, BN_) \
  if (dtype == DT_ && D == D_ && BN == BN_) return launch_stream_t<DT_, D_, BN_>(a, st);
  STA_ST(DT_F32, 64, 32) STA_ST(DT_F32, 64, 64) STA_ST(DT_F32, 128, 32) STA_ST(DT_F32, 128, 64)
  STA_ST(DT_BF16, 64, 32) STA_ST(DT_BF16, 64, 64) STA_ST(DT_BF16, 128, 32) STA_ST(DT_BF16, 128, 64)
  STA_ST(DT_F16, 64, 32) STA_ST(DT_F16, 64, 64) STA_ST(DT_F16, 128, 32) STA_ST(DT_F16, 128, 64)
#undef STA_ST
  return hipErrorInvalidValue;
}

}  // namespace sta
