// sta_gather.hip -- gather + repositioned attention over the selected keys (Kernel C).
//
// Reference: shared_selection_triton_exact_2.py:146-225 (_gather_attn_kernel).  Per (head,
// tile): rotate Q at newpos_q, then for 64-slot blocks gather the selected K and V rows, rotate
// K at newpos_k, mask causally on ORIGINAL positions (exact_2.py:210), run the -inf-safe online
// softmax (213-217) and accumulate P.V with P cast to the input dtype (220).  The reference
// always sweeps all k_max slots; slots past min(kept_size, k_max) are sentinels that contribute
// exactly nothing to the online softmax, so they are skipped.
//
// One workgroup per (head, tile); consumer wave w owns query rows 16w .. 16w+15.  Scores are computed
// transposed, S^T = K_rot . Q_rot^T (16x16x32 MFMA, lane <-> query row), so the P fragment the
// P.V product needs as its B operand is exactly the score accumulator the lane already holds:
//   O^T (dims x rows) += V^T (dims x slots) . P^T (slots x rows)
// with the contraction order over slots permuted identically in V^T and P^T.  V rows are stored
// row-major in LDS (16-byte writes) and read as the V^T operand by transposing LDS reads
// (ds_read_b64_tr_b16).  K rows arrive row-major (256 B per row at d128 bf16, 16-byte loads), are
// rotated in fp32 and stored to LDS as bf16.
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

template <int DT, int D, int NW>
struct GatherCfg {
  static constexpr int NC = NW * 64;           // consumer threads: wave w attends rows 16w..16w+15
  static constexpr int NP = 256;               // producer threads: gather, rotate, stage K / V
  static constexpr int NT = NC + NP;
  static constexpr int TPS = NP / 64;          // producer threads per slot for the K rotation
  static constexpr int FP = (D / 2) / TPS;     // frequencies per producer thread
  static constexpr int VUNITS = 16 * (D / 8);  // (4 slots x 8 dims) V units per block
  static constexpr int VU = (VUNITS + NP - 1) / NP;   // V units per producer thread
  static constexpr bool X3 = (DT == DT_F32);   // fp32 inputs: three-term bf16 products
  static constexpr int KSTR = D + 8;           // K LDS row stride (bf16 elements)
  // V rows are kept row-major in LDS; a row stride of D + 16 elements puts the 4 rows one
  // transposing read touches (32 bytes each) in distinct bank windows
  static constexpr int VRS = D + 16;
  static constexpr int KHALVES = X3 ? 2 : 1;
  static constexpr int KBUF = KHALVES * 64 * KSTR;     // elements of one K buffer
  static constexpr int VBUF = KHALVES * 64 * VRS;      // elements of one V buffer
  static constexpr size_t LDS_FIXED = (size_t)2 * (KBUF + VBUF) * 2;   // double-buffered
  // + the tile's kept positions (4 bytes per slot, rounded up to whole 64-slot blocks)
  static size_t lds_bytes(int k_max) { return LDS_FIXED + (size_t)((k_max + 63) / 64) * 64 * 4; }
};

// One workgroup per (head, tile), specialised waves.  Producer waves gather block b + 1's K and
// V rows (issued one block ahead of that), rotate K and write both to one half of a
// double-buffered LDS area while the consumer waves attend block b from the other half; one
// barrier per block hands the halves over.  A block then costs max(produce, consume).
// PQM: the per-query variant, whose slots carry a row mask (a.mask non-NULL)
template <int DT, int D, int NW, bool PQM>
__global__ __launch_bounds__(NW * 64 + 256, 1) void gather_kernel(GatherArgs a) {
  using Cfg = GatherCfg<DT, D, NW>;
  constexpr int NC = Cfg::NC, NT = Cfg::NT, TPS = Cfg::TPS, FP = Cfg::FP, VU = Cfg::VU;
  constexpr bool X3 = Cfg::X3;
  constexpr int KSTR = Cfg::KSTR, VRS = Cfg::VRS;
  constexpr int T = NW * 16;
  constexpr int KS = D / 32;                   // k steps of the score MFMA
  constexpr int DB = D / 16;                   // 16-dim blocks of the output
  extern __shared__ __align__(16) uint16_t sh[];
  // buffer p: K [64][KSTR] (hi, then lo when X3) followed by V [64][VRS] (hi, then lo)
  auto kbuf = [&](int p) { return sh + p * (Cfg::KBUF + Cfg::VBUF); };
  auto vbuf = [&](int p) { return sh + p * (Cfg::KBUF + Cfg::VBUF) + Cfg::KBUF; };
  int32_t* sidx = (int32_t*)(sh + Cfg::LDS_FIXED / 2);     // the tile's kept positions
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool consumer = tid < NC;
  int h, t;
  {
    const int bid = blockIdx.x;
    if ((a.H & 7) == 0) {   // XCD-aware: keep a head's tiles on one XCD (workgroup i -> XCD i % 8)
      const int hpx = a.H >> 3;
      const int r = bid >> 3;
      h = (bid & 7) * hpx + r % hpx;
      t = a.nt - 1 - r / hpx;
    } else {
      h = bid % a.H;
      t = a.nt - 1 - bid / a.H;
    }
  }
  const int kvh = h / (a.H / a.Hkv);
  const int N = a.N;
  const float rs = a.rope_scale;
  const float* invf = a.inv_freq;
  const int64_t tile_off = ((int64_t)h * a.nt + t) * a.k_max;
  const int nvalid = a.kept_size ? min(a.kept_size[h * a.nt + t], a.k_max) : a.k_max;
  const int nblk = (nvalid + 63) / 64;

  // ---- stage the tile's kept positions (sentinel N past the kept count) ----
  for (int s = tid; s < nblk * 64; s += NT) sidx[s] = s < nvalid ? a.idx[tile_off + s] : N;
  __syncthreads();

  if (!consumer) {
    // =================================== producers ===================================
    const int ptid = tid - NC;
    const int kslot = ptid / TPS, kpart = ptid % TPS;
    const int64_t kbase = (int64_t)kvh * a.k_head_stride;
    const int64_t vbase = (int64_t)kvh * a.v_head_stride;
    Raw8<DT> kx1[FP / 8], kx2[FP / 8], vx[VU][4];
    float np = 0.0f;
    float fr[FP];   // this thread's rotary frequencies
#pragma unroll
    for (int e = 0; e < FP; ++e) fr[e] = invf[kpart * FP + e];
    auto load_block = [&](int b) {
      const int j = sidx[b * 64 + kslot];
      if ((unsigned)j < (unsigned)N) {   // sentinel N (and any out-of-range index) -> zero row
        np = a.newpos_k[tile_off + b * 64 + kslot];
        const int64_t rb = kbase + (int64_t)j * a.k_tok_stride + kpart * FP;
#pragma unroll
        for (int c = 0; c < FP / 8; ++c) {
          kx1[c].load(a.k, rb + 8 * c);
          kx2[c].load(a.k, rb + D / 2 + 8 * c);
        }
      } else {
#pragma unroll
        for (int c = 0; c < FP / 8; ++c) { kx1[c].zero(); kx2[c].zero(); }
      }
#pragma unroll
      for (int vu = 0; vu < VU; ++vu) {
        const int u = ptid + vu * 256;
        const int sg = (u / (D / 8)) & 15, dc = u % (D / 8);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int jv = sidx[b * 64 + sg * 4 + k];
          if (u < Cfg::VUNITS && (unsigned)jv < (unsigned)N)
            vx[vu][k].load(a.v, vbase + (int64_t)jv * a.v_tok_stride + dc * 8);
          else
            vx[vu][k].zero();
        }
      }
    };
    // rotate K at newpos_k (exact_2.py:203-207); write K and V^T of block b to buffer b & 1.
    // SCALE: rope_scale != 1 (YaRN); otherwise the products with it are identities and skipped
    auto store_block = [&](auto scalec, int b) {
      constexpr bool SCALE = decltype(scalec)::value;
      uint16_t* kr_hi = kbuf(b & 1);
      uint16_t* kr_lo = kr_hi + 64 * KSTR;
      uint16_t* v_hi = vbuf(b & 1);
      uint16_t* v_lo = v_hi + 64 * VRS;
#pragma unroll
      for (int c = 0; c < FP / 8; ++c) {
        float x1[8], x2[8], o1[8], o2[8];
        kx1[c].to_f32(x1);
        kx2[c].to_f32(x2);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float sn, cs;
          fast_sincos(np * fr[8 * c + e], sn, cs);
          if constexpr (SCALE) {
            cs *= rs;
            sn *= rs;
          }
          o1[e] = x1[e] * cs - x2[e] * sn;
          o2[e] = x2[e] * cs + x1[e] * sn;
        }
        u32x4* d1 = (u32x4*)(kr_hi + kslot * KSTR + kpart * FP + 8 * c);
        u32x4* d2 = (u32x4*)(kr_hi + kslot * KSTR + D / 2 + kpart * FP + 8 * c);
        if constexpr (X3) {
          u32x4 h1, l1, h2, l2;
          split_bf16x8(o1, h1, l1);
          split_bf16x8(o2, h2, l2);
          *d1 = h1;
          *d2 = h2;
          *(u32x4*)(kr_lo + kslot * KSTR + kpart * FP + 8 * c) = l1;
          *(u32x4*)(kr_lo + kslot * KSTR + D / 2 + kpart * FP + 8 * c) = l2;
        } else {
          *d1 = pack_bf16x8(o1);
          *d2 = pack_bf16x8(o2);
        }
      }
#pragma unroll
      for (int vu = 0; vu < VU; ++vu) {
        const int u = ptid + vu * 256;
        if (u >= Cfg::VUNITS) continue;
        const int sg = u / (D / 8), dc = u % (D / 8);
#pragma unroll
        for (int k = 0; k < 4; ++k) {   // slot sg * 4 + k, dims dc * 8 .. dc * 8 + 7
          const int o = (sg * 4 + k) * VRS + dc * 8;
          if constexpr (!X3) {
            *(u32x4*)(v_hi + o) = vx[vu][k].w;
          } else {                      // fp32: bf16 hi and lo planes
            float vv[8];
            vx[vu][k].to_f32(vv);
            u32x4 hi, lo;
            split_bf16x8(vv, hi, lo);
            *(u32x4*)(v_hi + o) = hi;
            *(u32x4*)(v_lo + o) = lo;
          }
        }
      }
    };
    auto produce = [&](auto scalec) {
      if (nblk > 0) {
        load_block(0);
        store_block(scalec, 0);
        if (nblk > 1) load_block(1);
      }
      __syncthreads();
      for (int b = 0; b < nblk; ++b) {
        if (b + 1 < nblk) {
          store_block(scalec, b + 1);          // rows loaded one block earlier
          if (b + 2 < nblk) load_block(b + 2); // in flight during the next block
        }
        __syncthreads();
      }
    };
    if (rs == 1.0f) produce(std::false_type{});   // uniform: rope_scale is 1 except under YaRN
    else produce(std::true_type{});
    return;
  }

  // =================================== consumers ===================================
  // this lane's query row, rotated at newpos_q (exact_2.py:174-185)
  const int r = wave * 16 + (lane & 15);
  const int qrow = t * T + r;
  const bool row_ok = qrow < N;
  const int64_t qpos = (int64_t)a.q_pos_base + qrow;
  const int64_t qpos_first = (int64_t)a.q_pos_base + (int64_t)t * T;
  // kept positions are below N < 2^31: clamping the row's position keeps every comparison
  const int qpos32 = (int)(qpos < (int64_t)INT32_MAX ? qpos : (int64_t)INT32_MAX);
  // Q is rotated, then scaled by sm_scale * log2(e): scores come out in base-2 units and the
  // softmax uses exp2 (the scale commutes with the max and cancels in acc / l)
  const float qscale = a.sm_scale * 1.4426950408889634f;
  u32x4 qf_hi[KS], qf_lo[KS];
  {
    const float npq = a.newpos_q[((int64_t)h * a.nt + t) * T + r];
    const int64_t qb = (int64_t)h * a.q_head_stride + (int64_t)qrow * a.q_tok_stride;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = ks * 32 + 8 * (lane >> 4);
      float own[8], other[8], out[8];
      const bool first = d0 < D / 2;
      const int i0 = first ? d0 : d0 - D / 2;
      if (row_ok) {
        load8<DT>(a.q, qb + d0, own);
        load8<DT>(a.q, qb + (first ? d0 + D / 2 : d0 - D / 2), other);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) { own[e] = 0.0f; other[e] = 0.0f; }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float sn, cs;
        fast_sincos(npq * invf[i0 + e], sn, cs);
        cs *= rs;
        sn *= rs;
        out[e] = (first ? own[e] * cs - other[e] * sn : own[e] * cs + other[e] * sn) * qscale;
      }
      if constexpr (X3) split_bf16x8(out, qf_hi[ks], qf_lo[ks]);
      else qf_hi[ks] = pack_bf16x8(out);
    }
  }

  floatx4 oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) oacc[db] = floatx4{0.f, 0.f, 0.f, 0.f};
  float mR = -INFINITY, l_i = 0.0f;
  __syncthreads();   // block 0 is staged

  for (int b = 0; b < nblk; ++b) {
    const int s0 = b * 64;
    const uint16_t* kr_hi = kbuf(b & 1);
    const uint16_t* kr_lo = kr_hi + 64 * KSTR;
    const uint16_t* v_hi = vbuf(b & 1);
    const uint16_t* v_lo = v_hi + 64 * VRS;
    // ---- S^T = K_rot . Q_rot^T for 64 slots x this wave's 16 rows ----
    floatx4 sacc[4];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
      sacc[sb] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int off = (sb * 16 + (lane & 15)) * KSTR + ks * 32 + 8 * (lane >> 4);
        const u32x4 kh = *(const u32x4*)(kr_hi + off);
        if constexpr (X3) {
          const u32x4 kl = *(const u32x4*)(kr_lo + off);
          sacc[sb] = mfma16(kl, qf_hi[ks], sacc[sb]);
          sacc[sb] = mfma16(kh, qf_lo[ks], sacc[sb]);
        }
        sacc[sb] = mfma16(kh, qf_hi[ks], sacc[sb]);
      }
    }
    // ---- mask + online softmax (exact_2.py:209-217) ----
    // slots ascend and sentinels trail, so a block whose last slot is a real key before the
    // tile's first query needs no causal mask for any row
    const int jlast = sidx[s0 + 63];
    const bool unmasked = jlast < N && jlast <= qpos_first;
    float p[4][4];
    float bmax = -INFINITY;
    if (!PQM && unmasked) {   // uniform: every slot of the block is causal for every row
#pragma unroll
      for (int sb = 0; sb < 4; ++sb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[sb][i] = sacc[sb][i];
          bmax = fmaxf(bmax, p[sb][i]);
        }
    } else {
#pragma unroll
      for (int sb = 0; sb < 4; ++sb) {
        const int sl = s0 + sb * 16 + 4 * (lane >> 4);
        const int4 j4 = *(const int4*)(sidx + sl);
        const int jj[4] = {j4.x, j4.y, j4.z, j4.w};
        // per-query variant: bit r of the slot's mask says whether this lane's row attends it
        // (shared_selection_triton_perquery.py:296-297); slots past k_max read as empty
        uint32_t mk[4] = {~0u, ~0u, ~0u, ~0u};
        if constexpr (PQM) {
#pragma unroll
          for (int i = 0; i < 4; ++i) mk[i] = sl + i < a.k_max ? (uint32_t)a.mask[tile_off + sl + i] : 0u;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // exact_2.py:210, evaluated without short circuits (no per-slot branches)
          const bool causal = unmasked | (((unsigned)jj[i] < (unsigned)N) & (qpos32 >= jj[i]));
          const bool keep = causal & (!PQM || ((mk[i] >> (r & 31)) & 1u));
          const float v = keep ? sacc[sb][i] : -INFINITY;
          p[sb][i] = v;
          bmax = fmaxf(bmax, v);
        }
      }
    }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    // Online softmax with a lazily raised reference (exact_2.py:213-217 in exact arithmetic): the
    // reference mR only moves when a row's block max exceeds it by more than 2^8, so the rescale
    // of l and the accumulator is skipped for most blocks; exponents stay <= 8, which fp32 and the
    // bf16 P operand hold without loss of range.
    const bool raise = bmax > mR + 8.0f;
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {
      const float mnew = raise ? bmax : mR;
      const float alpha = raise ? __builtin_amdgcn_exp2f(mR - mnew) : 1.0f;   // 0 when mR = -inf
      l_i *= alpha;
#pragma unroll
      for (int db = 0; db < DB; ++db) oacc[db] *= alpha;
      mR = mnew;
    }
    const float msafe = (mR == -INFINITY) ? 0.0f : mR;
    float psum = 0.0f;
#pragma unroll
    for (int sb = 0; sb < 4; ++sb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[sb][i] = __builtin_amdgcn_exp2f(p[sb][i] - msafe);
        psum += p[sb][i];
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_i += psum;

    // ---- O^T += V^T . P^T (exact_2.py:218-220) ----
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int sb0 = 2 * k2, sb1 = 2 * k2 + 1;
      float pv[8] = {p[sb0][0], p[sb0][1], p[sb0][2], p[sb0][3], p[sb1][0], p[sb1][1], p[sb1][2], p[sb1][3]};
      u32x4 pb, pbl;
      if constexpr (DT == DT_F16) pb = pack_f16x8(pv);
      else if constexpr (X3) split_bf16x8(pv, pb, pbl);
      else pb = pack_bf16x8(pv);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        // V^T operand (dims db*16 + lane%16, slots {sb0, sb1}*16 + 4*(lane/16) + 0..3) by
        // transposing reads of row-major V: in each 16-lane group, lane L addresses slot
        // base + L/4, dims db*16 + 4*(L%4) .. +3, and receives dim db*16 + L of slots base .. base+3
        const int L = lane & 15;
        const int o0 = (sb0 * 16 + 4 * (lane >> 4) + (L >> 2)) * VRS + db * 16 + 4 * (L & 3);
        const int o1 = o0 + 16 * VRS;
        const u32x2 a0 = tr_read16x4(v_hi + o0);
        const u32x2 a1 = tr_read16x4(v_hi + o1);
        const u32x4 va = u32x4{a0[0], a0[1], a1[0], a1[1]};
        if constexpr (DT == DT_F16) {
          oacc[db] = mfma16_f16(va, pb, oacc[db]);
        } else if constexpr (X3) {
          const u32x2 b0 = tr_read16x4(v_lo + o0);
          const u32x2 b1 = tr_read16x4(v_lo + o1);
          const u32x4 vl = u32x4{b0[0], b0[1], b1[0], b1[1]};
          oacc[db] = mfma16(vl, pb, oacc[db]);
          oacc[db] = mfma16(va, pbl, oacc[db]);
          oacc[db] = mfma16(va, pb, oacc[db]);
        } else {
          oacc[db] = mfma16(va, pb, oacc[db]);
        }
      }
    }
    __syncthreads();   // hand this buffer back to the producers
  }

  // ---- out = acc / l (exact_2.py:223-225) ----
  if (row_ok) {
    const int64_t ob = ((int64_t)h * N + qrow) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int d0 = db * 16 + 4 * (lane >> 4);
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = oacc[db][i] / l_i;
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

template <int DT, int D, int NW, bool PQM>
static hipError_t launch_gather_m(const GatherArgs& a, hipStream_t st) {
  using Cfg = GatherCfg<DT, D, NW>;
  const size_t lds = Cfg::lds_bytes(a.k_max);
  hipError_t e = hipFuncSetAttribute((const void*)gather_kernel<DT, D, NW, PQM>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((gather_kernel<DT, D, NW, PQM>), dim3(a.H * a.nt), dim3(Cfg::NT), lds, st, a);
  return hipGetLastError();
}

// the per-query variant's row masks cover one 32-row tile (two consumer waves)
template <int DT, int D, int NW>
static hipError_t launch_gather_t(const GatherArgs& a, hipStream_t st) {
  if constexpr (NW == 2) {
    if (a.mask) return launch_gather_m<DT, D, NW, true>(a, st);
  } else {
    if (a.mask) return hipErrorInvalidValue;
  }
  return launch_gather_m<DT, D, NW, false>(a, st);
}

size_t gather_lds_bytes(int dtype, int D, int k_max) {
  const size_t halves = dtype == DT_F32 ? 2 : 1;
  const size_t fixed = 2 * halves * ((size_t)64 * (D + 8) * 2 + (size_t)64 * (D + 16) * 2);
  return fixed + (size_t)((k_max + 63) / 64) * 64 * 4;
}

hipError_t launch_gather(int dtype, int D, int tile, const GatherArgs& a, hipStream_t st) {
#define STA_G(DT_, D_, NW_) \
  if (dtype == DT_ && D == D_ && tile == NW_ * 16) return launch_gather_t<DT_, D_, NW_>(a, st);
  STA_G(DT_F32, 64, 2) STA_G(DT_F32, 64, 4) STA_G(DT_F32, 128, 2) STA_G(DT_F32, 128, 4)
  STA_G(DT_BF16, 64, 2) STA_G(DT_BF16, 64, 4) STA_G(DT_BF16, 128, 2) STA_G(DT_BF16, 128, 4)
  STA_G(DT_F16, 64, 2) STA_G(DT_F16, 64, 4) STA_G(DT_F16, 128, 2) STA_G(DT_F16, 128, 4)
#undef STA_G
  return hipErrorInvalidValue;
}

}  // namespace sta
