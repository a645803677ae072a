// sta_dca_dec.hip -- DCA (dual chunk attention) at decode, and the rotation of new keys into the
// KV cache.
//
// Reference: the decode branch of dca_forward (dca_kernel.py:491-522).  The cache holds keys
// already rotated at j mod L (:434-435); the new token's query at cur = M - 1 is rotated three
// ways (intra at cur mod L, succ at min(cur mod L + L, s), inter at min(2L - 1, s)) and scores
// the keys [0, inter_end) inter, [inter_end, chunk_start) succ and [chunk_start, M) intra, with
// chunk_start = floor(cur / L) L and inter_end = max(0, chunk_start - L).  The reference does
// this with model-dtype matmuls and one fp32 softmax:
//   s_j = rnd(rnd(q_var . k_j) * scale)     (matmul output and the scaled scores in the dtype)
//   p_j = rnd(exp(s_j - max s) / sum exp)   (softmax in fp32, cast back to the dtype)
//   out = rnd(sum_j p_j v_j)                (matmul output in the dtype)
// rnd = rounding to the model dtype (identity for fp32); dot products and sums accumulate in
// fp32.  These kernels keep every one of those roundings.
//
// Launches: dca_dec_qrot_kernel (the three query variants of every head), dca_dec_score_kernel
// (one workgroup = one kv head x 256 keys, one key per thread, all heads of the group; scores
// plus each block's max and sum of exp), dca_dec_pv_kernel (one workgroup = one head x 256
// keys: global max and sum from the block partials, weights, partial P.V), and
// dca_dec_combine_kernel (sum of the partials, rounded to the dtype).
#include "sta_dca_rot.h"
#include "sta_device.h"
#include "sta_kernels.h"

namespace sta {

constexpr int DCA_DEC_BK = 256;      // keys per score / P.V workgroup
constexpr int DCA_DEC_GMAX = 16;     // heads per kv head

template <int DT>
__device__ __forceinline__ void store8(void* p, int64_t i, const float* o) {
  if constexpr (DT == DT_F32) {
    float4* q = (float4*)((float*)p + i);
    q[0] = make_float4(o[0], o[1], o[2], o[3]);
    q[1] = make_float4(o[4], o[5], o[6], o[7]);
  } else if constexpr (DT == DT_F16) {
    *(u32x4*)((uint16_t*)p + i) = pack_f16x8(o);
  } else {
    *(u32x4*)((uint16_t*)p + i) = pack_bf16x8(o);
  }
}

// ------------------------------------------------------------------------------------------
// keys of the new tokens at positions pos0 .. pos0 + N - 1, rotated at (pos mod L) into out
// (dca_kernel.py:434-435 with the cyclic key table :187-190); one thread per 8 elements
// ------------------------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(256) void dca_rotate_keys_kernel(DcaRotArgs a) {
  constexpr int C = D / 8;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int64_t)a.heads * a.N * C) return;
  const int c = (int)(gid % C);
  const int64_t r = gid / C;
  const int row = (int)(r % a.N);
  const int head = (int)(r / a.N);
  const int d0 = c * 8;
  const bool first = d0 < D / 2;
  const int i0 = first ? d0 : d0 - D / 2;
  float x1[8], x2[8], o[8];
  const int64_t base = (int64_t)head * a.x_head_stride + (int64_t)row * a.x_tok_stride;
  load8<DT>(a.x, base + i0, x1);
  load8<DT>(a.x, base + D / 2 + i0, x2);
  dca_rot8<DT>(x1, x2, (int)(((int64_t)a.pos0 + row) % a.L), i0, first, a.inv_freq, a.mscale, o);
  store8<DT>(a.out, (int64_t)head * a.out_head_stride + (int64_t)row * a.out_tok_stride + d0, o);
}

// ------------------------------------------------------------------------------------------
// the query's three variants (dca_kernel.py:497-517): qrot (H, 3, D) fp32 holding dtype values
// ------------------------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(64) void dca_dec_qrot_kernel(DcaDecArgs a) {
  constexpr int C = D / 8;
  const int h = blockIdx.x;
  const int tid = threadIdx.x;
  if (tid >= 3 * C) return;
  const int var = tid / C;
  const int d0 = (tid % C) * 8;
  const int cur = a.M - 1;
  const int pid = cur % a.L;
  const int t = var == 0 ? pid : (var == 1 ? min(pid + a.L, a.chunk_size) : min(2 * a.L - 1, a.chunk_size));
  const bool first = d0 < D / 2;
  const int i0 = first ? d0 : d0 - D / 2;
  float x1[8], x2[8], o[8];
  const int64_t base = (int64_t)h * a.q_head_stride;
  load8<DT>(a.q, base + i0, x1);
  load8<DT>(a.q, base + D / 2 + i0, x2);
  dca_rot8<DT>(x1, x2, t, i0, first, a.inv_freq, a.mscale, o);
  float* dst = a.qrot + ((int64_t)h * 3 + var) * D + d0;
#pragma unroll
  for (int e = 0; e < 8; ++e) dst[e] = o[e];
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// ------------------------------------------------------------------------------------------
// scores of the keys [256 b, 256 b + 256) for every head of kv head g
// ------------------------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(DCA_DEC_BK) void dca_dec_score_kernel(DcaDecArgs a) {
#pragma clang fp contract(off)
  __shared__ float qs[DCA_DEC_GMAX * 3 * D];
  __shared__ float red[DCA_DEC_GMAX][DCA_DEC_BK / 64];
  const int g = blockIdx.x;
  const int blk = blockIdx.y;
  const int tid = threadIdx.x;
  const int G = a.H / a.Hkv;
  for (int i = tid; i < G * 3 * D; i += DCA_DEC_BK) qs[i] = a.qrot[(int64_t)g * G * 3 * D + i];
  __syncthreads();
  const int cur = a.M - 1;
  const int chunk_start = (cur / a.L) * a.L;
  const int inter_end = max(0, chunk_start - a.L);
  const int j = blk * DCA_DEC_BK + tid;
  const bool live = j < a.M;
  // the query variant this key is scored with (:513-517, cache order inter | succ | intra)
  const int var = j < inter_end ? 2 : (j < chunk_start ? 1 : 0);
  float acc[DCA_DEC_GMAX];
#pragma unroll
  for (int u = 0; u < DCA_DEC_GMAX; ++u) acc[u] = 0.0f;
  if (live) {
    const int64_t kb = (int64_t)g * a.k_head_stride + (int64_t)j * a.k_tok_stride;
    for (int d0 = 0; d0 < D; d0 += 8) {
      float kv[8];
      load8<DT>(a.k, kb + d0, kv);
#pragma unroll
      for (int u = 0; u < DCA_DEC_GMAX; ++u) {
        if (u < G) {
          const float* qq = qs + (u * 3 + var) * D + d0;
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[u] = acc[u] + qq[e] * kv[e];
        }
      }
    }
  }
  const int lane = tid & 63, wid = tid >> 6;
  float sv[DCA_DEC_GMAX];
#pragma unroll
  for (int u = 0; u < DCA_DEC_GMAX; ++u) {
    if (u < G) {
      sv[u] = live ? round_dt<DT>(opaque_f32(round_dt<DT>(acc[u]) * a.scale)) : -INFINITY;
      if (live) a.scores[(int64_t)(g * G + u) * a.M + j] = sv[u];
      const float m = wave_max(sv[u]);
      if (lane == 0) red[u][wid] = m;
    }
  }
  __syncthreads();
  float bmax[DCA_DEC_GMAX];
#pragma unroll
  for (int u = 0; u < DCA_DEC_GMAX; ++u) {
    if (u < G) {
      float m = red[u][0];
      for (int w = 1; w < DCA_DEC_BK / 64; ++w) m = fmaxf(m, red[u][w]);
      bmax[u] = m;
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < DCA_DEC_GMAX; ++u) {
    if (u < G) {
      const float e = live ? expf(sv[u] - bmax[u]) : 0.0f;
      const float s = wave_sum(e);
      if (lane == 0) red[u][wid] = s;
    }
  }
  __syncthreads();
  if (tid < G) {
    float s = 0.0f;
    for (int w = 0; w < DCA_DEC_BK / 64; ++w) s += red[tid][w];
    float m = bmax[0];
#pragma unroll
    for (int u = 0; u < DCA_DEC_GMAX; ++u)
      if (u == tid) m = bmax[u];
    const int64_t o = (int64_t)(g * G + tid) * a.nb + blk;
    a.pmax[o] = m;
    a.psum[o] = s;
  }
}

// ------------------------------------------------------------------------------------------
// softmax weights and partial P.V of head h over the keys [256 b, 256 b + 256)
// ------------------------------------------------------------------------------------------
template <int DT, int D>
__global__ __launch_bounds__(DCA_DEC_BK) void dca_dec_pv_kernel(DcaDecArgs a) {
#pragma clang fp contract(off)
  constexpr int KG = DCA_DEC_BK / D;      // key groups: 2 (D = 128) or 4 (D = 64)
  __shared__ float p[DCA_DEC_BK];
  __shared__ float red[DCA_DEC_BK / 64];
  __shared__ float accs[KG][D];
  const int h = blockIdx.x;
  const int blk = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wid = tid >> 6;
  const float* pm = a.pmax + (int64_t)h * a.nb;
  const float* ps = a.psum + (int64_t)h * a.nb;
  // the global max and the sum of exp(s - max) from the blocks' partials
  float m = -INFINITY;
  for (int b = tid; b < a.nb; b += DCA_DEC_BK) m = fmaxf(m, pm[b]);
  m = wave_max(m);
  if (lane == 0) red[wid] = m;
  __syncthreads();
  m = red[0];
  for (int w = 1; w < DCA_DEC_BK / 64; ++w) m = fmaxf(m, red[w]);
  __syncthreads();
  float l = 0.0f;
  for (int b = tid; b < a.nb; b += DCA_DEC_BK) l += ps[b] * expf(pm[b] - m);
  l = wave_sum(l);
  if (lane == 0) red[wid] = l;
  __syncthreads();
  l = 0.0f;
  for (int w = 0; w < DCA_DEC_BK / 64; ++w) l += red[w];
  // the weights, cast to the dtype as the reference's .to(q.dtype) does (:521)
  const int j = blk * DCA_DEC_BK + tid;
  p[tid] = j < a.M ? round_dt<DT>(opaque_f32(expf(a.scores[(int64_t)h * a.M + j] - m) / l)) : 0.0f;
  __syncthreads();
  const int kg = tid / D, d = tid % D;
  const int hk = h / (a.H / a.Hkv);
  const int n = min(DCA_DEC_BK, a.M - blk * DCA_DEC_BK);
  float acc = 0.0f;
  for (int jj = kg; jj < n; jj += KG) {
    const int64_t vi = (int64_t)hk * a.v_head_stride + (int64_t)(blk * DCA_DEC_BK + jj) * a.v_tok_stride + d;
    acc = acc + p[jj] * load_scalar<DT>(a.v, vi);
  }
  accs[kg][d] = acc;
  __syncthreads();
  if (tid < D) {
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < KG; ++u) s += accs[u][tid];
    a.part[((int64_t)h * a.nb + blk) * D + tid] = s;
  }
}

template <int DT, int D>
__global__ __launch_bounds__(D) void dca_dec_combine_kernel(DcaDecArgs a) {
#pragma clang fp contract(off)
  const int h = blockIdx.x;
  const int d = threadIdx.x;
  float s = 0.0f;
  for (int b = 0; b < a.nb; ++b) s += a.part[((int64_t)h * a.nb + b) * D + d];
  const int64_t oi = (int64_t)h * D + d;
  if constexpr (DT == DT_F32) ((float*)a.out)[oi] = s;
  else ((uint16_t*)a.out)[oi] = (uint16_t)(DT == DT_BF16 ? f32_to_bf16_bits(s) : f32_to_f16_bits(s));
}

// ------------------------------------------------------------------------------------------
// host launchers
// ------------------------------------------------------------------------------------------
template <int DT, int D>
static hipError_t launch_dca_rotate_keys_t(const DcaRotArgs& a, hipStream_t st) {
  const int64_t total = (int64_t)a.heads * a.N * (D / 8);
  hipLaunchKernelGGL((dca_rotate_keys_kernel<DT, D>), dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_dca_rotate_keys(int dtype, int D, const DcaRotArgs& a, hipStream_t st) {
#define STA_DK(DT_, D_) if (dtype == DT_ && D == D_) return launch_dca_rotate_keys_t<DT_, D_>(a, st);
  STA_DK(DT_F32, 64) STA_DK(DT_F32, 128) STA_DK(DT_BF16, 64) STA_DK(DT_BF16, 128)
  STA_DK(DT_F16, 64) STA_DK(DT_F16, 128)
#undef STA_DK
  return hipErrorInvalidValue;
}

int dca_dec_nblocks(int M) { return (M + DCA_DEC_BK - 1) / DCA_DEC_BK; }
int dca_dec_max_group() { return DCA_DEC_GMAX; }

template <int DT, int D>
static hipError_t launch_dca_decode_t(const DcaDecArgs& a, hipStream_t st) {
  hipLaunchKernelGGL((dca_dec_qrot_kernel<DT, D>), dim3(a.H), dim3(64), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((dca_dec_score_kernel<DT, D>), dim3(a.Hkv, a.nb), dim3(DCA_DEC_BK), 0, st, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((dca_dec_pv_kernel<DT, D>), dim3(a.H, a.nb), dim3(DCA_DEC_BK), 0, st, a);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((dca_dec_combine_kernel<DT, D>), dim3(a.H), dim3(D), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_dca_decode(int dtype, int D, const DcaDecArgs& a, hipStream_t st) {
#define STA_DD(DT_, D_) if (dtype == DT_ && D == D_) return launch_dca_decode_t<DT_, D_>(a, st);
  STA_DD(DT_F32, 64) STA_DD(DT_F32, 128) STA_DD(DT_BF16, 64) STA_DD(DT_BF16, 128)
  STA_DD(DT_F16, 64) STA_DD(DT_F16, 128)
#undef STA_DD
  return hipErrorInvalidValue;
}

}  // namespace sta
