// Row and element kernels of spark-gpt's bf16 SwiGLU MLP path (its default,
// non-FP8 path), around the three GEMMs of gemm.hip: _NormSwiGLU
// (train.py:2101-2131: RMSNorm folded into the gate/up weight) and
// _FusedSwiGLU (train.py:2067-2090: dense, or grouped over MoE experts).
//
// bf16 K-slab of a row-major X [R, C]: element (r, c) at byte
//   ((c / 32) * slab_rows(R) + r) * 64 + (c % 32) * 2,
// 32 elements of K per 64-byte slab row (the fp8 K-slab with 2-byte
// elements).  The GEMMs read the weights, the dgrad's d_gu operand and the
// weight gradient's token-contiguous copies in this form.
//
// Rows in padded order: with a MoE plan (common.h), padded row p of tile t
// holds expert-order row urow(t) + p % 256 while p % 256 < rows(t), else
// zeros; without one, row p for p < the row count, else zeros.
#include "common.h"

namespace sfp8 {

SFP8_DEV int64_t bslab(int64_t r, int64_t c, int64_t rpad) { return ((c >> 5) * rpad + r) * 64 + ((c & 31) << 1); }

// Source row of padded row p, or -1 (a zero row).
SFP8_DEV int64_t padded_source(const int* plan, int64_t p, int64_t nsrc) {
  if (!plan) return p < nsrc ? p : -1;
  const MoePlan P{plan};
  const int t = (int)(p >> 8), j = (int)(p & 255);
  if (t >= P.ntiles() || j >= P.rows(t)) return -1;
  const int64_t u = (int64_t)P.urow(t) + j;
  return u < nsrc ? u : -1;
}

SFP8_DEV void unpack8_bf16(const intx4& v, float (&x)[8]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    x[2 * q] = bf16_bits_to_f32((uint32_t)v[q] & 0xffffu);
    x[2 * q + 1] = bf16_bits_to_f32((uint32_t)v[q] >> 16);
  }
}

// 64 x 64 bf16 tiles transposed through LDS: element (row r, column j) at
// byte j * kTrStride + 2 r.  The 16 bytes a lane reads back (8 rows of one
// column) are 16-byte aligned, and a wave's writes of one column hit
// consecutive bytes.
constexpr int kTrStride = 144;

// Writes the 8 bf16 values of `o` (columns 8 c8 .. 8 c8 + 7 of tile row r)
// into the transposed tile.
SFP8_DEV void tr_put8(uint8_t* tile, int c8, int r, const uint32_t (&o)[4]) {
#pragma unroll
  for (int j = 0; j < 8; ++j)
    *reinterpret_cast<uint16_t*>(tile + (8 * c8 + j) * kTrStride + 2 * r) =
        (uint16_t)((j & 1) ? (o[j >> 1] >> 16) : (o[j >> 1] & 0xffffu));
}

// Writes transposed-tile column j, rows 32 hh .. 32 hh + 31 (16-byte chunk q)
// as the 64-byte slab row of K-slab row `row`, K piece (k0 / 32 + hh).
SFP8_DEV void tr_get16(const uint8_t* tile, int j, int hh, int q, uint8_t* out, int64_t k0, int64_t rpad,
                       int64_t row) {
  *reinterpret_cast<intx4*>(out + (((k0 >> 5) + hh) * rpad + row) * 64 + 16 * q) =
      *reinterpret_cast<const intx4*>(tile + j * kTrStride + 64 * hh + 16 * q);
}

// W [E][R][C] -> bf16 K-slab of each W[e] (ws, when given: [2C/64][slab_rows(R)][64],
// expert stride ws_estride bytes) and of W[e]^T (wt, when given:
// [2R/64][slab_rows(C)][64]).  Source fp32 (times nw[c] when nw is given:
// the RMSNorm weight folded into the gate/up weight, W' = bf16(W * w),
// train.py:2112) or bf16 (copied).  Padding rows are zero.  Work-group
// (rt, ct, e): rows 64 rt.., columns 64 ct..; the grid covers slab_rows(R)
// by slab_rows(C).  R % 64 == 0, C % 64 == 0.
__global__ __launch_bounds__(256) void bf16_weight_slabs_kernel(const void* __restrict__ w, int src_bf16,
                                                                const float* __restrict__ nw, int64_t R, int64_t C,
                                                                uint8_t* __restrict__ ws, uint8_t* __restrict__ wt,
                                                                int64_t ws_estride, int64_t wt_estride) {
  __shared__ __align__(16) uint8_t tile[64 * kTrStride];
  const int64_t e = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.x * 64, c0 = (int64_t)blockIdx.y * 64;
  const int64_t rp = slab_rows(R), cp = slab_rows(C);
  if (ws) ws += e * ws_estride;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int u = threadIdx.x + 256 * k;
    const int c8 = u & 7, r = u >> 3;
    const int64_t gr = r0 + r, gc = c0 + 8 * c8;
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (gr < R && gc < C) {
      if (src_bf16) {
        unpack8_bf16(*reinterpret_cast<const intx4*>(static_cast<const uint16_t*>(w) + (e * R + gr) * C + gc), x);
      } else {
        const float* p = static_cast<const float*>(w) + (e * R + gr) * C + gc;
        const floatx4 a = *reinterpret_cast<const floatx4*>(p), b = *reinterpret_cast<const floatx4*>(p + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[j] = a[j];
          x[4 + j] = b[j];
        }
        if (nw) {
          const floatx4 na = *reinterpret_cast<const floatx4*>(nw + gc);
          const floatx4 nb = *reinterpret_cast<const floatx4*>(nw + gc + 4);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            x[j] *= na[j];
            x[4 + j] *= nb[j];
          }
        }
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack2_bf16(x[2 * q], x[2 * q + 1]);
    if (ws && gc < C)  // gr < slab_rows(R): the grid's rows
      *reinterpret_cast<intx4*>(ws + bslab(gr, gc, rp)) = intx4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
    tr_put8(tile, c8, r, o);
  }
  if (!wt) return;  // work-group uniform
  wt += e * wt_estride;
  __syncthreads();
  // W^T rows c0 + j, K elements r0 .. r0 + 63: two 32-element slab pieces
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int v = threadIdx.x + 256 * k;
    const int q = v & 3, j = (v >> 2) & 63, hh = v >> 8;
    if (r0 + 32 * hh < R)  // R % 32 == 0: whole pieces
      tr_get16(tile, j, hh, q, wt, r0, cp, c0 + j);
  }
}

// x rows ([nsrc, D] bf16) in padded order -> xt (optional), the
// token-contiguous bf16 K-slab of x^T over the grid's 64 * gridDim.x padded
// rows ([2 ldp / 64][slab_rows(D)][64]: a weight gradient's plain B operand),
// and,
// when rstd is given (no plan), rstd[p] = 1 / sqrt(sum_d x[p, d]^2 / D + eps)
// for p < nsrc (the row scale of _swiglu_gemm_kernel's NORM mode,
// train.py:1689-1700; the sum of squares is exact, in fp64).  A work-group
// takes 64 padded rows, the columns in 64-wide chunks through an LDS
// transpose.  D % 64 == 0.
__global__ __launch_bounds__(256) void bf16_rows_prep_kernel(const uint16_t* __restrict__ x, int64_t nsrc, int64_t D,
                                                             const int* __restrict__ plan, float eps,
                                                             float* __restrict__ rstd, uint8_t* __restrict__ xt,
                                                             uint8_t* __restrict__ xs) {
  __shared__ __align__(16) uint8_t tile[64 * kTrStride];
  __shared__ int64_t rsrc[64];
  const int64_t p0 = (int64_t)blockIdx.x * 64;
  if (threadIdx.x < 64) rsrc[threadIdx.x] = padded_source(plan, p0 + threadIdx.x, nsrc);
  __syncthreads();
  const int64_t dp = slab_rows(D);
  double ss[2] = {0.0, 0.0};
  for (int64_t c0 = 0; c0 < D; c0 += 64) {
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int u = threadIdx.x + 256 * k;
      const int c8 = u & 7, r = u >> 3;
      const int64_t s = rsrc[r];
      intx4 v = {0, 0, 0, 0};
      if (s >= 0) v = *reinterpret_cast<const intx4*>(x + s * D + c0 + 8 * c8);
      // the row K-slab [2D/64][ldp][64]: columns c0 + 8 c8 .. are 16 bytes of
      // slab (c0 + 8 c8) / 32; eight lanes write two rows' 64-byte runs
      if (xs)
        *reinterpret_cast<intx4*>(xs + ((c0 >> 5) + (c8 >> 2)) * (int64_t)gridDim.x * 64 * 64 + (p0 + r) * 64 +
                                  16 * (c8 & 3)) = v;
      float f[8];
      unpack8_bf16(v, f);
#pragma unroll
      for (int j = 0; j < 8; ++j) ss[k] = __builtin_fma((double)f[j], (double)f[j], ss[k]);  // exact
      const uint32_t o[4] = {(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
      if (xt) tr_put8(tile, c8, r, o);
    }
    if (!xt) continue;  // work-group uniform
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int v = threadIdx.x + 256 * k;
      const int q = v & 3, j = (v >> 2) & 63, hh = v >> 8;
      tr_get16(tile, j, hh, q, xt, p0, dp, c0 + j);
    }
    __syncthreads();  // the next chunk overwrites the tile
  }
  if (!rstd) return;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    double t = ss[k];  // the 8 lanes of a row are consecutive
    t += __shfl_xor(t, 1, 64);
    t += __shfl_xor(t, 2, 64);
    t += __shfl_xor(t, 4, 64);
    const int u = threadIdx.x + 256 * k;
    const int64_t p = p0 + (u >> 3);
    if ((u & 7) == 0 && p < nsrc) {
      const float var = (float)t / (float)D + eps;
      rstd[p] = (float)(1.0 / __builtin_sqrt((double)var));
    }
  }
}

// SwiGLU backward of the rows (_swiglu_tiles, train.py:1900-1905, with the
// row scale of train.py:1965-1966): for padded row p with source row s and
// column i < I,
//   g = gu[s, i], u = gu[s, I + i], dh = dout[s, i] * rs  (rs = rstd[s], else 1),
//   sig = sigmoid(g),
//   d_gate = bf16(dh * u * (sig * (1 + g * (1 - sig)))),  d_up = bf16(dh * g * sig).
// G' = [d_gate | d_up] goes to gs, its bf16 K-slab over the grid's ldp padded
// rows ([4I/64][ldp][64]: the dgrad's A, and the weight gradient's through
// transposing reads), and optionally to gt, the token-contiguous K-slab of
// G'^T ([2 ldp / 64][slab_rows(2I)][64]: a weight gradient's plain A).
// Padding rows are zero.  Work-group (pb, ib): padded rows 64 pb..,
// columns 64 ib.. of each half.  I % 64 == 0.
__global__ __launch_bounds__(256) void bf16_swiglu_bwd_kernel(const uint16_t* __restrict__ gu,
                                                              const uint16_t* __restrict__ dout, int64_t nsrc,
                                                              int64_t I, const float* __restrict__ rstd,
                                                              const int* __restrict__ plan, uint8_t* __restrict__ gs,
                                                              uint8_t* __restrict__ gt) {
  __shared__ __align__(16) uint8_t tile[2][64 * kTrStride];
  __shared__ int64_t rsrc[64];
  const int64_t p0 = (int64_t)blockIdx.x * 64, ldp = (int64_t)gridDim.x * 64;
  const int64_t i0 = (int64_t)blockIdx.y * 64;
  if (threadIdx.x < 64) rsrc[threadIdx.x] = padded_source(plan, p0 + threadIdx.x, nsrc);
  __syncthreads();
  const float c_exp = -1.4426950408889634f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int u = threadIdx.x + 256 * k;
    const int c8 = u & 7, r = u >> 3;
    const int64_t s = rsrc[r], i = i0 + 8 * c8;
    intx4 gv = {0, 0, 0, 0}, uv = {0, 0, 0, 0}, dv = {0, 0, 0, 0};
    float rs = 1.0f;
    if (s >= 0) {
      gv = *reinterpret_cast<const intx4*>(gu + s * 2 * I + i);
      uv = *reinterpret_cast<const intx4*>(gu + s * 2 * I + I + i);
      dv = *reinterpret_cast<const intx4*>(dout + s * I + i);
      if (rstd) rs = rstd[s];
    }
    float g[8], uu[8], dh[8];
    unpack8_bf16(gv, g);
    unpack8_bf16(uv, uu);
    unpack8_bf16(dv, dh);
    uint32_t og[4], ou[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float dg2[2], du2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int j = 2 * q + h;
        const float d = dh[j] * rs;
        const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g[j] * c_exp));
        dg2[h] = d * uu[j] * (sig * (1.0f + g[j] * (1.0f - sig)));
        du2[h] = d * g[j] * sig;
      }
      og[q] = pack2_bf16(dg2[0], dg2[1]);
      ou[q] = pack2_bf16(du2[0], du2[1]);
    }
    *reinterpret_cast<intx4*>(gs + bslab(p0 + r, i, ldp)) = intx4{(int)og[0], (int)og[1], (int)og[2], (int)og[3]};
    *reinterpret_cast<intx4*>(gs + bslab(p0 + r, I + i, ldp)) = intx4{(int)ou[0], (int)ou[1], (int)ou[2], (int)ou[3]};
    if (gt) {
      tr_put8(tile[0], c8, r, og);
      tr_put8(tile[1], c8, r, ou);
    }
  }
  if (!gt) return;  // work-group uniform
  __syncthreads();
  const int64_t ip = slab_rows(2 * I);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int v = threadIdx.x + 256 * k;
    const int q = v & 3, j = (v >> 2) & 63, hh = (v >> 8) & 1, half = v >> 9;
    tr_get16(tile[half], j, hh, q, gt, p0, ip, half * I + i0 + j);
  }
}

// The RMSNorm backward of _NormSwiGLU (train.py:2125-2128) given p, the bf16
// dgrad output (rstd * d_gu @ W'): per row t,
//   coef = rstd[t] * rstd[t] * sum_d h[t, d] * p[t, d] / D,
//   dh[t] = bf16(p[t] - coef * h[t])   (fp32).
// One row per wave.  D % 8 == 0.
__global__ __launch_bounds__(256) void bf16_norm_dh_kernel(const uint16_t* __restrict__ p,
                                                           const uint16_t* __restrict__ h,
                                                           const float* __restrict__ rstd, int64_t T, int64_t D,
                                                           uint16_t* __restrict__ dh) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // wave uniform
  const uint16_t* pr = p + t * D;
  const uint16_t* hr = h + t * D;
  float s = 0.0f;
  for (int64_t d = 8 * lane; d < D; d += 512) {
    float pf[8], hf[8];
    unpack8_bf16(*reinterpret_cast<const intx4*>(pr + d), pf);
    unpack8_bf16(*reinterpret_cast<const intx4*>(hr + d), hf);
#pragma unroll
    for (int j = 0; j < 8; ++j) s += hf[j] * pf[j];
  }
  s = wave_sum_f32(s);
  const float r = rstd[t];
  const float coef = r * r * s / (float)D;
  for (int64_t d = 8 * lane; d < D; d += 512) {
    float pf[8], hf[8];
    unpack8_bf16(*reinterpret_cast<const intx4*>(pr + d), pf);
    unpack8_bf16(*reinterpret_cast<const intx4*>(hr + d), hf);
    uint32_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = pack2_bf16(pf[2 * q] - coef * hf[2 * q], pf[2 * q + 1] - coef * hf[2 * q + 1]);
    *reinterpret_cast<intx4*>(dh + t * D + d) = intx4{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
  }
}

// _NormSwiGLU's weight gradients from dwp, the bf16 gradient of the folded
// weight W' (train.py:2129-2131):
//   dw[m, n] = f32(dwp[m, n]) * nw[n]                         (fp32 [M, N])
//   part[b, n] = sum over the kFoldRows rows m of block b, ascending, of
//                f32(dwp[m, n]) * w[m, n]   (each product rounded first),
// then dnw[n] = the sum over b of part[b, n]: bf16_colsum_kernel sums
// groups of kColGroup consecutive b in order, then the groups in order.
// A thread takes 4 consecutive columns (N % 4 == 0).
constexpr int kFoldRows = 16;
constexpr int kColGroup = 16;

__global__ __launch_bounds__(256) void bf16_fold_grads_kernel(const uint16_t* __restrict__ dwp,
                                                              const float* __restrict__ w,
                                                              const float* __restrict__ nw, int64_t M, int64_t N,
                                                              float* __restrict__ dw, float* __restrict__ part) {
#pragma clang fp contract(off)
  const int64_t n = ((int64_t)blockIdx.y * 256 + threadIdx.x) * 4;
  const int64_t m0 = (int64_t)blockIdx.x * kFoldRows;
  if (n >= N) return;
  const floatx4 wn = *reinterpret_cast<const floatx4*>(nw + n);
  const int64_t m1 = m0 + kFoldRows < M ? m0 + kFoldRows : M;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int64_t m = m0; m < m1; ++m) {
    const intx2 gb = *reinterpret_cast<const intx2*>(dwp + m * N + n);
    const floatx4 g = {bf16_bits_to_f32((uint32_t)gb[0] & 0xffffu), bf16_bits_to_f32((uint32_t)gb[0] >> 16),
                       bf16_bits_to_f32((uint32_t)gb[1] & 0xffffu), bf16_bits_to_f32((uint32_t)gb[1] >> 16)};
    *reinterpret_cast<floatx4*>(dw + m * N + n) = g * wn;
    const floatx4 prod = g * *reinterpret_cast<const floatx4*>(w + m * N + n);
    acc += prod;
  }
  *reinterpret_cast<floatx4*>(part + blockIdx.x * N + n) = acc;
}

// out[j, n] = sum over b in [j * group, min((j + 1) * group, nb)) ascending of part[b, n].
__global__ __launch_bounds__(256) void bf16_colsum_kernel(const float* __restrict__ part, int64_t nb, int64_t N,
                                                          int group, float* __restrict__ out) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  const int64_t b0 = (int64_t)blockIdx.y * group;
  const int64_t b1 = b0 + group < nb ? b0 + group : nb;
  float acc = 0.0f;
  for (int64_t b = b0; b < b1; ++b) acc += part[b * N + n];
  out[blockIdx.y * N + n] = acc;
}

}  // namespace sfp8

// ============================================================================
// C ABI
// ============================================================================
using namespace sfp8;

namespace {
inline int bf_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}
inline bool bf_al16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }
inline unsigned bf_cdiv(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }
}  // namespace

extern "C" {

int64_t sfp8_bf16_slab_bytes(int64_t rows, int64_t cols) {
  if (rows < 0 || cols < 0 || cols % 32) return -1;
  return slab_rows(rows) * cols * 2;
}

int sfp8_bf16_weight_slabs(const void* w, int src_bf16, const float* nw, int64_t E, int64_t R, int64_t C, void* ws,
                           void* wt, void* stream) {
  if (!w || (!ws && !wt)) return kErrNullPointer;
  if (E <= 0 || R <= 0 || C <= 0 || R % 64 || C % 64 || (src_bf16 && nw)) return kErrBadShape;
  if (!bf_al16(w) || !bf_al16(nw) || !bf_al16(ws) || !bf_al16(wt)) return kErrBadAlignment;
  const int64_t rp = slab_rows(R), cp = slab_rows(C);
  hipLaunchKernelGGL(bf16_weight_slabs_kernel, dim3((unsigned)(rp / 64), (unsigned)(cp / 64), (unsigned)E), dim3(256),
                     0, (hipStream_t)stream, w, src_bf16, nw, R, C, (uint8_t*)ws, (uint8_t*)wt, 2 * C * rp, 2 * R * cp);
  return bf_status();
}

int sfp8_bf16_rows_prep(const void* x, int64_t nsrc, int64_t D, const int* plan, int64_t ldp, float eps, float* rstd,
                        void* xt, void* xs, void* stream) {
  if ((ldp > 0 && !xt && !rstd && !xs) || (nsrc > 0 && !x)) return kErrNullPointer;
  if (rstd && plan) return kErrBadShape;
  if (nsrc < 0 || D <= 0 || D % 64 || ldp < 0 || ldp % 256 || (!plan && ldp < nsrc)) return kErrBadShape;
  if (!bf_al16(x) || !bf_al16(xt) || !bf_al16(xs)) return kErrBadAlignment;
  if (ldp == 0) return kOk;
  hipLaunchKernelGGL(bf16_rows_prep_kernel, dim3((unsigned)(ldp / 64)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, nsrc, D, plan, eps, rstd, (uint8_t*)xt, (uint8_t*)xs);
  return bf_status();
}

int sfp8_bf16_swiglu_bwd(const void* gu, const void* dout, int64_t nsrc, int64_t I, const float* rstd,
                         const int* plan, int64_t ldp, void* gs, void* gt, void* stream) {
  if ((ldp > 0 && !gs) || (nsrc > 0 && (!gu || !dout))) return kErrNullPointer;
  if (nsrc < 0 || I <= 0 || I % 64 || ldp < 0 || ldp % 256 || (!plan && ldp < nsrc)) return kErrBadShape;
  if (!bf_al16(gu) || !bf_al16(dout) || !bf_al16(gs) || !bf_al16(gt)) return kErrBadAlignment;
  if (ldp == 0) return kOk;
  hipLaunchKernelGGL(bf16_swiglu_bwd_kernel, dim3((unsigned)(ldp / 64), (unsigned)(I / 64)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)gu, (const uint16_t*)dout, nsrc, I, rstd, plan,
                     (uint8_t*)gs, (uint8_t*)gt);
  return bf_status();
}

int sfp8_bf16_norm_dh(const void* p, const void* h, const float* rstd, int64_t T, int64_t D, void* dh, void* stream) {
  if (T > 0 && (!p || !h || !rstd || !dh)) return kErrNullPointer;
  if (T < 0 || D <= 0 || D % 8) return kErrBadShape;
  if (!bf_al16(p) || !bf_al16(h) || !bf_al16(dh)) return kErrBadAlignment;
  if (T == 0) return kOk;
  hipLaunchKernelGGL(bf16_norm_dh_kernel, dim3(bf_cdiv(T, 4)), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)p,
                     (const uint16_t*)h, rstd, T, D, (uint16_t*)dh);
  return bf_status();
}

int64_t sfp8_bf16_fold_partials(int64_t M, int64_t N) {
  if (M <= 0 || N <= 0) return -1;
  const int64_t nb = bf_cdiv(M, kFoldRows);
  return (nb + bf_cdiv(nb, kColGroup)) * N;  // block partials, then group sums
}

int sfp8_bf16_fold_grads(const void* dwp, const float* w, const float* nw, int64_t M, int64_t N, float* dw,
                         float* dnw, float* part, int64_t part_floats, void* stream) {
  if (!dwp || !w || !nw || !dw || !dnw || !part) return kErrNullPointer;
  if (M <= 0 || N <= 0 || N % 4) return kErrBadShape;
  if (!bf_al16(w) || !bf_al16(nw) || !bf_al16(dw) || !bf_al16(part) || (((uintptr_t)dwp) & 7u)) return kErrBadAlignment;
  if (part_floats < sfp8_bf16_fold_partials(M, N)) return kErrWorkspaceTooSmall;
  hipStream_t st = (hipStream_t)stream;
  const unsigned nb = bf_cdiv(M, kFoldRows);
  hipLaunchKernelGGL(bf16_fold_grads_kernel, dim3(nb, bf_cdiv(N, 1024)), dim3(256), 0, st, (const uint16_t*)dwp, w,
                     nw, M, N, dw, part);
  int rc = bf_status();
  if (rc) return rc;
  const unsigned ng = bf_cdiv(nb, kColGroup);
  float* grp = part + (int64_t)nb * N;
  hipLaunchKernelGGL(bf16_colsum_kernel, dim3(bf_cdiv(N, 256), ng), dim3(256), 0, st, part, (int64_t)nb, N,
                     kColGroup, grp);
  rc = bf_status();
  if (rc) return rc;
  hipLaunchKernelGGL(bf16_colsum_kernel, dim3(bf_cdiv(N, 256), 1), dim3(256), 0, st, grp, (int64_t)ng, N, (int)ng,
                     dnw);
  return bf_status();
}

}  // extern "C"
