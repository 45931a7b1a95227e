// Grouped (MoE expert) kernels of the FP8 MLP path that are not GEMMs
// (gfx950): the padded-expert-order plan, the gathered row quantizer and
// the top-k row sum.  The grouped GEMMs are in gemm.hip and read the plan.
//
// spark-gpt routes each token to top_k experts; the (token, expert) pairs
// sorted by expert are R "expert-order rows", expert e owning rows
// offsets[e-1] .. offsets[e] - 1 (offsets: inclusive prefix sums of the
// per-expert counts, train.py:2273-2290).  Here every expert's rows are
// laid out from a 256-row boundary ("padded expert order", common.h), so a
// GEMM tile never straddles two experts and the weight gradients reduce
// over whole 64-token stages of one expert; padding rows hold zeros.
#include "common.h"

namespace sfp8 {

constexpr int kMaxExperts = 1024;

// One work-group: thread 0 walks the experts (prefix sums of their tile
// counts); then every thread fills tiles t, t + 256, ... of the table, the
// expert of tile t found by binary search.  Counts are clamped so that no
// tile reaches past row R (offsets inconsistent with R only lose rows).
__global__ __launch_bounds__(256) void moe_plan_kernel(const int* __restrict__ offsets, int E, int64_t R,
                                                       int max_tiles, int* __restrict__ plan) {
  __shared__ int tstart[kMaxExperts + 1];
  __shared__ int ustart[kMaxExperts + 1];
  if (threadIdx.x == 0) {
    int prev = 0, tiles = 0;
    for (int e = 0; e < E; ++e) {
      int end = offsets[e];
      end = end < prev ? prev : (end > (int)R ? (int)R : end);
      int nt = (end - prev + 255) / 256;
      if (tiles + nt > max_tiles) nt = max_tiles - tiles;
      plan[kPlanHdr + e] = 256 * tiles;
      plan[kPlanHdr + E + e] = 256 * nt;
      tstart[e] = tiles;
      ustart[e] = prev;
      tiles += nt;
      prev = end;
    }
    tstart[E] = tiles;
    ustart[E] = prev;
    plan[0] = tiles;
    plan[1] = E;
  }
  __syncthreads();
  const int nt = tstart[E];
  for (int t = threadIdx.x; t < nt; t += 256) {
    int lo = 0, hi = E - 1;  // the largest e with tstart[e] <= t owns tile t
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tstart[mid] <= t) lo = mid;
      else hi = mid - 1;
    }
    const int j = t - tstart[lo];
    const int u0 = ustart[lo] + 256 * j;
    const int left = ustart[lo + 1] - u0;
    int* ent = plan + kPlanHdr + 2 * E + 3 * t;
    ent[0] = lo;
    ent[1] = u0;
    ent[2] = left < 256 ? left : 256;
  }
}

// Gathered rows -> fp8 in padded expert order.  Padded row p of tile
// t = p / 256 takes source row map[urow(t) + j] (token gather; map == null:
// urow(t) + j) for j = p % 256 < rows(t), else zeros.  Writes
//   q = fmt(clamp(src * scale[sslot]))  as the K-slab of [ldp, D] (xs: the
//   gate/up GEMM's A operand, and a weight gradient's through transposing
//   reads) and/or as the token-contiguous K-slab of [D, ldp] (xt: a weight
//   gradient's plain operand),
//   amax[aslot] = max |src| over the gathered rows.
// A work-group takes 64 padded rows; columns go in chunks of up to 512 (the
// last one ragged), staged in a 17 KiB LDS tile (eight work-groups per CU)
// and written transposed as whole 64-byte rows.  Within a chunk, 16-byte
// source unit f is (slab f >> 9, row (f >> 3) & 63, 8 columns 8 * (f & 7)):
// a wave reads 128-byte runs of 8 rows and writes 512 contiguous bytes of
// one xs slab; each thread keeps kRqBatch loads in flight.
constexpr int kRqRows = 64;
constexpr int kRqChunk = 256;
constexpr int kRqBatch = 4;

template <int FMT>
__global__ __launch_bounds__(256) void moe_rows_quant_kernel(
    const uint16_t* __restrict__ src, int64_t nsrc, int64_t D, const int64_t* __restrict__ map, int64_t nmap,
    const int* __restrict__ plan, const float* __restrict__ scale, int sslot, float* __restrict__ amax, int aslot,
    uint8_t* __restrict__ xs, uint8_t* __restrict__ xt, int64_t ldp) {
  extern __shared__ __align__(16) uint8_t tile[];
  __shared__ float red[4];
  __shared__ int64_t rsrc[kRqRows];
  const MoePlan P{plan};
  const int64_t p0 = (int64_t)blockIdx.x * kRqRows;
  if (threadIdx.x < kRqRows) {
    // source row of padded row p0 + threadIdx.x, or -1 (zeros)
    const int64_t p = p0 + threadIdx.x;
    const int t = (int)(p >> 8), j = (int)(p & 255);
    int64_t r = -1;
    if (t < P.ntiles() && j < P.rows(t)) {
      const int64_t u = (int64_t)P.urow(t) + j;
      if (map) r = u < nmap ? map[u] : -1;
      else r = u;
      if (r < 0 || r >= nsrc) r = -1;
    }
    rsrc[threadIdx.x] = r;
  }
  __syncthreads();
  const float s = scale[sslot];
  const int stride = (int)(D < kRqChunk ? D : kRqChunk) + 16;  // conflict-free transposing reads
  const int64_t cp = slab_rows(D);
  float m = 0.0f;
  for (int64_t cc = 0; cc < D; cc += kRqChunk) {
    const int C = (int)(D - cc < kRqChunk ? D - cc : kRqChunk);
    const int units = kRqRows * (C / 8);
    for (int f0 = threadIdx.x; f0 < units; f0 += kRqBatch * 256) {
      intx4 v[kRqBatch];
#pragma unroll
      for (int i = 0; i < kRqBatch; ++i) {
        const int f = f0 + 256 * i;
        const int64_t sr = rsrc[(f >> 3) & 63];
        v[i] = intx4{0, 0, 0, 0};
        if (f < units && sr >= 0)
          v[i] = *reinterpret_cast<const intx4*>(src + sr * D + cc + 64 * (f >> 9) + 8 * (f & 7));
      }
#pragma unroll
      for (int i = 0; i < kRqBatch; ++i) {
        const int f = f0 + 256 * i;
        if (f < units) {
          const int k = f & 7, r = (f >> 3) & 63, c = f >> 9;
          float x[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            x[2 * q] = bf16_bits_to_f32((uint32_t)v[i][q] & 0xffffu);
            x[2 * q + 1] = bf16_bits_to_f32((uint32_t)v[i][q] >> 16);
          }
#pragma unroll
          for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(x[q]));
          uint32_t lo, hi;
          if (FMT == kFmtE4M3) {
            lo = pack4_e4m3(x[0] * s, x[1] * s, x[2] * s, x[3] * s);
            hi = pack4_e4m3(x[4] * s, x[5] * s, x[6] * s, x[7] * s);
          } else {
            lo = pack4_e5m2(x[0] * s, x[1] * s, x[2] * s, x[3] * s);
            hi = pack4_e5m2(x[4] * s, x[5] * s, x[6] * s, x[7] * s);
          }
          if (xs)
            *reinterpret_cast<intx2*>(xs + ((cc >> 6) + c) * ldp * 64 + (p0 + r) * 64 + 8 * k) =
                intx2{(int)lo, (int)hi};
          if (xt) *reinterpret_cast<intx2*>(tile + r * stride + 64 * c + 8 * k) = intx2{(int)lo, (int)hi};
        }
      }
    }
    if (xt) {  // work-group uniform
      __syncthreads();
      lds_rows_store_slab_tr<kRqRows>(tile, C, stride, xt, cp, p0, cc);
      __syncthreads();  // the next chunk overwrites the tile
    }
  }
  block_amax_atomic<4>(m, red, amax + aslot);
}

// out[t, :] = bf16(sum over j = 0 .. k-1 of dx[inv[t*k + j], :]) with an
// fp32 sum in slot order (train.py:2213-2217); rows whose index is out of
// range add nothing.  One thread per 8 columns of one token.
__global__ __launch_bounds__(256) void moe_topk_sum_kernel(const uint16_t* __restrict__ dx, int64_t R, int64_t D,
                                                           const int64_t* __restrict__ inv, int64_t T, int k,
                                                           uint16_t* __restrict__ out) {
  const int64_t per_row = D / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= T * per_row) return;
  const int64_t t = i / per_row, d = 8 * (i % per_row);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < k; ++j) {
    const int64_t r = inv[t * k + j];
    if (r < 0 || r >= R) continue;
    const intx4 v = *reinterpret_cast<const intx4*>(dx + r * D + d);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += bf16_bits_to_f32((uint32_t)v[q] & 0xffffu);
      acc[2 * q + 1] += bf16_bits_to_f32((uint32_t)v[q] >> 16);
    }
  }
  intx4 o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = (int)pack2_bf16(acc[2 * q], acc[2 * q + 1]);
  *reinterpret_cast<intx4*>(out + t * D + d) = o;
}

}  // namespace sfp8

// ============================================================================
// C ABI
// ============================================================================
using namespace sfp8;

namespace {
inline int moe_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}
inline bool moe_al16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }

// dynamic LDS above 64 KiB must be opted into per kernel
template <typename K>
int moe_allow_lds(K kernel, size_t bytes) {
  if (bytes <= 65536) return kOk;
  const hipError_t e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)bytes);
  return e == hipSuccess ? kOk : (int)e;
}
}  // namespace

extern "C" {

int64_t sfp8_moe_plan_ints(int64_t R, int64_t E) {
  if (R < 0 || E <= 0 || E > kMaxExperts) return -1;
  return moe_plan_ints(R, E);
}

int64_t sfp8_moe_padded_rows(int64_t R, int64_t E) {
  if (R < 0 || E <= 0 || E > kMaxExperts) return -1;
  return 256 * moe_max_tiles(R, E);
}

int sfp8_moe_plan(const int* offsets, int64_t E, int64_t R, int* plan, int64_t plan_ints, void* stream) {
  if (!offsets || !plan) return kErrNullPointer;
  if (E <= 0 || E > kMaxExperts || R < 0 || R > (int64_t)1 << 30) return kErrBadShape;
  if (plan_ints < moe_plan_ints(R, E)) return kErrWorkspaceTooSmall;
  hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, offsets, (int)E, R,
                     (int)moe_max_tiles(R, E), plan);
  return moe_status();
}

int sfp8_moe_rows_quant(const void* src, int64_t nsrc, int64_t D, const int64_t* map, int64_t nmap,
                        const int* plan, int64_t ldp, const float* scale, int sslot, float* amax, int aslot,
                        int fmt, void* xs, void* xt, void* stream) {
  if (!scale || !amax || !plan || (ldp > 0 && !xs && !xt) || (nsrc > 0 && !src)) return kErrNullPointer;
  if (D <= 0 || D % 128 || ldp < 0 || ldp % 256 || nsrc < 0 || nmap < 0) return kErrBadShape;
  if (sslot < 0 || sslot > 4 || aslot < 0 || aslot > 4 || (fmt != kFmtE4M3 && fmt != kFmtE5M2) ||
      (xs && fmt != kFmtE4M3))
    return kErrBadShape;
  if (!moe_al16(src) || !moe_al16(xs) || !moe_al16(xt)) return kErrBadAlignment;
  if (ldp == 0) return kOk;
  const int64_t C = D < kRqChunk ? D : kRqChunk;
  const size_t lds = xt ? (size_t)kRqRows * (C + 16) : 0;  // the transposing tile
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)(ldp / kRqRows));
  const int rc = fmt == kFmtE4M3 ? moe_allow_lds(moe_rows_quant_kernel<kFmtE4M3>, lds)
                                 : moe_allow_lds(moe_rows_quant_kernel<kFmtE5M2>, lds);
  if (rc) return rc;
  if (fmt == kFmtE4M3) {
    hipLaunchKernelGGL(moe_rows_quant_kernel<kFmtE4M3>, grid, dim3(256), lds, st, (const uint16_t*)src, nsrc, D, map,
                       nmap, plan, scale, sslot, amax, aslot, (uint8_t*)xs, (uint8_t*)xt, ldp);
  } else {
    hipLaunchKernelGGL(moe_rows_quant_kernel<kFmtE5M2>, grid, dim3(256), lds, st, (const uint16_t*)src, nsrc, D, map,
                       nmap, plan, scale, sslot, amax, aslot, (uint8_t*)xs, (uint8_t*)xt, ldp);
  }
  return moe_status();
}

int sfp8_moe_topk_sum(const void* dx, int64_t R, int64_t D, const int64_t* inv, int64_t T, int64_t k, void* out,
                      void* stream) {
  if ((T > 0 && (!out || !inv)) || (R > 0 && !dx)) return kErrNullPointer;
  if (R < 0 || T < 0 || D <= 0 || D % 8 || k <= 0) return kErrBadShape;
  if (!moe_al16(dx) || !moe_al16(out)) return kErrBadAlignment;
  if (T == 0) return kOk;
  const int64_t n = T * (D / 8);
  hipLaunchKernelGGL(moe_topk_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)dx, R, D, inv, T, (int)k, (uint16_t*)out);
  return moe_status();
}

}  // extern "C"
