// FP8 / bf16 MFMA GEMMs of the FP8 MLP block (gfx950, CDNA4).
//
// Every GEMM here is C[m, n] = sum_k A[m, k] * B[n, k]: both operands are
// K-contiguous rows in HBM.  One work-group (256 threads = 4 waves, one wave
// per SIMD) computes a 256 x 256 output tile with the pipelined main loop of
// mainloop.h; each wave owns 128 x 128 as 4 x 4 blocks of 32 x 32 MFMA
// accumulators.
//
// MFMA: v_mfma_f32_32x32x64_f8f6f4 (e4m3/e5m2 chosen per operand) or
// v_mfma_f32_32x32x16_bf16.  The B fragment is passed as the instruction's
// first operand and the A fragment as its second, so each lane ends up holding
// ONE row m (lane % 32) and runs of 4 consecutive n: element v of a 32x32
// block is (m = lane % 32, n = 8*(v/4) + 4*(lane/32) + v%4).  Row-major
// epilogue stores are therefore 4-element runs.  Within one instruction both
// operands use the same (lane-half, byte) -> k assignment, so any consistent
// placement of K inside a fragment gives the same dot product.
#include "common.h"
#include "mainloop.h"
#include "scale.h"

namespace sfp8 {

// Work-group -> tile mapping.  Work-groups are dispatched round-robin over
// the 8 XCDs; consecutive logical tiles are placed on the same XCD (each XCD
// has its own L2), then grouped 8 tile-rows at a time so a column of B tiles
// is reused from L2 across neighbouring A tiles.
SFP8_DEV void tile_coords(int pid, int nwg, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int per = nwg >> 3, rem = nwg & 7;
  const int xcd = pid & 7, local = pid >> 3;
  const int lid = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  constexpr int G = 8;
  const int group = G * tiles_n;
  const int first_m = (lid / group) * G;
  const int gsz = (tiles_m - first_m) < G ? (tiles_m - first_m) : G;
  tm = first_m + (lid % group) % gsz;
  tn = (lid % group) / gsz;
}

SFP8_DEV floatx16 zero16() {
  return floatx16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
}

// Row-major copy-out of a byte tile staged in LDS: rows x cols bytes (cols
// multiple of 16), row r -> out + r*ldo, rows >= rows_valid skipped.
SFP8_DEV void lds_tile_store_rows(const uint8_t* lds, int rows, int cols, int stride, uint8_t* out,
                                  int64_t ldo, int rows_valid) {
  const int cpr = cols >> 4;
  for (int idx = threadIdx.x; idx < rows * cpr; idx += 256) {
    const int r = idx / cpr, c = idx % cpr;
    if (r < rows_valid)
      *reinterpret_cast<intx4*>(out + (int64_t)r * ldo + c * 16) =
          *reinterpret_cast<const intx4*>(lds + r * stride + c * 16);
  }
}

// Transposed copy-out of an LDS byte tile (see quant.hip for the scheme).
SFP8_DEV void lds_tile_store_cols(const uint8_t* lds, int rows, int cols, int stride, uint8_t* out,
                                  int64_t ldo, int rows_valid) {
  const int nb_c = cols >> 2;
  const int nblocks = (rows >> 4) * nb_c;
  for (int idx = threadIdx.x; idx < nblocks; idx += 256) {
    const int b = idx % nb_c, a = idx / nb_c;
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = a * 16 + i;
      w[i] = (r < rows_valid) ? *reinterpret_cast<const uint32_t*>(lds + r * stride + b * 4) : 0u;
    }
    uint32_t t[4][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint32_t o[4];
      transpose4x4_bytes(&w[4 * q], o);
#pragma unroll
      for (int c = 0; c < 4; ++c) t[c][q] = o[c];
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<intx4*>(out + (int64_t)(b * 4 + c) * ldo + a * 16) =
          intx4{(int)t[c][0], (int)t[c][1], (int)t[c][2], (int)t[c][3]};
  }
}

// ---------------------------------------------------------------------------
// (a6) gate/up forward + SwiGLU epilogue (spark-gpt train.py:975-1016).
// Tile: 256 tokens x 128 intermediate columns; the B tile holds gate rows
// n0..n0+127 then up rows I+n0..I+n0+127, and each wave's B blocks pair a gate
// block with the up block of the same columns.
constexpr int kEpiStride = 144;

__global__ __launch_bounds__(256, 1) void swiglu_fwd_kernel(
    const uint8_t* __restrict__ x8, const uint8_t* __restrict__ w8, int64_t T, int64_t D, int64_t I,
    const float* __restrict__ scale, const float* __restrict__ wscale, float* __restrict__ amax,
    uint8_t* __restrict__ gu8, uint8_t* __restrict__ h8, uint8_t* __restrict__ h8t, int64_t ldt,
    int tiles_m, int tiles_n) {
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ float red[8];
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * 128;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  floatx16 acc[4][4];
  MainLoop<false, kFmtE4M3, kFmtE4M3, true>::run(
      lds, x8 + m0 * D, (T - m0) * D, [=](int r) { return r * (int)D; }, w8 + n0 * D, (2 * I - n0) * D,
      [=](int r) { return (r < 128 ? r : (int)I + r - 128) * (int)D; }, 0, (int)(D / kStage), acc);
  // ---- epilogue
  const float deq = 1.0f / (scale[0] * wscale[0]);
  const float q1 = scale[1], q2 = scale[2];
  uint8_t* Gt = lds;
  uint8_t* Ut = lds + kTile * kEpiStride;
  uint8_t* Ht = lds + 2 * kTile * kEpiStride;
  float m_gu = 0.f, m_h = 0.f;
  const int fr = lane & 31, g = lane >> 5;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int row = 128 * wm + 32 * tb + fr;  // token within the tile
    const bool valid = m0 + row < T;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float gg[4], uu[4], hh[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          gg[e] = acc[tb][nb][4 * q + e] * deq;
          uu[e] = acc[tb][nb + 2][4 * q + e] * deq;
        }
        // g, u rounded to bf16 as in the bf16 path (train.py:1006-1007)
        round2_bf16(gg[0], gg[1]);
        round2_bf16(gg[2], gg[3]);
        round2_bf16(uu[0], uu[1]);
        round2_bf16(uu[2], uu[3]);
        float mg = 0.f, mh = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          hh[e] = gg[e] * sigmoid_fast(gg[e]) * uu[e];
          mg = fmaxf(mg, fmaxf(fabsf(gg[e]), fabsf(uu[e])));
          mh = fmaxf(mh, fabsf(hh[e]));
        }
        if (valid) {
          m_gu = fmaxf(m_gu, mg);
          m_h = fmaxf(m_h, mh);
        }
        const int col = 64 * wn + 32 * nb + 8 * q + 4 * g;  // column within the 128-wide tile
        const uint32_t pg = pack4_e4m3(gg[0] * q1, gg[1] * q1, gg[2] * q1, gg[3] * q1);
        const uint32_t pu = pack4_e4m3(uu[0] * q1, uu[1] * q1, uu[2] * q1, uu[3] * q1);
        const uint32_t ph = pack4_e4m3(hh[0] * q2, hh[1] * q2, hh[2] * q2, hh[3] * q2);
        *reinterpret_cast<uint32_t*>(Gt + row * kEpiStride + col) = pg;
        *reinterpret_cast<uint32_t*>(Ut + row * kEpiStride + col) = pu;
        *reinterpret_cast<uint32_t*>(Ht + row * kEpiStride + col) = valid ? ph : 0u;
      }
    }
  }
  __syncthreads();
  const int rows_valid = (int)((T - m0) < kTile ? (T - m0) : kTile);
  lds_tile_store_rows(Gt, kTile, 128, kEpiStride, gu8 + m0 * 2 * I + n0, 2 * I, rows_valid);
  lds_tile_store_rows(Ut, kTile, 128, kEpiStride, gu8 + m0 * 2 * I + I + n0, 2 * I, rows_valid);
  lds_tile_store_rows(Ht, kTile, 128, kEpiStride, h8 + m0 * I + n0, I, rows_valid);
  lds_tile_store_cols(Ht, kTile, 128, kEpiStride, h8t + n0 * ldt + m0, ldt, rows_valid);
  m_gu = wave_max(m_gu);
  m_h = wave_max(m_h);
  if (lane == 0) { red[wave] = m_gu; red[4 + wave] = m_h; }
  __syncthreads();
  if (tid == 0) {
    atomic_max_nonneg(amax + 1, fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
    atomic_max_nonneg(amax + 2, fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7])));
  }
}

// ---------------------------------------------------------------------------
// (a7) down forward + residual (spark-gpt train.py:1019-1046):
//   y = bf16(res + bf16(acc / (s2 * q_d)))
__global__ __launch_bounds__(256, 1) void down_fwd_kernel(
    const uint8_t* __restrict__ h8, const uint8_t* __restrict__ wd8, const uint16_t* __restrict__ res,
    int64_t T, int64_t D, int64_t I, const float* __restrict__ scale, const float* __restrict__ wscale,
    uint16_t* __restrict__ y, int tiles_m, int tiles_n) {
  extern __shared__ __align__(16) uint8_t lds[];
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int wb_row[4] = {128 * wn, 128 * wn + 32, 128 * wn + 64, 128 * wn + 96};
  floatx16 acc[4][4];
  MainLoop<false, kFmtE4M3, kFmtE4M3, false>::run(
      lds, h8 + m0 * I, (T - m0) * I, [=](int r) { return r * (int)I; }, wd8 + n0 * I, (D - n0) * I,
      [=](int r) { return r * (int)I; }, 0, (int)(I / kStage), acc);
  const float deq = 1.0f / (scale[2] * wscale[1]);
  const int fr = lane & 31, g = lane >> 5;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int64_t t = m0 + 128 * wm + 32 * tb + fr;
    if (t >= T) continue;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wb_row[nb] + 8 * q + 4 * g;
        if (n >= D) continue;
        const intx2 rv = *reinterpret_cast<const intx2*>(res + t * D + n);
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = acc[tb][nb][4 * q + e] * deq;
        // out rounded to bf16 before the residual add (train.py:1043)
        round2_bf16(o[0], o[1]);
        round2_bf16(o[2], o[3]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t u = (uint32_t)rv[e >> 1];
          o[e] += bf16_bits_to_f32((e & 1) ? (u >> 16) : (u & 0xffffu));
        }
        *reinterpret_cast<intx2*>(y + t * D + n) = intx2{(int)pack2_bf16(o[0], o[1]), (int)pack2_bf16(o[2], o[3])};
      }
  }
}

// ---------------------------------------------------------------------------
// (a9) bf16 down dgrad + SwiGLU backward (spark-gpt train.py:1049-1094):
//   dh = bf16(dy @ Wd); g, u = gu8 / s1; sig = sigmoid(g)
//   d_gate = dh*u*(sig*(1+g*(1-sig))), d_up = dh*g*sig
//   dgu8 = e5m2(d * s3) row-major and transposed (ldt), amax slot 3.
// B = Wd^T (bf16, [I, D]).  Tile 256 tokens x 256 intermediate columns.
constexpr int kEpiStride2 = 272;

__global__ __launch_bounds__(256, 1) void down_dgrad_swiglu_kernel(
    const uint16_t* __restrict__ dy, const uint16_t* __restrict__ wdt, const uint8_t* __restrict__ gu8,
    int64_t T, int64_t D, int64_t I, const float* __restrict__ scale, float* __restrict__ amax,
    uint8_t* __restrict__ dgu8, uint8_t* __restrict__ dgu8t, int64_t ldt, int tiles_m, int tiles_n) {
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ float red[4];
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t ldb = D * 2;  // bytes
  const int wb_row[4] = {128 * wn, 128 * wn + 32, 128 * wn + 64, 128 * wn + 96};
  floatx16 acc[4][4];
  MainLoop<true, 0, 0, false>::run(
      lds, reinterpret_cast<const uint8_t*>(dy) + m0 * ldb, (T - m0) * ldb, [=](int r) { return r * (int)ldb; },
      reinterpret_cast<const uint8_t*>(wdt) + n0 * ldb, (I - n0) * ldb, [=](int r) { return r * (int)ldb; }, 0,
      (int)(ldb / kStage), acc);
  const float s_gu = 1.0f / scale[1];
  const float q3 = scale[3];
  uint8_t* Gt = lds;
  uint8_t* Ut = lds + kTile * kEpiStride2;
  float m3 = 0.f;
  const int fr = lane & 31, g = lane >> 5;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int row = 128 * wm + 32 * tb + fr;
    const int64_t t = m0 + row;
    const bool valid = t < T;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = wb_row[nb] + 8 * q + 4 * g;
        const int64_t j = n0 + col;
        uint32_t pg = 0u, pu = 0u;
        if (valid && j < I) {
          const uint32_t wg = *reinterpret_cast<const uint32_t*>(gu8 + t * 2 * I + j);
          const uint32_t wu = *reinterpret_cast<const uint32_t*>(gu8 + t * 2 * I + I + j);
          float dh[4], dg[4], du[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) dh[e] = acc[tb][nb][4 * q + e];
          // dh rounded to bf16 (train.py:1082)
          round2_bf16(dh[0], dh[1]);
          round2_bf16(dh[2], dh[3]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gv = e4m3_to_f32(wg, e) * s_gu;
            const float uv = e4m3_to_f32(wu, e) * s_gu;
            const float sg = sigmoid_fast(gv);
            dg[e] = dh[e] * uv * (sg * (1.0f + gv * (1.0f - sg)));
            du[e] = dh[e] * gv * sg;
            m3 = fmaxf(m3, fmaxf(fabsf(dg[e]), fabsf(du[e])));
          }
          pg = pack4_e5m2(dg[0] * q3, dg[1] * q3, dg[2] * q3, dg[3] * q3);
          pu = pack4_e5m2(du[0] * q3, du[1] * q3, du[2] * q3, du[3] * q3);
        }
        *reinterpret_cast<uint32_t*>(Gt + row * kEpiStride2 + col) = pg;
        *reinterpret_cast<uint32_t*>(Ut + row * kEpiStride2 + col) = pu;
      }
  }
  __syncthreads();
  const int rows_valid = (int)((T - m0) < kTile ? (T - m0) : kTile);
  const int cols = (int)((I - n0) < kTile ? (I - n0) : kTile);
  lds_tile_store_rows(Gt, kTile, cols, kEpiStride2, dgu8 + m0 * 2 * I + n0, 2 * I, rows_valid);
  lds_tile_store_rows(Ut, kTile, cols, kEpiStride2, dgu8 + m0 * 2 * I + I + n0, 2 * I, rows_valid);
  lds_tile_store_cols(Gt, kTile, cols, kEpiStride2, dgu8t + n0 * ldt + m0, ldt, rows_valid);
  lds_tile_store_cols(Ut, kTile, cols, kEpiStride2, dgu8t + (I + n0) * ldt + m0, ldt, rows_valid);
  block_amax_atomic<4>(m3, red, amax + 3);
}

// ---------------------------------------------------------------------------
// (a10) gate/up dgrad (spark-gpt train.py:1239-1241):
//   dxn = bf16(acc * (1/s3) * (1/q_gu)), A = d_gu8 (e5m2, [T, 2I]), B = W8^T (e4m3, [D, 2I]).
__global__ __launch_bounds__(256, 1) void gateup_dgrad_kernel(
    const uint8_t* __restrict__ dgu8, const uint8_t* __restrict__ w8t, int64_t T, int64_t D, int64_t I,
    const float* __restrict__ scale, const float* __restrict__ wscale, uint16_t* __restrict__ dxn,
    int tiles_m, int tiles_n) {
  extern __shared__ __align__(16) uint8_t lds[];
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t K = 2 * I;
  const int wb_row[4] = {128 * wn, 128 * wn + 32, 128 * wn + 64, 128 * wn + 96};
  floatx16 acc[4][4];
  MainLoop<false, kFmtE5M2, kFmtE4M3, false>::run(
      lds, dgu8 + m0 * K, (T - m0) * K, [=](int r) { return r * (int)K; }, w8t + n0 * K, (D - n0) * K,
      [=](int r) { return r * (int)K; }, 0, (int)(K / kStage), acc);
  const float sa = 1.0f / scale[3], sb = 1.0f / wscale[0];
  const int fr = lane & 31, g = lane >> 5;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int64_t t = m0 + 128 * wm + 32 * tb + fr;
    if (t >= T) continue;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wb_row[nb] + 8 * q + 4 * g;
        if (n >= D) continue;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = acc[tb][nb][4 * q + e] * sa * sb;
        *reinterpret_cast<intx2*>(dxn + t * D + n) = intx2{(int)pack2_bf16(o[0], o[1]), (int)pack2_bf16(o[2], o[3])};
      }
  }
}

// ---------------------------------------------------------------------------
// (a12, a13) weight gradients, reduced over tokens:
//   out[m, n] = sum_t A[m, t] * B[n, t] / (sa * sb)
// A, B are the token-contiguous (transposed) fp8 copies with leading
// dimension ldt (zero-padded past T).  blockIdx.y splits K; with splits > 1
// each split writes raw fp32 partials to ws[split] and splitk_reduce sums
// them in split order (deterministic).
template <int FMT_A, int FMT_B>
__global__ __launch_bounds__(256, 1) void wgrad_kernel(
    const uint8_t* __restrict__ at, const uint8_t* __restrict__ bt, int64_t M, int64_t N, int64_t ldt,
    int64_t kchunk, const float* __restrict__ sa, const float* __restrict__ sb, float* __restrict__ out,
    int tiles_m, int tiles_n) {
  extern __shared__ __align__(16) uint8_t lds[];
  int tm, tn;
  tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * kTile, n0 = (int64_t)tn * kTile;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int wb_row[4] = {128 * wn, 128 * wn + 32, 128 * wn + 64, 128 * wn + 96};
  floatx16 acc[4][4];
  const int64_t kb = (int64_t)blockIdx.y * kchunk;
  MainLoop<false, FMT_A, FMT_B, false>::run(
      lds, at + m0 * ldt, (M - m0) * ldt, [=](int r) { return r * (int)ldt; }, bt + n0 * ldt, (N - n0) * ldt,
      [=](int r) { return r * (int)ldt; }, kb, (int)(kchunk / kStage), acc);
  const bool split = gridDim.y > 1;
  const float deq = split ? 1.0f : 1.0f / (sa[0] * sb[0]);
  float* dst = out + (split ? (int64_t)blockIdx.y * M * N : 0);
  const int fr = lane & 31, g = lane >> 5;
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    const int64_t m = m0 + 128 * wm + 32 * tb + fr;
    if (m >= M) continue;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t n = n0 + wb_row[nb] + 8 * q + 4 * g;
        if (n >= N) continue;
        floatx4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = acc[tb][nb][4 * q + e] * deq;
        *reinterpret_cast<floatx4*>(dst + m * N + n) = o;
      }
  }
}

}  // namespace sfp8

// ============================================================================
// C ABI
// ============================================================================
using namespace sfp8;

namespace {

constexpr int kSwigluLds = 3 * kTile * kEpiStride;   // 110592 < kMainLds
constexpr int kDgradLds = 2 * kTile * kEpiStride2;   // 139264 > kMainLds

template <typename K>
int prep(K kernel, int lds_bytes) {
  // dynamic LDS above 64 KiB must be opted into once per kernel
  const hipError_t e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           lds_bytes);
  return e == hipSuccess ? kOk : (int)e;
}

inline int status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}

inline bool al16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }
inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
// offsets inside one operand tile are 32-bit
inline bool fits32(int64_t rows, int64_t ld) { return rows * ld < (int64_t)1 << 31; }

}  // namespace

extern "C" {

int sfp8_gemm_gateup_swiglu_fwd(const void* x8, const void* w8, int64_t T, int64_t D, int64_t I,
                                const float* scale, const float* wscale, float* amax, void* gu8, void* h8,
                                void* h8t, int64_t ldt, void* stream) {
  if (!x8 || !w8 || !scale || !wscale || !amax || !gu8 || !h8 || !h8t) return kErrNullPointer;
  if (T < 0 || D <= 0 || I <= 0 || D % (2 * kStage) || I % 128 || ldt < T || ldt % kTile) return kErrBadShape;
  if (!fits32(kTile, D) || !fits32(2 * I, D)) return kErrBadShape;
  if (!al16(x8) || !al16(w8) || !al16(gu8) || !al16(h8) || !al16(h8t)) return kErrBadAlignment;
  if (T == 0) return kOk;
  const int tiles_m = cdiv(T, kTile), tiles_n = (int)(I / 128);
  int rc = prep(swiglu_fwd_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(swiglu_fwd_kernel, dim3(tiles_m * tiles_n), dim3(256), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)x8, (const uint8_t*)w8, T, D, I, scale, wscale, amax, (uint8_t*)gu8,
                     (uint8_t*)h8, (uint8_t*)h8t, ldt, tiles_m, tiles_n);
  return status();
}

int sfp8_gemm_down_fwd(const void* h8, const void* wd8, const void* res, int64_t T, int64_t D, int64_t I,
                       const float* scale, const float* wscale, void* y, void* stream) {
  if (!h8 || !wd8 || !res || !scale || !wscale || !y) return kErrNullPointer;
  if (T < 0 || D <= 0 || I <= 0 || I % (2 * kStage) || D % 4) return kErrBadShape;
  if (!fits32(kTile, I)) return kErrBadShape;
  if (!al16(h8) || !al16(wd8) || !al16(res) || !al16(y)) return kErrBadAlignment;
  if (T == 0) return kOk;
  const int tiles_m = cdiv(T, kTile), tiles_n = cdiv(D, kTile);
  int rc = prep(down_fwd_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(down_fwd_kernel, dim3(tiles_m * tiles_n), dim3(256), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)h8, (const uint8_t*)wd8, (const uint16_t*)res, T, D, I, scale, wscale,
                     (uint16_t*)y, tiles_m, tiles_n);
  return status();
}

int sfp8_gemm_down_dgrad_swiglu(const void* dy, const void* wdt, const void* gu8, int64_t T, int64_t D,
                                int64_t I, const float* scale, float* amax, void* dgu8, void* dgu8t,
                                int64_t ldt, void* stream) {
  if (!dy || !wdt || !gu8 || !scale || !amax || !dgu8 || !dgu8t) return kErrNullPointer;
  if (T < 0 || D <= 0 || I <= 0 || (2 * D) % (2 * kStage) || I % 16 || ldt < T || ldt % kTile) return kErrBadShape;
  if (!fits32(kTile, 2 * D)) return kErrBadShape;
  if (!al16(dy) || !al16(wdt) || !al16(gu8) || !al16(dgu8) || !al16(dgu8t)) return kErrBadAlignment;
  if (T == 0) return kOk;
  const int tiles_m = cdiv(T, kTile), tiles_n = cdiv(I, kTile);
  int rc = prep(down_dgrad_swiglu_kernel, kDgradLds);
  if (rc) return rc;
  hipLaunchKernelGGL(down_dgrad_swiglu_kernel, dim3(tiles_m * tiles_n), dim3(256), kDgradLds,
                     (hipStream_t)stream, (const uint16_t*)dy, (const uint16_t*)wdt, (const uint8_t*)gu8, T, D,
                     I, scale, amax, (uint8_t*)dgu8, (uint8_t*)dgu8t, ldt, tiles_m, tiles_n);
  return status();
}

int sfp8_gemm_gateup_dgrad(const void* dgu8, const void* w8t, int64_t T, int64_t D, int64_t I,
                           const float* scale, const float* wscale, void* dxn, void* stream) {
  if (!dgu8 || !w8t || !scale || !wscale || !dxn) return kErrNullPointer;
  if (T < 0 || D <= 0 || I <= 0 || (2 * I) % (2 * kStage) || D % 4) return kErrBadShape;
  if (!fits32(kTile, 2 * I)) return kErrBadShape;
  if (!al16(dgu8) || !al16(w8t) || !al16(dxn)) return kErrBadAlignment;
  if (T == 0) return kOk;
  const int tiles_m = cdiv(T, kTile), tiles_n = cdiv(D, kTile);
  int rc = prep(gateup_dgrad_kernel, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL(gateup_dgrad_kernel, dim3(tiles_m * tiles_n), dim3(256), kMainLds, (hipStream_t)stream,
                     (const uint8_t*)dgu8, (const uint8_t*)w8t, T, D, I, scale, wscale, (uint16_t*)dxn, tiles_m,
                     tiles_n);
  return status();
}

// Number of K splits the library uses for an (M, N, ldt) weight gradient and
// the workspace (floats) it needs: splits * M * N when splits > 1, else 0.
int64_t sfp8_wgrad_splits(int64_t M, int64_t N, int64_t ldt) {
  const int64_t tiles = (int64_t)cdiv(M, kTile) * cdiv(N, kTile);
  int64_t s = 1;
  while (tiles * s < 512 && ldt % (s * 2) == 0 && (ldt / (s * 2)) % (2 * kStage) == 0 && ldt / (s * 2) >= 2048)
    s *= 2;
  return s;
}

int64_t sfp8_wgrad_workspace_floats(int64_t M, int64_t N, int64_t ldt) {
  const int64_t s = sfp8_wgrad_splits(M, N, ldt);
  return s > 1 ? s * M * N : 0;
}

int sfp8_splitk_reduce(const float* ws, int64_t splits, int64_t M, int64_t N, const float* sa,
                       const float* sb, float* out, void* stream);

int sfp8_gemm_wgrad(const void* at, int fmt_a, const void* bt, int fmt_b, int64_t M, int64_t N, int64_t ldt,
                    const float* sa, const float* sb, float* out, float* ws, int64_t ws_floats, void* stream) {
  if (!at || !bt || !sa || !sb || !out) return kErrNullPointer;
  if (M <= 0 || N <= 0 || ldt < 0 || ldt % kTile || N % 4) return kErrBadShape;
  if (fmt_a != kFmtE5M2 || fmt_b != kFmtE4M3) return kErrBadShape;
  if (!fits32(kTile, ldt)) return kErrBadShape;
  if (!al16(at) || !al16(bt) || !al16(out)) return kErrBadAlignment;
  hipStream_t st = (hipStream_t)stream;
  const int64_t splits = sfp8_wgrad_splits(M, N, ldt);
  if (splits > 1 && (!ws || ws_floats < splits * M * N)) return kErrWorkspaceTooSmall;
  if (ldt == 0) {
    return hipMemsetAsync(out, 0, (size_t)(M * N * 4), st) == hipSuccess ? kOk : status();
  }
  const int tiles_m = cdiv(M, kTile), tiles_n = cdiv(N, kTile);
  int rc = prep(wgrad_kernel<kFmtE5M2, kFmtE4M3>, kMainLds);
  if (rc) return rc;
  hipLaunchKernelGGL((wgrad_kernel<kFmtE5M2, kFmtE4M3>), dim3(tiles_m * tiles_n, (unsigned)splits), dim3(256),
                     kMainLds, st, (const uint8_t*)at, (const uint8_t*)bt, M, N, ldt, ldt / splits, sa, sb,
                     splits > 1 ? ws : out, tiles_m, tiles_n);
  rc = status();
  if (rc || splits == 1) return rc;
  return sfp8_splitk_reduce(ws, splits, M, N, sa, sb, out, stream);
}

}  // extern "C"
