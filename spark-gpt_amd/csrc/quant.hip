// HBM-bound kernels of the FP8 MLP block (gfx950):
//   quant_rowcol    standalone bf16 -> e4m3 row-major + transposed, amax
//   norm_quant      RMSNorm -> e4m3 K-slab (+ optional transposed copy), rstd, amax slot 0
//   weight_quant    just-in-time per-tensor pow2 e4m3 copy of an fp32 master
//   update_scales   delayed-scale roll of the 5 recipe slots
//   norm_bwd        RMSNorm backward + residual, dnw partials, e5m2 dy (K-slab and/or
//                   transposed copy), amax slot 4
//   reductions      dnw partial sum, split-K sum
//
// Byte transposes go through an LDS tile: the row-major pass writes the fp8
// tile into LDS, then each thread gathers a 16(row) x 4(col) byte block with
// dword reads, transposes it in registers (v_perm) and writes 16-byte runs of
// the transposed output.
#include <mutex>

#include "common.h"
#include "scale.h"

namespace sfp8 {

// Row block of work-group pid in a 1-D grid of nblk row blocks.  Work-groups
// are dispatched round-robin over the 8 XCDs (pid % 8); XCD x gets a
// contiguous run of row blocks, so neighbouring blocks -- whose token-
// contiguous (transposed) outputs share 128-byte lines -- run on the same XCD
// and their partial lines merge in its L2.  A bijection of [0, nblk).
SFP8_DEV int xcd_row_block(int pid, int nblk) {
  const int per = nblk >> 3, rem = nblk & 7;
  const int xcd = pid & 7, local = pid >> 3;
  return (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}


// --------------------------------------------------------------------------
// Standalone quantizer: x8 = e4m3(x * s) row-major, x8t = the K-slab of
// x8^T over ldt tokens ([ldt/64][slab_rows(C)][64]), amax = max|x|.
// A work-group of 256 threads takes COLS columns of 16384 / COLS rows (64 x
// 256, or 128 x 128 when C is not a multiple of 256).  Every thread issues
// its eight 16-byte row loads before converting any of them; NaN lanes are
// patched on a wave-uniform path taken only when the wave saw a NaN.  The
// tile goes to LDS, is read back transposed with lds_read_tr8 (a 16-lane
// group turns a 16 x 16 byte block into 16 column runs of 16 rows) into a
// column-major LDS tile, and leaves as 64-byte slab rows: each 64-token slab
// of the tile is one contiguous block of COLS * 64 bytes of x8t.  Work-groups
// past column C write the slab's zero padding rows.
template <int COLS>
struct QuantRowcolCfg {
  static constexpr int kRows = 16384 / COLS;
  static constexpr int kRowsPerPass = 256 / (COLS / 8);
  static constexpr int kTileStride = COLS + 16;   // = 4 (mod 8) dwords: conflict-free transposing reads
  static constexpr int kColStride = kRows + 16;   // = 4 (mod 16) dwords: a group's 16 writes hit distinct banks
};

template <int COLS>
__global__ __launch_bounds__(256) void quant_rowcol_kernel(
    const uint16_t* __restrict__ x, int64_t R, int64_t C, const float* __restrict__ scale,
    float* __restrict__ amax, uint8_t* __restrict__ x8, uint8_t* __restrict__ x8t, int64_t ldt) {
  using Cfg = QuantRowcolCfg<COLS>;
  constexpr int ROWS = Cfg::kRows, TS = Cfg::kTileStride, CS = Cfg::kColStride;
  __shared__ __align__(16) uint8_t tile[ROWS * TS];
  __shared__ __align__(16) uint8_t tcol[COLS * CS];  // [column][ROWS rows]
  __shared__ float red[4];
  // consecutive work-groups take consecutive column blocks of the same rows,
  // so each input row is read while its DRAM page is open
  const int64_t r0 = (int64_t)blockIdx.y * ROWS;
  const int64_t c0 = (int64_t)blockIdx.x * COLS;
  const bool live = c0 < C;  // work-group uniform; false: slab padding only
  const float s = scale[0];
  const int c8 = threadIdx.x % (COLS / 8);  // 8-element chunk within the tile row
  const int rr = threadIdx.x / (COLS / 8);  // row within a pass
  intx4 v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int64_t gr = r0 + rr + Cfg::kRowsPerPass * i;
    v[i] = live && gr < R ? __builtin_nontemporal_load(reinterpret_cast<const intx4*>(x + gr * C + c0 + c8 * 8))
                           : intx4{0, 0, 0, 0};
  }
  float m = 0.0f;
  bool nan = false;
  uint32_t lo[8], hi[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t u = (uint32_t)v[i][j];
      f[2 * j] = bf16_bits_to_f32(u & 0xffffu);
      f[2 * j + 1] = bf16_bits_to_f32(u >> 16);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      m = fmaxf(m, fabsf(f[j]));
      nan |= f[j] != f[j];
    }
    lo[i] = pack4_e4m3_nofix(f[0] * s, f[1] * s, f[2] * s, f[3] * s);
    hi[i] = pack4_e4m3_nofix(f[4] * s, f[5] * s, f[6] * s, f[7] * s);
  }
  if (__builtin_amdgcn_ballot_w64(nan)) {  // wave-uniform, taken only with NaN data
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      // re-read the row chunk (keeps the loaded vectors dead after the cast)
      const int64_t gr = r0 + rr + Cfg::kRowsPerPass * i;
      const intx4 w = gr < R ? *reinterpret_cast<const intx4*>(x + gr * C + c0 + c8 * 8) : intx4{0, 0, 0, 0};
      float f[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t u = (uint32_t)w[j];
        f[2 * j] = bf16_bits_to_f32(u & 0xffffu);
        f[2 * j + 1] = bf16_bits_to_f32(u >> 16);
      }
      lo[i] = fix_nan4(lo[i], f[0] * s, f[1] * s, f[2] * s, f[3] * s);
      hi[i] = fix_nan4(hi[i], f[4] * s, f[5] * s, f[6] * s, f[7] * s);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = rr + Cfg::kRowsPerPass * i;
    const int64_t gr = r0 + r;
    if (live && gr < R) *reinterpret_cast<intx2*>(x8 + gr * C + c0 + c8 * 8) = intx2{(int)lo[i], (int)hi[i]};
    *reinterpret_cast<intx2*>(tile + r * TS + c8 * 8) = intx2{(int)lo[i], (int)hi[i]};  // zeros past R
  }
  __syncthreads();
  // 16 x 16 byte blocks: (ROWS / 16) x (COLS / 16) = 64 of them, four per
  // 16-lane group; group g takes column block (g + 16 p) % (COLS / 16) ...
  const int lane = threadIdx.x & 63;
  const int g = threadIdx.x >> 4, li = lane & 15;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int blk = 16 * p + g;
    const int cb = 16 * (blk % (COLS / 16)), rb = 16 * (blk / (COLS / 16));
    // source lane li = 2b + h points at tile row rb + b (+8), columns cb + 8h ..
    const uint8_t* src = tile + (rb + (li >> 1)) * TS + cb + 8 * (li & 1);
    const intx2 t0 = lds_read_tr8(src);
    const intx2 t1 = lds_read_tr8(src + 8 * TS);
    *reinterpret_cast<intx4*>(tcol + (cb + li) * CS + rb) = intx4{t0[0], t0[1], t1[0], t1[1]};
  }
  __syncthreads();
  // slab rows: 4 lanes per 64-token column run, consecutive columns in
  // consecutive lanes, so a wave store covers 16 whole slab rows (1 KiB)
  const int64_t cp = slab_rows(C);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int idx = k * 256 + threadIdx.x;
    const int sl = idx / (4 * COLS), col = (idx % (4 * COLS)) >> 2, ch = idx & 3;
    const int64_t t = r0 + 64 * sl;
    if (t >= ldt) continue;  // ldt % 64 == 0
    const intx4 w = *reinterpret_cast<const intx4*>(tcol + col * CS + 64 * sl + 16 * ch);
    *reinterpret_cast<intx4*>(x8t + (t >> 6) * cp * 64 + (c0 + col) * 64 + 16 * ch) = w;
  }
  block_amax_atomic<4>(m, red, amax);
}

// --------------------------------------------------------------------------
// Norm-fused quantizer (spark-gpt train.py:955-972).
//   rstd[t] = fl32(1/sqrt(fl64(fl32(sum h^2)/D + eps)))   (sum exact in fp64)
//   n = (h * rstd) * w;  x8 = e4m3(n * s0);  amax0 = max |n|
// x8 is the K-slab [D/64][ldt][64] over ldt tokens (a multiple of 256);
// tokens T..ldt-1 are written as zeros so a GEMM can reduce over ldt tokens.
// x8t (optional: null skips it) is the token-contiguous
// K-slab copy (common.h), for weight gradients that read token-contiguous
// operands.
// Each work-group owns RT rows; a row is split over LPR lanes holding CPL
// 8-element chunks each.
template <int D>
struct NormCfg {
  static constexpr int LPR = (D / 8) < 64 ? (D / 8) : 64;  // lanes per row
  static constexpr int RPW = 64 / LPR;                       // rows per wave pass
  static constexpr int CPL = D / (8 * LPR);                  // chunks per lane
  static constexpr int RT = (65536 / D) < 64 ? (65536 / D) : 64;  // rows per WG
  // LDS row stride: D + 16 bytes puts the 8 rows of a transposing read on
  // distinct bank pairs
  static constexpr int STRIDE = D + 16;
  // norm_quant: 8 waves per work-group up to D = 1024 (two work-groups per
  // CU fit the LDS, so 4 waves per SIMD), 4 beyond (whose registers need 2
  // waves per SIMD); QPASSES row passes per wave, PB of them with their loads
  // issued together and their square roots taken together: about 8 chunks
  // of 16 bytes per lane, 4 from D = 1024 on (at D = 1024 eight need more
  // than the 128 registers of 4 waves per SIMD, and spill)
  static constexpr int QW = D <= 1024 ? 8 : 4;
  static constexpr int QPASSES = RT / (QW * RPW);
  static constexpr int QCH = CPL >= 2 ? 4 : 8;
  static constexpr int PB = (QCH / CPL) < QPASSES ? ((QCH / CPL) > 0 ? QCH / CPL : 1) : QPASSES;
  // norm_bwd: BW waves per work-group (8 up to D = 1024: 4 waves per SIMD
  // beside the LDS tile, as for norm_quant), PASSES row passes per wave,
  // PB_BWD per batch
  static constexpr int BW = D <= 1024 ? 8 : 4;
  static constexpr int PASSES = RT / (BW * RPW);
  static constexpr int LB = (BW == 8 ? 2 : 4) / CPL;  // row chunks per lane in one load batch
  static constexpr int PB_BWD = LB < PASSES ? (LB > 0 ? LB : 1) : PASSES;
  // norm_bwd loads the next batch while it computes one (two register sets)
  // at D = 2048 (3 % faster alone); at D = 4096 two sets do not fit the
  // registers, and up to D = 1024 they need 2 waves per SIMD instead of 4,
  // which measured 5 % slower in the block's step (as did the same for
  // norm_quant's batches: no faster)
  static constexpr bool PIPE_BWD = CPL == 4;
  static_assert(QPASSES % PB == 0 && PASSES % PB_BWD == 0, "whole load batches");
};

template <int D>
__global__ __launch_bounds__(64 * NormCfg<D>::QW) __attribute__((amdgpu_waves_per_eu(NormCfg<D>::QW / 2)))
void norm_quant_kernel(
    const uint16_t* __restrict__ h, const float* __restrict__ nw, int64_t T, float eps,
    const float* __restrict__ scale, float* __restrict__ amax, uint8_t* __restrict__ x8,
    uint8_t* __restrict__ x8t, int64_t ldt, float* __restrict__ rstd) {
  using Cfg = NormCfg<D>;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float red[Cfg::QW];
  uint8_t* tile = smem;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wid_s = __builtin_amdgcn_readfirstlane(wid);
  const int sr = lane / Cfg::LPR, li = lane % Cfg::LPR;
  const int blk = xcd_row_block(blockIdx.x, gridDim.x);
  const int64_t t0 = (int64_t)blk * Cfg::RT;
  const float s0 = scale[0];
  const float inv0 = 1.0f / s0, bnd0 = kE4M3Max * inv0;
  float m = 0.0f;
  // norm weight for this lane's chunks
  float w[Cfg::CPL][8];
#pragma unroll
  for (int c = 0; c < Cfg::CPL; ++c) {
    const int d = (c * Cfg::LPR + li) * 8;
    const floatx4 a = *reinterpret_cast<const floatx4*>(nw + d);
    const floatx4 b = *reinterpret_cast<const floatx4*>(nw + d + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) { w[c][j] = a[j]; w[c][4 + j] = b[j]; }
  }
  // wave wid takes row passes wid, wid + QW, ...; PB passes' loads are
  // issued before any of them is reduced
#pragma unroll 1
  for (int pb = 0; pb < Cfg::QPASSES; pb += Cfg::PB) {
    intx4 v[Cfg::PB][Cfg::CPL];
#pragma unroll
    for (int q = 0; q < Cfg::PB; ++q) {
      const int64_t t = t0 + (wid + Cfg::QW * (pb + q)) * Cfg::RPW + sr;
#pragma unroll
      for (int c = 0; c < Cfg::CPL; ++c) {
        const int d = (c * Cfg::LPR + li) * 8;
        v[q][c] = t < T ? __builtin_nontemporal_load(reinterpret_cast<const intx4*>(h + t * D + d)) : intx4{0, 0, 0, 0};
      }
    }
    // the batch's row sums first; then lane li of each row group evaluates
    // the rstd of the batch's row li (one square root and division per lane
    // for PB rows), and every lane takes its rows' values back
    double ss[Cfg::PB];
#pragma unroll
    for (int q = 0; q < Cfg::PB; ++q) {
      ss[q] = 0.0;
#pragma unroll
      for (int c = 0; c < Cfg::CPL; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t u = (uint32_t)v[q][c][j];
          const float a = bf16_bits_to_f32(u & 0xffffu), b = bf16_bits_to_f32(u >> 16);
          // squares of bf16 values are exact in fp64
          ss[q] = __builtin_fma((double)a, (double)a, ss[q]);
          ss[q] = __builtin_fma((double)b, (double)b, ss[q]);
        }
#pragma unroll
      for (int o = Cfg::LPR / 2; o > 0; o >>= 1) ss[q] += __shfl_xor(ss[q], o, 64);
    }
    static_assert(Cfg::PB <= Cfg::LPR, "one lane per row of the batch");
    double sel = ss[0];
#pragma unroll
    for (int q = 1; q < Cfg::PB; ++q) sel = li == q ? ss[q] : sel;
    const float rl = (float)(1.0 / __builtin_sqrt((double)((float)sel / (float)D + eps)));
#pragma unroll
    for (int q = 0; q < Cfg::PB; ++q) {
      const int r = (wid + Cfg::QW * (pb + q)) * Cfg::RPW + sr;
      const int64_t t = t0 + r;
      const bool valid = t < T;
      const float r_ = __shfl(rl, sr * Cfg::LPR + q, 64);
      float f[Cfg::CPL][8];
#pragma unroll
      for (int c = 0; c < Cfg::CPL; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t u = (uint32_t)v[q][c][j];
          f[c][2 * j] = bf16_bits_to_f32(u & 0xffffu);
          f[c][2 * j + 1] = bf16_bits_to_f32(u >> 16);
        }
      if (valid && li == 0) rstd[t] = r_;
      float n[Cfg::CPL][8];
      float mw = 0.0f;  // max |n| over this lane's values, NaN if one is NaN
#pragma unroll
      for (int c = 0; c < Cfg::CPL; ++c)
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
          n[c][j] = (f[c][j] * r_) * w[c][j];
          n[c][j + 1] = (f[c][j + 1] * r_) * w[c][j + 1];
          mw = max3_nan(mw, fabsf(n[c][j]), fabsf(n[c][j + 1]));
        }
      // Common case, decided once per row set of the wave: every value finite
      // and |n * s0| <= 448, so the clamp is the identity and the scaled
      // converter (which divides by 1/s0, exact for a power of two) gives the
      // codes directly.  Otherwise the clamp and the NaN codes per value.
      const bool fast = !__builtin_amdgcn_ballot_w64(!(mw <= bnd0));
      if (fast && valid) m = fmaxf(m, mw);
#pragma unroll
      for (int c = 0; c < Cfg::CPL; ++c) {
        const int d = (c * Cfg::LPR + li) * 8;
        uint32_t lo, hi;
        if (fast) {
          lo = pack4_e4m3_scaled_noclamp(n[c][0], n[c][1], n[c][2], n[c][3], inv0, 0u);
          hi = pack4_e4m3_scaled_noclamp(n[c][4], n[c][5], n[c][6], n[c][7], inv0, 0u);
          if (!valid) lo = hi = 0u;
        } else {
          lo = hi = 0u;
          if (valid) {
#pragma unroll
            for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(n[c][j]));
            lo = pack4_e4m3(n[c][0] * s0, n[c][1] * s0, n[c][2] * s0, n[c][3] * s0);
            hi = pack4_e4m3(n[c][4] * s0, n[c][5] * s0, n[c][6] * s0, n[c][7] * s0);
          }
        }
        // x8 is a K-slab [D/64][ldt][64] (the gate/up GEMM's A operand),
        // zeros for tokens T..ldt-1.  Written from the registers: without
        // x8t the kernel needs no LDS tile, and the occupancy that buys
        // outweighs whole-run stores staged through one (4 % at D = 1024)
        *reinterpret_cast<intx2*>(x8 + (int64_t)(d >> 6) * ldt * 64 + t * 64 + (d & 63)) = intx2{(int)lo, (int)hi};
        if (x8t) *reinterpret_cast<intx2*>(tile + r * Cfg::STRIDE + d) = intx2{(int)lo, (int)hi};
      }
      __builtin_amdgcn_sched_barrier(0);  // rows one after another (register pressure)
    }
  }
  if (x8t) {  // the optional token-contiguous copy (rows past T hold zero codes)
    __syncthreads();
    lds_rows_store_slab_tr<Cfg::RT, Cfg::QW>(tile, D, Cfg::STRIDE, x8t, slab_rows(D), t0, 0);
  }
  block_amax_atomic_w<Cfg::QW>(m, red, amax, wid_s);
}

// --------------------------------------------------------------------------
// Norm-fused quantizer for wide rows (D >= 8192, D % 4096 == 0), same
// results as norm_quant_kernel: a row no longer fits a wave's registers, so
// a work-group of 64 tokens makes two passes.  Pass 1: each wave reduces
// sum h^2 of 16 rows (fp64, exact) into rstd.  Pass 2, per 1024-column
// chunk: each wave normalises and quantizes its 16 rows' chunk into the x8
// K-slab and, when the token-contiguous x8t is asked for, an LDS tile that
// leaves as whole 64-byte rows of x8t (transposing LDS reads).  The chunk's
// second read of h mostly hits the caches.
constexpr int kWideRows = 64;
constexpr int kWideChunk = 1024;
constexpr int kWideStride = kWideChunk + 16;  // LDS tile row stride (conflict-free transposing reads)
constexpr int kWideLdsTile = kWideRows * kWideStride;

__host__ __device__ inline bool wide_hidden(int64_t D) { return D >= 8192 && D % 4096 == 0; }

__global__ __launch_bounds__(256) void norm_quant_wide_kernel(
    const uint16_t* __restrict__ h, const float* __restrict__ nw, int64_t T, int64_t D, float eps,
    const float* __restrict__ scale, float* __restrict__ amax, uint8_t* __restrict__ x8,
    uint8_t* __restrict__ x8t, int64_t ldt, float* __restrict__ rstd) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float red[4];
  __shared__ float rs_sh[kWideRows];
  uint8_t* tile = smem;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int blk = xcd_row_block(blockIdx.x, gridDim.x);
  const int64_t t0 = (int64_t)blk * kWideRows;
  const float s0 = scale[0];
  // pass 1: sum of squares, 8 loads of 16 bytes per lane in flight
  for (int rr = 0; rr < 16; ++rr) {
    const int r = 16 * wid + rr;
    const int64_t t = t0 + r;
    double ss = 0.0;
    if (t < T) {
      const uint16_t* row = h + t * D;
      for (int64_t c0 = 0; c0 < D; c0 += 8 * 512) {
        intx4 v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = *reinterpret_cast<const intx4*>(row + c0 + 512 * k + 8 * lane);
#pragma unroll
        for (int k = 0; k < 8; ++k)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float a = bf16_bits_to_f32((uint32_t)v[k][j] & 0xffffu), b = bf16_bits_to_f32((uint32_t)v[k][j] >> 16);
            ss = __builtin_fma((double)a, (double)a, ss);  // squares of bf16 values are exact in fp64
            ss = __builtin_fma((double)b, (double)b, ss);
          }
      }
    }
    ss = wave_sum_f64(ss);
    const float var = (float)ss / (float)D + eps;
    const float r_ = (float)(1.0 / __builtin_sqrt((double)var));
    if (lane == 0) {
      rs_sh[r] = r_;
      if (t < T) rstd[t] = r_;
    }
  }
  __syncthreads();
  float m = 0.0f;
  const int64_t cp = slab_rows(D);
  for (int64_t cc = 0; cc < D; cc += kWideChunk) {
    // the lane's 8 columns of each 512-column half of the chunk
    float w[2][8];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(nw + cc + 512 * hf + 8 * lane);
      const floatx4 b = *reinterpret_cast<const floatx4*>(nw + cc + 512 * hf + 8 * lane + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) { w[hf][j] = a[j]; w[hf][4 + j] = b[j]; }
    }
#pragma unroll 1
    for (int rb = 0; rb < 16; rb += 4) {
      intx4 v[4][2];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int64_t t = t0 + 16 * wid + rb + q;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
          v[q][hf] = t < T ? *reinterpret_cast<const intx4*>(h + t * D + cc + 512 * hf + 8 * lane) : intx4{0, 0, 0, 0};
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 16 * wid + rb + q;
        const int64_t t = t0 + r;
        const bool valid = t < T;
        const float r_ = rs_sh[r];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          float n[8];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            n[2 * j] = (bf16_bits_to_f32((uint32_t)v[q][hf][j] & 0xffffu) * r_) * w[hf][2 * j];
            n[2 * j + 1] = (bf16_bits_to_f32((uint32_t)v[q][hf][j] >> 16) * r_) * w[hf][2 * j + 1];
          }
          uint32_t lo = 0u, hi = 0u;
          if (valid) {
#pragma unroll
            for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(n[j]));
            lo = pack4_e4m3(n[0] * s0, n[1] * s0, n[2] * s0, n[3] * s0);
            hi = pack4_e4m3(n[4] * s0, n[5] * s0, n[6] * s0, n[7] * s0);
          }
          const int64_t d = cc + 512 * hf + 8 * lane;
          // x8 is a K-slab [D/64][ldt][64], zeros for tokens T..ldt-1
          *reinterpret_cast<intx2*>(x8 + (d >> 6) * ldt * 64 + t * 64 + (d & 63)) = intx2{(int)lo, (int)hi};
          if (x8t)
            *reinterpret_cast<intx2*>(tile + r * kWideStride + 512 * hf + 8 * lane) = intx2{(int)lo, (int)hi};
        }
      }
    }
    if (x8t) {
      __syncthreads();
      lds_rows_store_slab_tr<kWideRows>(tile, kWideChunk, kWideStride, x8t, cp, t0, cc);
      __syncthreads();  // the next chunk overwrites the tile
    }
  }
  block_amax_atomic<4>(m, red, amax);
}

// --------------------------------------------------------------------------
// Weight quantization (spark-gpt train.py:949-952), two launches:
//   weight_amax_kernel:  per-block max|w| partials (no zero-init needed)
//   weight_quant_kernel: every block folds the partials into amax and
//     q = exp2(floor(log2(448 / max(amax, 1e-30)))), then writes its tile of
//     w8 = e4m3(w * q) as a K-slab over W's columns and/or over its rows
//     (the GEMMs' B operands: rows of 64 contiguous K bytes), and optionally
//     a bf16 K-slab of W^T.  Block 0 stores q.
constexpr int WQ_PARTS = 512;

// Expert e = blockIdx.y of a batch (E matrices of n elements, partials
// gridDim.x per expert); a dense weight is the batch of one.
// Block b of nb: the max |w| over its grid-stride share of w[0, n), to partials[b].
SFP8_DEV void weight_amax_block(const float* __restrict__ w, int64_t n, int b, int nb, float* __restrict__ partials) {
  __shared__ float red[4];
  float m = 0.0f;
  const int64_t n4 = n >> 2;
  const int64_t step = (int64_t)nb * 256;
  const floatx4* w4 = reinterpret_cast<const floatx4*>(w);
  int64_t i = (int64_t)b * 256 + threadIdx.x;
  // four independent loads in flight per trip
  for (; i + 3 * step < n4; i += 4 * step) {
    floatx4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = w4[i + u * step];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v[u][0]), fabsf(v[u][1])), fmaxf(fabsf(v[u][2]), fabsf(v[u][3]))));
  }
  for (; i < n4; i += step) {
    const floatx4 v = w4[i];
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
  }
  if (b == 0)
    for (int64_t i = (n4 << 2) + threadIdx.x; i < n; i += 256) m = fmaxf(m, fabsf(w[i]));
  m = wave_max(m);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = m;
  __syncthreads();
  if (threadIdx.x == 0) partials[b] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ __launch_bounds__(256) void weight_amax_kernel(const float* __restrict__ w, int64_t n,
                                                           float* __restrict__ partials) {
  weight_amax_block(w + (int64_t)blockIdx.y * n, n, blockIdx.x, gridDim.x,
                    partials + (int64_t)blockIdx.y * gridDim.x);
}

constexpr int WQ_TILE = 64;

// Tile (bx, by) of one matrix: rows 64 bx.., columns 64 by.. (the tiles
// cover rows and columns up to multiples of 256, so that the padding rows of
// every K-slab output are written, as zeros).
SFP8_DEV void weight_quant_tile(const float* __restrict__ w, int64_t R, int64_t C, const float* __restrict__ partials,
                                int nparts, float* __restrict__ q_out, uint8_t* __restrict__ w8,
                                uint8_t* __restrict__ w8t, uint16_t* __restrict__ wbt, int bx, int by) {
  __shared__ float red[4];
  __shared__ float qs;
  __shared__ __align__(16) uint8_t t8[WQ_TILE * (WQ_TILE + 8)];
  __shared__ __align__(16) uint16_t t16[WQ_TILE * (WQ_TILE + 2)];
  const int64_t r0 = (int64_t)bx * WQ_TILE, c0 = (int64_t)by * WQ_TILE;
  const int64_t rp = (R + 255) / 256 * 256, cp = (C + 255) / 256 * 256;
  // each thread: 4 consecutive columns of 4 rows (64x64 tile = 1024 quads);
  // the tile's loads are issued first, so their latency overlaps the fold
  // of the amax partials below
  floatx4 vq[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int idx = threadIdx.x + 256 * k;
    const int64_t gr = r0 + idx / (WQ_TILE / 4), gc = c0 + (idx % (WQ_TILE / 4)) * 4;
    vq[k] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (gr < R && gc < C) vq[k] = *reinterpret_cast<const floatx4*>(w + gr * C + gc);
  }
  float m = 0.0f;
  for (int i = threadIdx.x; i < nparts; i += 256) m = fmaxf(m, partials[i]);
  m = wave_max(m);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float a = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float q = pow2_scale(a, kE4M3Max, 0, true);
    qs = q;
    if (bx == 0 && by == 0) *q_out = q;
  }
  __syncthreads();
  const float q = qs;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int idx = threadIdx.x + 256 * k;
    const int r = idx / (WQ_TILE / 4), c4 = idx % (WQ_TILE / 4);
    const int64_t gr = r0 + r, gc = c0 + c4 * 4;
    const floatx4 v = vq[k];
    const uint32_t p = pack4_e4m3(v[0] * q, v[1] * q, v[2] * q, v[3] * q);
    // w8: K-slab of W over its columns, [C/64][rp][64]
    if (w8 && c0 < C) *reinterpret_cast<uint32_t*>(w8 + (gc >> 6) * rp * 64 + gr * 64 + (gc & 63)) = p;
    *reinterpret_cast<uint32_t*>(t8 + r * (WQ_TILE + 8) + c4 * 4) = p;
#pragma unroll
    for (int j = 0; j < 4; ++j) t16[(c4 * 4 + j) * (WQ_TILE + 2) + r] = (uint16_t)f32_to_bf16_bits(v[j]);
  }
  __syncthreads();
  if (r0 >= R) return;  // row padding of w8 only
  // w8t: K-slab of W^T over its columns (W's rows), [R/64][cp][64]: this
  // tile is 64 slab rows (W columns c0..) of 64 bytes (W rows r0..)
  if (w8t) {
    const int c = threadIdx.x >> 2, ch = threadIdx.x & 3;
    uint32_t wv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t word = 0u;
#pragma unroll
      for (int b = 0; b < 4; ++b) word |= (uint32_t)t8[(16 * ch + 4 * k + b) * (WQ_TILE + 8) + c] << (8 * b);
      wv[k] = word;
    }
    *reinterpret_cast<intx4*>(w8t + (r0 >> 6) * cp * 64 + (c0 + c) * 64 + 16 * ch) =
        intx4{(int)wv[0], (int)wv[1], (int)wv[2], (int)wv[3]};
  }
  // wbt: K-slab of bf16(W)^T, [R/32][cp][32] bf16 (64-byte rows of 32 W rows)
  if (wbt) {
    for (int idx = threadIdx.x; idx < 512; idx += 256) {
      const int c = idx >> 3, hp = (idx >> 2) & 1, j = idx & 3;
      if (r0 + 32 * hp >= R) continue;  // R % 64 == 32: the tile's second panel is past the end
      const uint32_t* src = reinterpret_cast<const uint32_t*>(t16 + c * (WQ_TILE + 2) + 32 * hp + 8 * j);
      *reinterpret_cast<intx4*>(wbt + ((r0 >> 5) + hp) * cp * 32 + (c0 + c) * 32 + 8 * j) =
          intx4{(int)src[0], (int)src[1], (int)src[2], (int)src[3]};
    }
  }
}

__global__ __launch_bounds__(256) void weight_quant_kernel(
    const float* __restrict__ w, int64_t R, int64_t C, const float* __restrict__ partials, int nparts,
    float* __restrict__ q_out, uint8_t* __restrict__ w8, uint8_t* __restrict__ w8t,
    uint16_t* __restrict__ wbt) {
  // expert e = blockIdx.z of a batch: its matrix, partials, scale and the
  // three K-slab copies (each a whole K-slab per expert)
  const int64_t e = blockIdx.z;
  const int64_t rp = (R + 255) / 256 * 256, cp = (C + 255) / 256 * 256;
  weight_quant_tile(w + e * R * C, R, C, partials + e * nparts, nparts, q_out + e, w8 ? w8 + e * C * rp : nullptr,
                    w8t ? w8t + e * R * cp : nullptr, wbt ? wbt + e * R * cp : nullptr, blockIdx.x, blockIdx.y);
}

// --------------------------------------------------------------------------
// The post-step quantization of one dense block in two launches instead of
// five: the gate/up master W_gu [R0, C0] -> w8, w8t and the down master
// W_down [R1, C1] -> wd8, wdt (bf16 K-slab of its transpose), with the
// delayed-scale roll of the block's 5 slots done by the first launch's
// block (0, 0) (the roll and the quantizations share no data).
struct WeightPair {
  const float* w[2];
  int64_t R[2], C[2];
  float* partials;  // WQ_PARTS per matrix
  int nparts[2];
  float* q_out;     // [q_gu, q_d]
  uint8_t* w8[2];
  uint8_t* w8t;     // W_gu's
  uint16_t* wbt;    // W_down's
  int tiles_r[2], tiles_c[2];
  float* scale;     // the 5 slots to roll, or null
  float* amax;
};

__global__ __launch_bounds__(256) void weight_amax_pair_kernel(WeightPair p) {
  const int j = blockIdx.y;
  if (j == 0 && blockIdx.x == 0 && p.scale && threadIdx.x < 5) {
    const int slot = threadIdx.x;
    const float a = p.amax[slot];
    if (a > 0.0f) p.scale[slot] = pow2_scale(a, slot < 3 ? kE4M3Max : kE5M2Max, 1, false);
    p.amax[slot] = 0.0f;
  }
  if ((int)blockIdx.x >= p.nparts[j]) return;  // work-group uniform
  weight_amax_block(p.w[j], p.R[j] * p.C[j], blockIdx.x, p.nparts[j], p.partials + j * WQ_PARTS);
}

// 1-D grid: W_gu's tiles (row-major over tiles_r[0] x tiles_c[0]), then W_down's.
__global__ __launch_bounds__(256) void weight_quant_pair_kernel(WeightPair p) {
  int t = blockIdx.x;
  const int j = t < p.tiles_r[0] * p.tiles_c[0] ? 0 : 1;
  if (j) t -= p.tiles_r[0] * p.tiles_c[0];
  weight_quant_tile(p.w[j], p.R[j], p.C[j], p.partials + j * WQ_PARTS, p.nparts[j], p.q_out + j, p.w8[j],
                    j ? nullptr : p.w8t, j ? p.wbt : nullptr, t / p.tiles_c[j], t % p.tiles_c[j]);
}

// --------------------------------------------------------------------------
// Delayed-scale roll (spark-gpt train.py:937-946): for each slot with amax > 0,
// scale = exp2(floor(log2(fmax / amax)) - 1); amax = 0.
__global__ void update_scales_kernel(float* __restrict__ scale, float* __restrict__ amax, int nsets,
                                     int headroom) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nsets * 5) return;
  const int slot = i % 5;
  const float fmax = slot < 3 ? kE4M3Max : kE5M2Max;
  const float a = amax[i];
  if (a > 0.0f) scale[i] = pow2_scale(a, fmax, headroom, false);
  amax[i] = 0.0f;
}

// --------------------------------------------------------------------------
// RMSNorm backward + residual (spark-gpt train.py:1130-1147):
//   g = dxn, gw = g*w, S = sum_d gw*h
//   dh = bf16(gw*r - h*(S*r*r*r*(1/D)) + dy)
//   dnw_part[block][d] = sum over the block's rows of g*(h*r)
// plus, for the down-proj weight gradient, e5m2(dy * s4) as the K-slab dy8
// [D/64][ldt][64] and/or the token-contiguous K-slab copy dy8t (each
// optional; zeros for tokens T..ldt-1), and amax slot 4 = max|dy|
// (recorded at train.py:1074-1081).
template <int D>
__global__ __launch_bounds__(64 * NormCfg<D>::BW) __attribute__((amdgpu_waves_per_eu(NormCfg<D>::BW == 8 ? 4 : 1)))
void norm_bwd_kernel(
    const uint16_t* __restrict__ h, const float* __restrict__ rstd, const uint16_t* __restrict__ dxn,
    const uint16_t* __restrict__ dy, const float* __restrict__ nw, int64_t T,
    const float* __restrict__ scale, float* __restrict__ amax, uint16_t* __restrict__ dh,
    float* __restrict__ dnw_part, uint8_t* __restrict__ dy8, uint8_t* __restrict__ dy8t, int64_t ldt) {
  using Cfg = NormCfg<D>;
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float red[Cfg::BW];
  uint8_t* tile = smem;
  // [BW waves][D] floats, in the tile's LDS after the dy8 / dy8t stores have
  // read it (the only LDS when there is neither)
  float* dnw_red = reinterpret_cast<float*>(smem);
  static_assert(Cfg::BW * D * sizeof(float) <= Cfg::RT * Cfg::STRIDE, "dnw reduction fits in the tile");
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int sr = lane / Cfg::LPR, li = lane % Cfg::LPR;
  const int blk = xcd_row_block(blockIdx.x, gridDim.x);
  const int64_t t0 = (int64_t)blk * Cfg::RT;
  const float s4 = scale[4];
  float m = 0.0f;
  float w[Cfg::CPL][8], acc[Cfg::CPL][8];
#pragma unroll
  for (int c = 0; c < Cfg::CPL; ++c) {
    const int d = (c * Cfg::LPR + li) * 8;
    const floatx4 a = *reinterpret_cast<const floatx4*>(nw + d);
    const floatx4 b = *reinterpret_cast<const floatx4*>(nw + d + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) { w[c][j] = a[j]; w[c][4 + j] = b[j]; acc[c][j] = 0.f; acc[c][4 + j] = 0.f; }
  }
  // wave wid takes row passes wid, wid + BW, ...; a batch is PB_BWD passes
  // whose loads are issued together, and the next batch's loads are issued
  // before this batch is computed (two register sets, so each wave keeps a
  // batch of loads in flight while it computes)
  struct Batch {
    intx4 vh[Cfg::PB_BWD][Cfg::CPL], vg[Cfg::PB_BWD][Cfg::CPL], vd[Cfg::PB_BWD][Cfg::CPL];
    float rsv[Cfg::PB_BWD];
  };
  const auto load_batch = [&](int pb, Batch& B) {
#pragma unroll
    for (int q = 0; q < Cfg::PB_BWD; ++q) {
      const int64_t t = t0 + (wid + Cfg::BW * (pb + q)) * Cfg::RPW + sr;
      const bool valid = t < T;
#pragma unroll
      for (int c = 0; c < Cfg::CPL; ++c) {
        const int d = (c * Cfg::LPR + li) * 8;
        const intx4 z = {0, 0, 0, 0};
        B.vh[q][c] = valid ? __builtin_nontemporal_load(reinterpret_cast<const intx4*>(h + t * D + d)) : z;
        B.vg[q][c] = valid ? __builtin_nontemporal_load(reinterpret_cast<const intx4*>(dxn + t * D + d)) : z;
        B.vd[q][c] = valid ? __builtin_nontemporal_load(reinterpret_cast<const intx4*>(dy + t * D + d)) : z;
      }
      B.rsv[q] = valid ? rstd[t] : 0.0f;
    }
  };
  const auto compute_batch = [&](int pb, const Batch& B) {
#pragma unroll
    for (int q = 0; q < Cfg::PB_BWD; ++q) {
      const int r = (wid + Cfg::BW * (pb + q)) * Cfg::RPW + sr;
      const int64_t t = t0 + r;
      const bool valid = t < T;
      const float rs = B.rsv[q];
      float S = 0.0f;
#pragma unroll
      for (int c = 0; c < Cfg::CPL; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t uh = (uint32_t)B.vh[q][c][j >> 1], ug = (uint32_t)B.vg[q][c][j >> 1];
          const float hf = bf16_bits_to_f32((j & 1) ? (uh >> 16) : (uh & 0xffffu));
          const float g = bf16_bits_to_f32((j & 1) ? (ug >> 16) : (ug & 0xffffu));
          S += (g * w[c][j]) * hf;
        }
#pragma unroll
      for (int o = Cfg::LPR / 2; o > 0; o >>= 1) S += __shfl_xor(S, o, 64);
      const float coef = S * rs * rs * rs * (1.0f / (float)D);
#pragma unroll
      for (int c = 0; c < Cfg::CPL; ++c) {
        const int d = (c * Cfg::LPR + li) * 8;
        float o[8], dyf[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t uh = (uint32_t)B.vh[q][c][j >> 1], ug = (uint32_t)B.vg[q][c][j >> 1];
          const uint32_t ud = (uint32_t)B.vd[q][c][j >> 1];
          const float hf = bf16_bits_to_f32((j & 1) ? (uh >> 16) : (uh & 0xffffu));
          const float g = bf16_bits_to_f32((j & 1) ? (ug >> 16) : (ug & 0xffffu));
          dyf[j] = bf16_bits_to_f32((j & 1) ? (ud >> 16) : (ud & 0xffffu));
          const float gw = g * w[c][j];
          o[j] = (gw * rs - hf * coef) + dyf[j];
          acc[c][j] += g * (hf * rs);
          m = fmaxf(m, fabsf(dyf[j]));
        }
        uint32_t lo = 0u, hi = 0u;
        if (valid) {
          intx4 ov;
#pragma unroll
          for (int j = 0; j < 4; ++j) ov[j] = (int)pack2_bf16(o[2 * j], o[2 * j + 1]);
          *reinterpret_cast<intx4*>(dh + t * D + d) = ov;
          lo = pack4_e5m2(dyf[0] * s4, dyf[1] * s4, dyf[2] * s4, dyf[3] * s4);
          hi = pack4_e5m2(dyf[4] * s4, dyf[5] * s4, dyf[6] * s4, dyf[7] * s4);
        }
        // staged for whole 64-row slab runs of dy8 (7 % faster than 8-byte
        // stores from the registers here, where the LDS is needed anyway)
        if (dy8 || dy8t) *reinterpret_cast<intx2*>(tile + r * Cfg::STRIDE + d) = intx2{(int)lo, (int)hi};
      }
    }
  };
  if constexpr (Cfg::PIPE_BWD) {
    Batch b0, b1;
    load_batch(0, b0);
#pragma unroll 1
    for (int pb = 0; pb < Cfg::PASSES; pb += 2 * Cfg::PB_BWD) {
      if (pb + Cfg::PB_BWD < Cfg::PASSES) load_batch(pb + Cfg::PB_BWD, b1);
      compute_batch(pb, b0);
      if (pb + 2 * Cfg::PB_BWD < Cfg::PASSES) load_batch(pb + 2 * Cfg::PB_BWD, b0);
      if (pb + Cfg::PB_BWD < Cfg::PASSES) compute_batch(pb + Cfg::PB_BWD, b1);
    }
  } else {
#pragma unroll 1
    for (int pb = 0; pb < Cfg::PASSES; pb += Cfg::PB_BWD) {
      Batch b;
      load_batch(pb, b);
      compute_batch(pb, b);
    }
  }
  if (dy8 || dy8t) {  // whole slab runs from the tile; rows past T hold zero codes
    __syncthreads();
    if (dy8) lds_rows_store_slab<Cfg::RT, Cfg::BW>(tile, D, Cfg::STRIDE, dy8, ldt, t0, 0);
    if (dy8t) lds_rows_store_slab_tr<Cfg::RT, Cfg::BW>(tile, D, Cfg::STRIDE, dy8t, slab_rows(D), t0, 0);
  }
  // fold this lane's dnw accumulators over the rows sharing its columns
#pragma unroll
  for (int c = 0; c < Cfg::CPL; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float v = acc[c][j];
      for (int o = Cfg::LPR; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
      acc[c][j] = v;
    }
  __syncthreads();  // every wave has read the tile
  if (sr == 0) {
#pragma unroll
    for (int c = 0; c < Cfg::CPL; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) dnw_red[wid * D + (c * Cfg::LPR + li) * 8 + j] = acc[c][j];
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 64 * Cfg::BW) {
    float v = dnw_red[d];  // the waves' sums in wave order
#pragma unroll
    for (int w2 = 1; w2 < Cfg::BW; ++w2) v += dnw_red[w2 * D + d];
    dnw_part[(int64_t)blk * D + d] = v;
  }
  block_amax_atomic<Cfg::BW>(m, red, amax + 4);
}

// RMSNorm backward for wide rows (D >= 8192, D % 4096 == 0), the same
// computation as norm_bwd_kernel in two passes over a work-group of 64
// tokens: pass 1 reduces S = sum (g*w)*h per row; pass 2, per 1024-column
// chunk, writes dh, accumulates the chunk's dnw partial (each wave over its
// 16 rows in order, then the 4 waves in order) and writes e5m2(dy*s4) into
// the dy8 K-slab and/or stages it for the token-contiguous dy8t, written as
// whole 64-byte rows.
__global__ __launch_bounds__(256) void norm_bwd_wide_kernel(
    const uint16_t* __restrict__ h, const float* __restrict__ rstd, const uint16_t* __restrict__ dxn,
    const uint16_t* __restrict__ dy, const float* __restrict__ nw, int64_t T, int64_t D,
    const float* __restrict__ scale, float* __restrict__ amax, uint16_t* __restrict__ dh,
    float* __restrict__ dnw_part, uint8_t* __restrict__ dy8, uint8_t* __restrict__ dy8t, int64_t ldt) {
  extern __shared__ __align__(16) uint8_t smem[];
  __shared__ float red[4];
  __shared__ float coef_sh[kWideRows], rs_sh[kWideRows];
  uint8_t* tile = smem;
  float* dnw_red = reinterpret_cast<float*>(smem + kWideLdsTile);  // [4 waves][1024]
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int blk = xcd_row_block(blockIdx.x, gridDim.x);
  const int64_t t0 = (int64_t)blk * kWideRows;
  const float s4 = scale[4];
  // pass 1: S per row
  for (int rr = 0; rr < 16; ++rr) {
    const int r = 16 * wid + rr;
    const int64_t t = t0 + r;
    float S = 0.0f, rs = 0.0f;
    if (t < T) {
      rs = rstd[t];
      for (int64_t c0 = 0; c0 < D; c0 += 4 * 512) {
        intx4 vh[4], vg[4];
        floatx4 wa[4], wb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int64_t d = c0 + 512 * k + 8 * lane;
          vh[k] = *reinterpret_cast<const intx4*>(h + t * D + d);
          vg[k] = *reinterpret_cast<const intx4*>(dxn + t * D + d);
          wa[k] = *reinterpret_cast<const floatx4*>(nw + d);
          wb[k] = *reinterpret_cast<const floatx4*>(nw + d + 4);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t uh = (uint32_t)vh[k][j >> 1], ug = (uint32_t)vg[k][j >> 1];
            const float hf = bf16_bits_to_f32((j & 1) ? (uh >> 16) : (uh & 0xffffu));
            const float g = bf16_bits_to_f32((j & 1) ? (ug >> 16) : (ug & 0xffffu));
            const float wv = j < 4 ? wa[k][j] : wb[k][j - 4];
            S += (g * wv) * hf;
          }
      }
    }
    S = wave_sum_f32(S);
    if (lane == 0) {
      coef_sh[r] = S * rs * rs * rs * (1.0f / (float)D);
      rs_sh[r] = rs;
    }
  }
  __syncthreads();
  float m = 0.0f;
  const int64_t cp = slab_rows(D);
  for (int64_t cc = 0; cc < D; cc += kWideChunk) {
    float w[2][8], acc[2][8];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(nw + cc + 512 * hf + 8 * lane);
      const floatx4 b = *reinterpret_cast<const floatx4*>(nw + cc + 512 * hf + 8 * lane + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) { w[hf][j] = a[j]; w[hf][4 + j] = b[j]; }
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[hf][j] = 0.0f;
    }
#pragma unroll 1
    for (int rb = 0; rb < 16; rb += 2) {
      intx4 vh[2][2], vg[2][2], vd[2][2];
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int64_t t = t0 + 16 * wid + rb + q;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          const int64_t o = t * D + cc + 512 * hf + 8 * lane;
          const intx4 z = {0, 0, 0, 0};
          vh[q][hf] = t < T ? *reinterpret_cast<const intx4*>(h + o) : z;
          vg[q][hf] = t < T ? *reinterpret_cast<const intx4*>(dxn + o) : z;
          vd[q][hf] = t < T ? *reinterpret_cast<const intx4*>(dy + o) : z;
        }
      }
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int r = 16 * wid + rb + q;
        const int64_t t = t0 + r;
        const bool valid = t < T;
        const float rs = rs_sh[r], coef = coef_sh[r];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          float o[8], dyf[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t uh = (uint32_t)vh[q][hf][j >> 1], ug = (uint32_t)vg[q][hf][j >> 1];
            const uint32_t ud = (uint32_t)vd[q][hf][j >> 1];
            const float hv = bf16_bits_to_f32((j & 1) ? (uh >> 16) : (uh & 0xffffu));
            const float g = bf16_bits_to_f32((j & 1) ? (ug >> 16) : (ug & 0xffffu));
            dyf[j] = bf16_bits_to_f32((j & 1) ? (ud >> 16) : (ud & 0xffffu));
            const float gw = g * w[hf][j];
            o[j] = (gw * rs - hv * coef) + dyf[j];
            acc[hf][j] += g * (hv * rs);
            m = fmaxf(m, fabsf(dyf[j]));
          }
          const int64_t d = cc + 512 * hf + 8 * lane;
          uint32_t lo = 0u, hi = 0u;
          if (valid) {
            intx4 ov;
#pragma unroll
            for (int j = 0; j < 4; ++j) ov[j] = (int)pack2_bf16(o[2 * j], o[2 * j + 1]);
            *reinterpret_cast<intx4*>(dh + t * D + d) = ov;
            lo = pack4_e5m2(dyf[0] * s4, dyf[1] * s4, dyf[2] * s4, dyf[3] * s4);
            hi = pack4_e5m2(dyf[4] * s4, dyf[5] * s4, dyf[6] * s4, dyf[7] * s4);
          }
          if (dy8) *reinterpret_cast<intx2*>(dy8 + (d >> 6) * ldt * 64 + t * 64 + (d & 63)) = intx2{(int)lo, (int)hi};
          if (dy8t)
            *reinterpret_cast<intx2*>(tile + r * kWideStride + 512 * hf + 8 * lane) = intx2{(int)lo, (int)hi};
        }
      }
    }
    // this wave's dnw partial of the chunk (its 16 rows, in order)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int j = 0; j < 8; ++j) dnw_red[wid * kWideChunk + 512 * hf + 8 * lane + j] = acc[hf][j];
    __syncthreads();
    if (dy8t) lds_rows_store_slab_tr<kWideRows>(tile, kWideChunk, kWideStride, dy8t, cp, t0, cc);
    for (int d = threadIdx.x; d < kWideChunk; d += 256)
      dnw_part[(int64_t)blk * D + cc + d] =
          ((dnw_red[d] + dnw_red[kWideChunk + d]) + dnw_red[2 * kWideChunk + d]) + dnw_red[3 * kWideChunk + d];
    __syncthreads();  // the next chunk overwrites the tile and the reduction rows
  }
  block_amax_atomic<4>(m, red, amax + 4);
}

// Fixed-order column sums over row groups: out[y][d] = sum of part[b][d] for
// b in [y*rpg, min(nb, (y+1)*rpg)).  Work-group (x, y) owns 64 columns of
// group y; thread (r, c) sums rows r, r+4, r+8, ... of the group in ascending
// order, then the 4 partial sums are added in the order r = 0, 1, 2, 3.  Two
// launches (groups, then one group over the group sums) give a sum whose
// order depends only on nb.
constexpr int kColsumGroups = 32;

__global__ __launch_bounds__(256) void zero_f32_kernel(float* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = 0.0f;
}

__global__ __launch_bounds__(256) void colsum_kernel(const float* __restrict__ part, int64_t nb,
                                                     int64_t rpg, int64_t D, float* __restrict__ out) {
  __shared__ float red[4][64];
  const int c = threadIdx.x & 63, r = threadIdx.x >> 6;
  const int64_t d = (int64_t)blockIdx.x * 64 + c;
  const int64_t b0 = (int64_t)blockIdx.y * rpg;
  const int64_t b1 = (b0 + rpg) < nb ? (b0 + rpg) : nb;
  float s = 0.0f;
  if (d < D)
    for (int64_t b = b0 + r; b < b1; b += 4) s += part[b * D + d];
  red[r][c] = s;
  __syncthreads();
  if (r == 0 && d < D) out[(int64_t)blockIdx.y * D + d] = ((red[0][c] + red[1][c]) + red[2][c]) + red[3][c];
}

// Row groups of the first colsum pass for nb partial rows.
static inline int64_t colsum_groups(int64_t nb) { return nb < kColsumGroups ? nb : kColsumGroups; }

// The same sums in one launch for up to kColsum1Rows partial rows (the
// block's 1024 row blocks at 65536 tokens): work-group x owns 32 columns;
// thread (g, c), g = 0..31, sums rows g, g + 32, ... in ascending order,
// then thread c of group 0 adds the 32 group sums in the order g = 0..31.
// The order depends only on nb.
constexpr int kColsum1Rows = 2048;
__global__ __launch_bounds__(1024) void colsum1_kernel(const float* __restrict__ part, int64_t nb, int64_t D,
                                                       float* __restrict__ out) {
  __shared__ float red[32][33];
  const int c = threadIdx.x & 31, g = threadIdx.x >> 5;
  const int64_t d = (int64_t)blockIdx.x * 32 + c;
  float s = 0.0f;
  if (d < D) {
#pragma unroll 16
    for (int64_t b = g; b < nb; b += 32) s += __builtin_nontemporal_load(part + b * D + d);
  }
  red[g][c] = s;
  __syncthreads();
  if (g == 0 && d < D) {
    float t = red[0][c];
#pragma unroll
    for (int i = 1; i < 32; ++i) t += red[i][c];
    out[d] = t;
  }
}

}  // namespace sfp8

// ============================================================================
// Fixed scratch of the allocation-free norm backward (sfp8_norm_bwd_noalloc).
// Every GPU the library runs on holds its own copy of this array until the
// process ends.  In host code `scratch` names a host-side stand-in, not a
// device address: the device address comes from hipGetSymbolAddress, once
// per device, and only that address is passed to kernels.
// ============================================================================
constexpr int64_t kNoAllocScratchFloats = int64_t(8) << 20;  // 32 MiB of fp32 partials (SFP8_NOALLOC_SCRATCH_FLOATS)
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on the first call on
// that device, with that device current).
int scratch_address(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return sfp8::kErrBadShape;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return sfp8::kErrNullPointer;
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return sfp8::kOk;
}
}  // namespace

// ============================================================================
// C ABI
// ============================================================================
using namespace sfp8;

static inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}

static inline bool aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }

// d_norm_w = the column sums of the nb partial rows at part (group sums,
// when two passes are needed, after them).
static int colsum_launch(float* part, int64_t nb, int64_t D, float* dnw, hipStream_t st) {
  if (nb <= kColsum1Rows) {
    hipLaunchKernelGGL(colsum1_kernel, dim3((unsigned)((D + 31) / 32)), dim3(1024), 0, st, (const float*)part, nb, D,
                       dnw);
    return launch_status();
  }
  // partial rows: nb from the norm kernel, then the group sums after them
  const int64_t G = colsum_groups(nb), rpg = (nb + G - 1) / G;
  float* group_sums = part + nb * D;
  const unsigned cblk = (unsigned)((D + 63) / 64);
  hipLaunchKernelGGL(colsum_kernel, dim3(cblk, (unsigned)G), dim3(256), 0, st, part, nb, rpg, D, group_sums);
  hipLaunchKernelGGL(colsum_kernel, dim3(cblk, 1), dim3(256), 0, st, (const float*)group_sums, G, G, D, dnw);
  return launch_status();
}


template <typename K>
static int allow_lds(K kernel, size_t bytes) {
  // dynamic LDS above 64 KiB must be opted into per kernel
  if (bytes <= 65536) return kOk;
  const hipError_t e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)bytes);
  return e == hipSuccess ? kOk : (int)e;
}

template <int D>
static int launch_norm_quant(const void* h, const float* nw, int64_t T, float eps, const float* scale,
                             float* amax, void* x8, void* x8t, int64_t ldt, float* rstd, hipStream_t st) {
  using Cfg = NormCfg<D>;
  const size_t lds = x8t ? (size_t)Cfg::RT * Cfg::STRIDE : 0;  // the transposing tile
  const unsigned nblk = (unsigned)(ldt / Cfg::RT);
  const int rc = allow_lds(norm_quant_kernel<D>, lds);
  if (rc) return rc;
  hipLaunchKernelGGL(norm_quant_kernel<D>, dim3(nblk), dim3(64 * Cfg::QW), lds, st, (const uint16_t*)h, nw, T,
                     eps, scale, amax, (uint8_t*)x8, (uint8_t*)x8t, ldt, rstd);
  return launch_status();
}

template <int D>
static int launch_norm_bwd(const void* h, const float* rstd, const void* dxn, const void* dy,
                           const float* nw, int64_t T, const float* scale, float* amax, void* dh,
                           float* dnw, float* part, void* dy8, void* dy8t, int64_t ldt, hipStream_t st) {
  using Cfg = NormCfg<D>;
  // the transposing tile, or only the dnw reduction rows
  const size_t lds = (dy8 || dy8t) ? (size_t)Cfg::RT * Cfg::STRIDE : (size_t)Cfg::BW * D * sizeof(float);
  const unsigned nblk = (unsigned)(ldt / Cfg::RT);
  const int rc = allow_lds(norm_bwd_kernel<D>, lds);
  if (rc) return rc;
  hipLaunchKernelGGL(norm_bwd_kernel<D>, dim3(nblk), dim3(64 * Cfg::BW), lds, st, (const uint16_t*)h, rstd,
                     (const uint16_t*)dxn, (const uint16_t*)dy, nw, T, scale, amax, (uint16_t*)dh, part,
                     (uint8_t*)dy8, (uint8_t*)dy8t, ldt);
  const int rc2 = launch_status();
  if (rc2) return rc2;
  return colsum_launch(part, (int64_t)nblk, D, dnw, st);
}


static int launch_norm_bwd_wide(const void* h, const float* rstd, const void* dxn, const void* dy, const float* nw,
                                int64_t T, int64_t D, const float* scale, float* amax, void* dh, float* dnw,
                                float* part, void* dy8, void* dy8t, int64_t ldt, hipStream_t st) {
  const size_t lds = (size_t)kWideLdsTile + 4 * kWideChunk * sizeof(float);
  const int rc = allow_lds(norm_bwd_wide_kernel, lds);
  if (rc) return rc;
  const int64_t nb = ldt / kWideRows;
  hipLaunchKernelGGL(norm_bwd_wide_kernel, dim3((unsigned)nb), dim3(256), lds, st, (const uint16_t*)h, rstd,
                     (const uint16_t*)dxn, (const uint16_t*)dy, nw, T, D, scale, amax, (uint16_t*)dh, part,
                     (uint8_t*)dy8, (uint8_t*)dy8t, ldt);
  const int e = launch_status();
  return e ? e : colsum_launch(part, nb, D, dnw, st);
}

extern "C" {

int sfp8_quant_e4m3_rowcol(const void* x, int64_t rows, int64_t cols, const float* scale, float* amax,
                           void* x8, void* x8t, int64_t ldt, void* stream) {
  // row- and token-sized buffers may be null when there are no rows
  if (!scale || !amax || (rows > 0 && cols > 0 && (!x || !x8 || !x8t))) return kErrNullPointer;
  if (rows < 0 || cols < 0 || (cols % 128) != 0 || ldt < rows || (ldt % 64) != 0) return kErrBadShape;
  if (!aligned16(x) || !aligned16(x8) || !aligned16(x8t)) return kErrBadAlignment;
  if (rows == 0 || cols == 0) return kOk;
  // the grid covers the slab's padded columns and all ldt tokens, so that
  // every byte of x8t is written (zeros past rows and cols)
  const int64_t cp = slab_rows(cols);
  hipStream_t st = (hipStream_t)stream;
  if (cols % 256 == 0) {
    constexpr int COLS = 256, ROWS = QuantRowcolCfg<COLS>::kRows;
    dim3 grid((unsigned)(cp / COLS), (unsigned)((ldt + ROWS - 1) / ROWS));
    hipLaunchKernelGGL(quant_rowcol_kernel<COLS>, grid, dim3(256), 0, st, (const uint16_t*)x, rows, cols, scale,
                       amax, (uint8_t*)x8, (uint8_t*)x8t, ldt);
  } else {
    constexpr int COLS = 128, ROWS = QuantRowcolCfg<COLS>::kRows;
    dim3 grid((unsigned)(cp / COLS), (unsigned)((ldt + ROWS - 1) / ROWS));
    hipLaunchKernelGGL(quant_rowcol_kernel<COLS>, grid, dim3(256), 0, st, (const uint16_t*)x, rows, cols, scale,
                       amax, (uint8_t*)x8, (uint8_t*)x8t, ldt);
  }
  return launch_status();
}

static int launch_norm_quant_wide(const void* h, const float* nw, int64_t T, int64_t D, float eps,
                                  const float* scale, float* amax, void* x8, void* x8t, int64_t ldt, float* rstd,
                                  hipStream_t st) {
  const int rc = allow_lds(norm_quant_wide_kernel, kWideLdsTile);
  if (rc) return rc;
  hipLaunchKernelGGL(norm_quant_wide_kernel, dim3((unsigned)(ldt / kWideRows)), dim3(256), kWideLdsTile, st,
                     (const uint16_t*)h, nw, T, D, eps, scale, amax, (uint8_t*)x8, (uint8_t*)x8t, ldt, rstd);
  return launch_status();
}

int sfp8_norm_quant(const void* h, const float* norm_w, int64_t T, int64_t D, float eps,
                    const float* scale, float* amax, void* x8, void* x8t, int64_t ldt, float* rstd,
                    void* stream) {
  // token-sized buffers may be null when there are no tokens
  if (!norm_w || !scale || !amax || (T > 0 && (!h || !x8 || !rstd))) return kErrNullPointer;
  if (T < 0 || ldt < T || (ldt % 256) != 0) return kErrBadShape;
  if (!aligned16(h) || !aligned16(norm_w) || !aligned16(x8) || !aligned16(x8t)) return kErrBadAlignment;
  if (ldt == 0) return kOk;
  hipStream_t st = (hipStream_t)stream;
  switch (D) {
    case 128: return launch_norm_quant<128>(h, norm_w, T, eps, scale, amax, x8, x8t, ldt, rstd, st);
    case 256: return launch_norm_quant<256>(h, norm_w, T, eps, scale, amax, x8, x8t, ldt, rstd, st);
    case 512: return launch_norm_quant<512>(h, norm_w, T, eps, scale, amax, x8, x8t, ldt, rstd, st);
    case 1024: return launch_norm_quant<1024>(h, norm_w, T, eps, scale, amax, x8, x8t, ldt, rstd, st);
    case 2048: return launch_norm_quant<2048>(h, norm_w, T, eps, scale, amax, x8, x8t, ldt, rstd, st);
    case 4096: return launch_norm_quant<4096>(h, norm_w, T, eps, scale, amax, x8, x8t, ldt, rstd, st);
    default:
      if (wide_hidden(D)) return launch_norm_quant_wide(h, norm_w, T, D, eps, scale, amax, x8, x8t, ldt, rstd, st);
      return kErrBadShape;
  }
}

static int weight_quant_batch(const float* w, int64_t E, int64_t rows, int64_t cols, float* partials,
                              int64_t nparts_cap, float* q_out, void* w8, void* w8t, void* wbf16t, hipStream_t st) {
  if (!w || !partials || !q_out) return kErrNullPointer;
  if (E <= 0 || E > 65535 || rows <= 0 || cols <= 0 || (cols % 64) != 0 || (w8t && rows % 64) ||
      (wbf16t && rows % 32))
    return kErrBadShape;
  if (nparts_cap < WQ_PARTS * E) return kErrWorkspaceTooSmall;
  if (!aligned16(w)) return kErrBadAlignment;
  const int64_t n = rows * cols;
  if (n % 4) return kErrBadShape;  // every expert's matrix starts 16-byte aligned
  int nparts = (int)((n / 4 + 255) / 256);
  if (nparts > WQ_PARTS) nparts = WQ_PARTS;
  if (nparts < 1) nparts = 1;
  hipLaunchKernelGGL(weight_amax_kernel, dim3(nparts, (unsigned)E), dim3(256), 0, st, w, n, partials);
  // 64 x 64 tiles over rows and columns rounded up to 256 (K-slab padding), one z-plane per expert
  dim3 grid((unsigned)((rows + 255) / 256 * 4), (unsigned)((cols + 255) / 256 * 4), (unsigned)E);
  hipLaunchKernelGGL(weight_quant_kernel, grid, dim3(256), 0, st, w, rows, cols, partials, nparts, q_out,
                     (uint8_t*)w8, (uint8_t*)w8t, (uint16_t*)wbf16t);
  return launch_status();
}

int sfp8_weight_quant(const float* w, int64_t rows, int64_t cols, float* partials, int64_t nparts_cap,
                      float* q_out, void* w8, void* w8t, void* wbf16t, void* stream) {
  return weight_quant_batch(w, 1, rows, cols, partials, nparts_cap, q_out, w8, w8t, wbf16t, (hipStream_t)stream);
}

int sfp8_weight_quant_experts(const float* w, int64_t E, int64_t rows, int64_t cols, float* partials,
                              int64_t nparts_cap, float* q_out, void* w8, void* w8t, void* wbf16t, void* stream) {
  return weight_quant_batch(w, E, rows, cols, partials, nparts_cap, q_out, w8, w8t, wbf16t, (hipStream_t)stream);
}

int sfp8_block_weight_quant(const float* w_gu, int64_t gu_rows, int64_t gu_cols, const float* w_down, int64_t d_rows,
                            int64_t d_cols, float* partials, int64_t nparts_cap, float* q_out, void* w8, void* w8t,
                            void* wd8, void* wdt, float* scale, float* amax, void* stream) {
  if (!w_gu || !w_down || !partials || !q_out || !w8 || !w8t || !wd8 || !wdt || (!scale != !amax))
    return kErrNullPointer;
  if (gu_rows <= 0 || gu_cols <= 0 || d_rows <= 0 || d_cols <= 0 || gu_cols % 64 || gu_rows % 64 || d_cols % 64 ||
      d_rows % 32)
    return kErrBadShape;
  if (nparts_cap < 2 * WQ_PARTS) return kErrWorkspaceTooSmall;
  if (!aligned16(w_gu) || !aligned16(w_down)) return kErrBadAlignment;
  WeightPair p{};
  p.w[0] = w_gu;
  p.w[1] = w_down;
  p.R[0] = gu_rows;
  p.C[0] = gu_cols;
  p.R[1] = d_rows;
  p.C[1] = d_cols;
  p.partials = partials;
  for (int j = 0; j < 2; ++j) {
    int np = (int)((p.R[j] * p.C[j] / 4 + 255) / 256);
    p.nparts[j] = np > WQ_PARTS ? WQ_PARTS : (np < 1 ? 1 : np);
    p.tiles_r[j] = (int)((p.R[j] + 255) / 256 * 4);
    p.tiles_c[j] = (int)((p.C[j] + 255) / 256 * 4);
  }
  const int64_t ntiles = (int64_t)p.tiles_r[0] * p.tiles_c[0] + (int64_t)p.tiles_r[1] * p.tiles_c[1];
  if (ntiles > 0x7fffffff) return kErrBadShape;
  p.q_out = q_out;
  p.w8[0] = (uint8_t*)w8;
  p.w8[1] = (uint8_t*)wd8;
  p.w8t = (uint8_t*)w8t;
  p.wbt = (uint16_t*)wdt;
  p.scale = scale;
  p.amax = amax;
  const hipStream_t st = (hipStream_t)stream;
  const int gx = p.nparts[0] > p.nparts[1] ? p.nparts[0] : p.nparts[1];
  hipLaunchKernelGGL(weight_amax_pair_kernel, dim3(gx, 2), dim3(256), 0, st, p);
  hipLaunchKernelGGL(weight_quant_pair_kernel, dim3((unsigned)ntiles), dim3(256), 0, st, p);
  return launch_status();
}

int sfp8_update_scales(float* scale, float* amax, int64_t nsets, void* stream) {
  if (!scale || !amax) return kErrNullPointer;
  if (nsets < 0) return kErrBadShape;
  if (nsets == 0) return kOk;
  const int n = (int)(nsets * 5);
  hipLaunchKernelGGL(update_scales_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     scale, amax, (int)nsets, 1);
  return launch_status();
}

static int64_t norm_bwd_blocks(int64_t D, int64_t ldt) {
  switch (D) {
    case 128: return ldt / NormCfg<128>::RT;
    case 256: return ldt / NormCfg<256>::RT;
    case 512: return ldt / NormCfg<512>::RT;
    case 1024: return ldt / NormCfg<1024>::RT;
    case 2048: return ldt / NormCfg<2048>::RT;
    case 4096: return ldt / NormCfg<4096>::RT;
    default: return wide_hidden(D) ? ldt / kWideRows : -1;
  }
}

int64_t sfp8_norm_bwd_partials(int64_t D, int64_t ldt) {
  const int64_t nb = norm_bwd_blocks(D, ldt);
  return nb < 0 ? -1 : nb + colsum_groups(nb);
}

// Shared by sfp8_norm_bwd (caller's workspace) and sfp8_norm_bwd_noalloc
// (the fixed scratch); the arguments are checked by the callers.
static int norm_bwd_launch(const void* h, const float* rstd, const void* dxn, const void* dy, const float* norm_w,
                           int64_t T, int64_t D, const float* scale, float* amax, void* dh, float* dnw,
                           float* partials, void* dy8, void* dy8t, int64_t ldt, hipStream_t st) {
  if (ldt == 0) {
    // no tokens: d_norm_w is an empty sum (zero); nothing else is written
    hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)((D + 255) / 256)), dim3(256), 0, st, dnw, D);
    return launch_status();
  }
  switch (D) {
    case 128: return launch_norm_bwd<128>(h, rstd, dxn, dy, norm_w, T, scale, amax, dh, dnw, partials, dy8, dy8t, ldt, st);
    case 256: return launch_norm_bwd<256>(h, rstd, dxn, dy, norm_w, T, scale, amax, dh, dnw, partials, dy8, dy8t, ldt, st);
    case 512: return launch_norm_bwd<512>(h, rstd, dxn, dy, norm_w, T, scale, amax, dh, dnw, partials, dy8, dy8t, ldt, st);
    case 1024: return launch_norm_bwd<1024>(h, rstd, dxn, dy, norm_w, T, scale, amax, dh, dnw, partials, dy8, dy8t, ldt, st);
    case 2048: return launch_norm_bwd<2048>(h, rstd, dxn, dy, norm_w, T, scale, amax, dh, dnw, partials, dy8, dy8t, ldt, st);
    case 4096: return launch_norm_bwd<4096>(h, rstd, dxn, dy, norm_w, T, scale, amax, dh, dnw, partials, dy8, dy8t, ldt, st);
    default:
      if (wide_hidden(D)) return launch_norm_bwd_wide(h, rstd, dxn, dy, norm_w, T, D, scale, amax, dh, dnw, partials,
                                                     dy8, dy8t, ldt, st);
      return kErrBadShape;
  }
}

// Argument checks common to both norm backward entry points.
static int norm_bwd_check(const void* h, const float* rstd, const void* dxn, const void* dy, const float* norm_w,
                          int64_t T, int64_t D, const float* scale, float* amax, void* dh, float* dnw, void* dy8,
                          void* dy8t, int64_t ldt) {
  // dy8 and dy8t are each optional
  if (!norm_w || !scale || !amax || !dnw || (T > 0 && (!h || !rstd || !dxn || !dy || !dh)))
    return kErrNullPointer;
  if (T < 0 || ldt < T || (ldt % 256) != 0) return kErrBadShape;
  if (sfp8_norm_bwd_partials(D, ldt) < 0) return kErrBadShape;
  if (!aligned16(h) || !aligned16(dxn) || !aligned16(dy) || !aligned16(dh) || !aligned16(norm_w) ||
      !aligned16(dy8) || !aligned16(dy8t))
    return kErrBadAlignment;
  return kOk;
}

int sfp8_norm_bwd(const void* h, const float* rstd, const void* dxn, const void* dy, const float* norm_w,
                  int64_t T, int64_t D, const float* scale, float* amax, void* dh, float* dnw,
                  float* partials, int64_t partials_cap, void* dy8, void* dy8t, int64_t ldt, void* stream) {
  // token-sized buffers (and the partials) may be null when there are no tokens
  int rc = norm_bwd_check(h, rstd, dxn, dy, norm_w, T, D, scale, amax, dh, dnw, dy8, dy8t, ldt);
  if (rc) return rc;
  if (T > 0 && !partials) return kErrNullPointer;
  if (partials_cap < sfp8_norm_bwd_partials(D, ldt) * D) return kErrWorkspaceTooSmall;
  return norm_bwd_launch(h, rstd, dxn, dy, norm_w, T, D, scale, amax, dh, dnw, partials, dy8, dy8t, ldt,
                         (hipStream_t)stream);
}

int sfp8_norm_bwd_noalloc(const void* h, const float* rstd, const void* dxn, const void* dy, const float* norm_w,
                          int64_t T, int64_t D, const float* scale, float* amax, void* dh, float* dnw, void* dy8,
                          void* dy8t, int64_t ldt, void* stream) {
  int rc = norm_bwd_check(h, rstd, dxn, dy, norm_w, T, D, scale, amax, dh, dnw, dy8, dy8t, ldt);
  if (rc) return rc;
  // the dnw partials (every row of which the kernels write before reading:
  // nothing has to start at zero) must fit the fixed scratch
  if (sfp8_norm_bwd_partials(D, ldt) * D > kNoAllocScratchFloats) return kErrScratchLimit;
  float* partials = nullptr;
  rc = scratch_address(&partials);
  if (rc) return rc;
  return norm_bwd_launch(h, rstd, dxn, dy, norm_w, T, D, scale, amax, dh, dnw, partials, dy8, dy8t, ldt,
                         (hipStream_t)stream);
}

}  // extern "C"
