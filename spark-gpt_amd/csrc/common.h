// Shared device helpers for the gfx950 FP8 MLP kernels.
//
// Conventions used by every kernel in this library:
//  * FP8 is OCP e4m3fn / e5m2 (gfx950 hardware formats), bit-identical to
//    torch.float8_e4m3fn / torch.float8_e5m2.
//  * Every cast clamps first (to +-448 or +-57344) and keeps NaN, as the
//    reference does before each .to(fp8) (spark-gpt train.py:952, 968, 1013-1014,
//    1091-1092, 1172); the hardware converter then rounds to nearest even.
//  * amax slots are fp32 and are max-accumulated with an unsigned atomic max on
//    the bit pattern of |x| (exact and order independent for x >= 0).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SFP8_DEV __device__ __forceinline__

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx2 __attribute__((ext_vector_type(2)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

namespace sfp8 {

constexpr float kE4M3Max = 448.0f;
constexpr float kE5M2Max = 57344.0f;
// fp8 format selectors (the f8f6f4 MFMA's operand format fields use the same codes)
constexpr int kFmtE4M3 = 0;
constexpr int kFmtE5M2 = 1;
// Cache-policy operand of the buffer-load builtins: the nontemporal (nt) bit,
// for data a kernel reads once (streamed through the caches without
// displacing the lines other work-groups re-read).  Plain pointer loads of
// such data use __builtin_nontemporal_load, which sets the same bit.
constexpr int kNT = 2;

// Library status codes (hipError_t values are passed through unchanged and are
// all positive; ours are negative).
enum Status : int {
  kOk = 0,
  kErrNullPointer = -1,
  kErrBadShape = -2,
  kErrBadAlignment = -3,
  kErrWorkspaceTooSmall = -4,
  kErrScratchLimit = -5,  // the allocation-free entry point's fixed scratch is too small
};

SFP8_DEV float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet (torch semantics).
SFP8_DEV uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

SFP8_DEV float round_bf16(float f) { return __uint_as_float(f32_to_bf16_bits(f) << 16); }

// clamp that keeps NaN (comparisons with NaN are false)
SFP8_DEV float clamp_keep_nan(float x, float m) {
  x = (x > m) ? m : x;
  x = (x < -m) ? -m : x;
  return x;
}

// The gfx950 converters write an all-ones pattern (0xFF / 0xFE) for every NaN
// input; torch writes 0x7F with the input's sign bit.  NaNs are rare, so the
// fix-up runs only when one of the four inputs is NaN.
SFP8_DEV uint32_t fix_nan4(uint32_t p, float a, float b, float c, float d) {
  const float v[4] = {a, b, c, d};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (v[i] != v[i]) {
      const uint32_t code = 0x7Fu | ((__float_as_uint(v[i]) >> 24) & 0x80u);
      p = (p & ~(0xFFu << (8 * i))) | (code << (8 * i));
    }
  }
  return p;
}

SFP8_DEV bool any_nan4(float a, float b, float c, float d) {
  return (a != a) | (b != b) | (c != c) | (d != d);
}

// Four fp32 -> four e4m3 bytes packed little-endian (a = lowest byte).  The
// clamp is one v_med3 per value; the converter itself does not saturate.
SFP8_DEV uint32_t pack4_e4m3(float a, float b, float c, float d) {
  int v = 0;
  v = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(a, -kE4M3Max, kE4M3Max),
                                      __builtin_amdgcn_fmed3f(b, -kE4M3Max, kE4M3Max), v, false);
  v = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(c, -kE4M3Max, kE4M3Max),
                                      __builtin_amdgcn_fmed3f(d, -kE4M3Max, kE4M3Max), v, true);
  uint32_t p = (uint32_t)v;
  if (__builtin_expect(any_nan4(a, b, c, d), 0)) p = fix_nan4(p, a, b, c, d);
  return p;
}

// pack4_e4m3 without the NaN fix-up: NaN inputs come out as the code of -448
// (v_med3 maps NaN to the low bound); callers patch them with fix_nan4 on a
// wave-uniform rare path.
SFP8_DEV uint32_t pack4_e4m3_nofix(float a, float b, float c, float d) {
  int v = 0;
  v = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(a, -kE4M3Max, kE4M3Max),
                                      __builtin_amdgcn_fmed3f(b, -kE4M3Max, kE4M3Max), v, false);
  v = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(c, -kE4M3Max, kE4M3Max),
                                      __builtin_amdgcn_fmed3f(d, -kE4M3Max, kE4M3Max), v, true);
  return (uint32_t)v;
}

// gfx950 LDS transpose read (ds_read_b64_tr_b8).  Within each group of 16
// lanes, lane i receives byte (i % 8) of the 8-byte rows addressed by the
// group's lanes 2b + i/8, b = 0..7, as its byte b.  With lane 2b + h pointing
// at row R + b, columns C + 8h .. C + 8h + 7 of a byte matrix, lane i gets
// rows R .. R+7 of column C + i.
SFP8_DEV intx2 lds_read_tr8(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) intx2*)p);
}

// ds_read_b64_tr_b16: in each 16-lane group, lane 4a + b receives element b
// of the 4 16-bit elements addressed by lanes a, a + 4, a + 8, a + 12.
SFP8_DEV intx2 lds_read_tr16(const uint8_t* p) {
  typedef short shortx4 __attribute__((ext_vector_type(4)));
  const shortx4 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) shortx4*)p);
  return __builtin_bit_cast(intx2, t);
}

SFP8_DEV uint32_t pack4_e5m2(float a, float b, float c, float d) {
  int v = 0;
  v = __builtin_amdgcn_cvt_pk_bf8_f32(__builtin_amdgcn_fmed3f(a, -kE5M2Max, kE5M2Max),
                                      __builtin_amdgcn_fmed3f(b, -kE5M2Max, kE5M2Max), v, false);
  v = __builtin_amdgcn_cvt_pk_bf8_f32(__builtin_amdgcn_fmed3f(c, -kE5M2Max, kE5M2Max),
                                      __builtin_amdgcn_fmed3f(d, -kE5M2Max, kE5M2Max), v, true);
  uint32_t p = (uint32_t)v;
  if (__builtin_expect(any_nan4(a, b, c, d), 0)) p = fix_nan4(p, a, b, c, d);
  return p;
}

// Scaled conversions: bytes of e4m3/e5m2(clamp(x * m)) for a power-of-two m,
// given inv_m = 1/m and bound = fmax/m.  Clamping x to +-bound before the
// scaling is the same as clamping x*m to +-fmax because m is a power of two;
// the converter divides by its scale operand.  NaN inputs are left to the
// caller (med3 maps NaN to -bound).
typedef short shortx2 __attribute__((ext_vector_type(2)));

template <bool HI>
SFP8_DEV uint32_t pack2_e4m3_scaled(uint32_t old, float a, float b, float inv_m, float bound) {
  const shortx2 o = __builtin_bit_cast(shortx2, old);
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(
      o, __builtin_amdgcn_fmed3f(a, -bound, bound), __builtin_amdgcn_fmed3f(b, -bound, bound), inv_m, HI));
}

template <bool HI>
SFP8_DEV uint32_t pack2_e5m2_scaled(uint32_t old, float a, float b, float inv_m, float bound) {
  const shortx2 o = __builtin_bit_cast(shortx2, old);
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(
      o, __builtin_amdgcn_fmed3f(a, -bound, bound), __builtin_amdgcn_fmed3f(b, -bound, bound), inv_m, HI));
}

SFP8_DEV uint32_t pack4_e4m3_scaled(float a, float b, float c, float d, float inv_m, float bound) {
  return pack2_e4m3_scaled<true>(pack2_e4m3_scaled<false>(0u, a, b, inv_m, bound), c, d, inv_m, bound);
}

SFP8_DEV uint32_t pack4_e5m2_scaled(float a, float b, float c, float d, float inv_m, float bound) {
  return pack2_e5m2_scaled<true>(pack2_e5m2_scaled<false>(0u, a, b, inv_m, bound), c, d, inv_m, bound);
}

// The same without the clamp, for callers that have checked every input is
// finite and within +-bound (the clamp is then the identity).  Both halves
// of `any` are overwritten; passing a live register saves zeroing one.
SFP8_DEV uint32_t pack4_e5m2_scaled_noclamp(float a, float b, float c, float d, float inv_m, uint32_t any) {
  shortx2 o = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(__builtin_bit_cast(shortx2, any), a, b, inv_m, false);
  o = __builtin_amdgcn_cvt_scalef32_pk_bf8_f32(o, c, d, inv_m, true);
  return __builtin_bit_cast(uint32_t, o);
}

SFP8_DEV uint32_t pack4_e4m3_scaled_noclamp(float a, float b, float c, float d, float inv_m, uint32_t any) {
  shortx2 o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(__builtin_bit_cast(shortx2, any), a, b, inv_m, false);
  o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, c, d, inv_m, true);
  return __builtin_bit_cast(uint32_t, o);
}

// max(a, b, c) that returns NaN when any input is NaN (v_maximum3_f32).
SFP8_DEV float max3_nan(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

// Two fp32 -> two bf16 (hardware round-to-nearest-even), packed lo/hi.
SFP8_DEV uint32_t pack2_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(floatx2{a, b}, bf16x2_t));
}

// Round two fp32 values to bf16 precision (returned as fp32).
SFP8_DEV void round2_bf16(float& a, float& b) {
  const uint32_t p = pack2_bf16(a, b);
  a = __uint_as_float(p << 16);
  b = __uint_as_float(p & 0xffff0000u);
}

// Logistic sigmoid with the hardware exp2 / reciprocal (about 1 ulp each).
SFP8_DEV float sigmoid_fast(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// The Muon momentum stage of four elements (train.py:2805-2820): v <- lerp(v,
// g, w_v) (torch.lerp's weight < 0.5 form), u = bf16(lerp(g, v, 1 - w_u1))
// (its weight >= 0.5 form), each lerp one fused multiply-add as torch's GPU
// lerp evaluates it.  w_u1 = 1 - w_u.
SFP8_DEV void momentum4(const floatx4& g, floatx4& v, float w_v, float w_u1, uint32_t (&u)[2]) {
  floatx4 vn, un;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    vn[i] = __builtin_fmaf(w_v, g[i] - v[i], v[i]);
    un[i] = __builtin_fmaf(-(vn[i] - g[i]), w_u1, vn[i]);
  }
  v = vn;
  u[0] = pack2_bf16(un[0], un[1]);
  u[1] = pack2_bf16(un[2], un[3]);
}

// fp8 byte -> fp32 (exact).  Hardware converter on gfx950.
SFP8_DEV float e4m3_to_f32(uint32_t word, int byte) {
  switch (byte) {
    case 0: return __builtin_amdgcn_cvt_f32_fp8(word, 0);
    case 1: return __builtin_amdgcn_cvt_f32_fp8(word, 1);
    case 2: return __builtin_amdgcn_cvt_f32_fp8(word, 2);
    default: return __builtin_amdgcn_cvt_f32_fp8(word, 3);
  }
}

SFP8_DEV float e5m2_to_f32(uint32_t word, int byte) {
  switch (byte) {
    case 0: return __builtin_amdgcn_cvt_f32_bf8(word, 0);
    case 1: return __builtin_amdgcn_cvt_f32_bf8(word, 1);
    case 2: return __builtin_amdgcn_cvt_f32_bf8(word, 2);
    default: return __builtin_amdgcn_cvt_f32_bf8(word, 3);
  }
}

SFP8_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

SFP8_DEV double wave_sum_f64(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

SFP8_DEV float wave_sum_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// |x| is non-negative, so the unsigned order of its bits is the float order
// (NaN patterns sort above +inf, so a NaN amax sticks, as torch.amax would).
SFP8_DEV void atomic_max_nonneg(float* addr, float v) {
  // An amax slot only grows within a kernel, so a read of it is never above
  // its current value: when it already holds >= v the atomic is skipped.  (A
  // stale low read costs one unneeded atomic, never a lost maximum.)  This
  // keeps thousands of work-groups from serialising on one L2 address.
  const unsigned int u = __float_as_uint(v);
  if (u > *reinterpret_cast<volatile unsigned int*>(addr)) atomicMax(reinterpret_cast<unsigned int*>(addr), u);
}

// Work-group max of a non-negative value; one atomic per work-group.
// `red` must hold one float per wave.
template <int NWAVES>
SFP8_DEV void block_amax_atomic(float v, float* red, float* dst) {
  v = wave_max(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = red[0];
#pragma unroll
    for (int i = 1; i < NWAVES; ++i) m = fmaxf(m, red[i]);
    atomic_max_nonneg(dst, m);
  }
}

// The same for a caller that holds its wave index in a scalar register: the
// lane index is recomputed (mbcnt), so the work-item id need not stay live
// to the kernel's end.
template <int NWAVES>
SFP8_DEV void block_amax_atomic_w(float v, float* red, float* dst, int wid_s) {
  v = wave_max(v);
  const bool lane0 = __lane_id() == 0;
  if (lane0) red[wid_s] = v;
  __syncthreads();
  if (lane0 && wid_s == 0) {
    float m = red[0];
#pragma unroll
    for (int i = 1; i < NWAVES; ++i) m = fmaxf(m, red[i]);
    atomic_max_nonneg(dst, m);
  }
}

// K-slab layout of a token-contiguous FP8 copy of an R-row operand (the weight
// gradients' operands x8t, h8t, d_gu8t, dy8t): [ldt / 64][slab_rows(R)][64]
// bytes, element (r, t) at
//   (t / 64) * slab_rows(R) * 64 + r * 64 + t % 64.
// One 64-token K stage of a 256-row GEMM tile is then one contiguous 16 KiB
// block.  Rows are padded to a multiple of 256 (the tile), so every tile read
// stays inside the buffer; padding rows only feed discarded output rows.
__host__ __device__ inline int64_t slab_rows(int64_t R) { return (R + 255) / 256 * 256; }

// Writes a 256-token LDS tile of NC16 * 16 columns (row stride `stride`
// bytes) into a K-slab copy through transposing LDS reads:
//   out(c0 + c, t0 + t) = tile[t][c]  for t < 256, c < NC16 * 16.
// Every tile row is copied (callers keep zero codes in rows past the last
// token); t0 % 64 == 0.  The 16-lane group q of a wave turns a 16 x 16 byte
// block into 16 column runs of 16 tokens (two ds_read_b64_tr_b8), and the
// four groups take consecutive 16-token blocks, so each wave store covers 16
// whole 64-byte slab rows.  Work unit u (64-token block u % 4, 16-column
// block u / 4) goes to wave u % NW (NW = waves in the work-group, 4 or 8).
template <int NC16, int NW = 4>
SFP8_DEV void lds_tile_store_slab_tr(const uint8_t* lds, int stride, uint8_t* out, int64_t rpad, int64_t t0,
                                     int64_t c0) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4, li = lane & 15;
#pragma unroll 4
  for (int p = 0; p < NC16 * 4 / NW; ++p) {
    const int u = p * NW + wave;
    const int r = 64 * (u & 3) + 16 * q, c = 16 * (u >> 2);
    const uint8_t* src = lds + (r + (li >> 1)) * stride + c + 8 * (li & 1);
    const intx2 a = lds_read_tr8(src);
    const intx2 b = lds_read_tr8(src + 8 * stride);
    const int64_t t = t0 + r;
    *reinterpret_cast<intx4*>(out + (t >> 6) * rpad * 64 + (c0 + c + li) * 64 + (t & 63)) =
        intx4{a[0], a[1], b[0], b[1]};
  }
}

// The same for an LDS tile of NTOK = 16, 32 or 64 tokens and ncols columns
// (ncols % 64 == 0, t0 % NTOK == 0): NTOK / 16 lane groups take the token
// blocks of one 16-column block, so a wave store covers 64 / NTOK * 16 slab
// rows of NTOK bytes each (whole 64-byte rows when NTOK = 64).  NW = waves
// in the work-group.
template <int NTOK, int NW = 4>
SFP8_DEV void lds_rows_store_slab_tr(const uint8_t* lds, int ncols, int stride, uint8_t* out, int64_t rpad,
                                     int64_t t0, int64_t c0) {
  static_assert(NTOK == 16 || NTOK == 32 || NTOK == 64, "16, 32 or 64 tokens");
  constexpr int G = NTOK / 16;  // 16-token blocks per column block
  constexpr int CB = 4 / G;     // column blocks per wave pass
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane >> 4, li = lane & 15;
  const int r = 16 * (q % G);
  const int64_t t = t0 + r;
  uint8_t* dst = out + (t >> 6) * rpad * 64 + (t & 63);
  const int passes = ncols / (16 * CB);
  for (int u = wave; u < passes; u += NW) {
    const int c = 16 * (u * CB + q / G);
    const uint8_t* src = lds + (r + (li >> 1)) * stride + c + 8 * (li & 1);
    const intx2 a = lds_read_tr8(src);
    const intx2 b = lds_read_tr8(src + 8 * stride);
    *reinterpret_cast<intx4*>(dst + (c0 + c + li) * 64) = intx4{a[0], a[1], b[0], b[1]};
  }
}

// The rows t0 .. t0 + NTOK - 1 of an LDS tile (NTOK rows of ncols bytes,
// ncols % 64 == 0, `stride` bytes apart) into the K-slab [L/64][ldt][64] of a
// token-major activation, columns c0 .. c0 + ncols - 1 (c0 % 64 == 0): each
// 64-column block of the tile is one contiguous NTOK * 64-byte run of the
// slab, written 16 bytes per lane.  NW = waves in the work-group.
template <int NTOK, int NW = 4>
SFP8_DEV void lds_rows_store_slab(const uint8_t* lds, int ncols, int stride, uint8_t* out, int64_t ldt, int64_t t0,
                                  int64_t c0) {
  const int pieces = (ncols >> 6) * NTOK * 4;
  for (int i = threadIdx.x; i < pieces; i += 64 * NW) {
    const int ch = i & 3, r = (i >> 2) % NTOK, k = (i >> 2) / NTOK;
    const intx4 v = *reinterpret_cast<const intx4*>(lds + r * stride + 64 * k + 16 * ch);
    *reinterpret_cast<intx4*>(out + ((c0 >> 6) + k) * ldt * 64 + (t0 + r) * 64 + 16 * ch) = v;
  }
}

// ---------------------------------------------------------------------------
// MoE plan: the expert-order rows of a grouped (MoE) layer in "padded expert
// order", every expert's rows starting on a 256-row boundary, so that each
// 256-row GEMM tile belongs to one expert.  Tile t covers padded rows
// 256t .. 256t + 255.  The plan is an int32 array written on the device
// from the experts' inclusive row-count prefix sums (no host sync):
//   [0] NT, the number of tiles; [1] E
//   [kPlanHdr + e]          padded start row of expert e (a multiple of 256)
//   [kPlanHdr + E + e]      padded row count of expert e (a multiple of 256)
//   [kPlanHdr + 2E + 3t]    tile t: expert, first unpadded row, valid rows
constexpr int kPlanHdr = 8;

__host__ __device__ inline int64_t moe_max_tiles(int64_t R, int64_t E) { return (R + 255) / 256 + E; }
__host__ __device__ inline int64_t moe_plan_ints(int64_t R, int64_t E) {
  return kPlanHdr + 2 * E + 3 * moe_max_tiles(R, E);
}

struct MoePlan {
  const int* p;
  SFP8_DEV int ntiles() const { return p[0]; }
  SFP8_DEV int experts() const { return p[1]; }
  SFP8_DEV int pstart(int e) const { return p[kPlanHdr + e]; }
  SFP8_DEV int pcount(int e) const { return p[kPlanHdr + experts() + e]; }
  SFP8_DEV int expert(int t) const { return p[kPlanHdr + 2 * experts() + 3 * t]; }
  SFP8_DEV int urow(int t) const { return p[kPlanHdr + 2 * experts() + 3 * t + 1]; }
  SFP8_DEV int rows(int t) const { return p[kPlanHdr + 2 * experts() + 3 * t + 2]; }
};

}  // namespace sfp8
