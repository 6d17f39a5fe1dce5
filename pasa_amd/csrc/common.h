// Shared device-side definitions for the gfx950 PISA-PG kernels.
//
// Layout conventions used by K2 and K4:
//  * 16-byte "chunks": 8 bf16 values.  LDS tiles use PadTile (padded rows,
//    even-first chunk order), which keeps the MFMA operand reads of 16
//    consecutive rows conflict-free and makes a lane's successive k-step reads
//    immediate offsets from one base address.
//  * Transposed tiles ([feature][token]) additionally permute tokens inside
//    each 16-token group (tok_perm), so that the 8 tokens one lane feeds to a
//    32x32x16 MFMA as its A-operand slots are one contiguous 16-byte chunk.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pasa {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// ---- bf16 helpers ---------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN kept quiet); returns the 16 bits.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  __bf16 b = (__bf16)f;
  return (uint32_t)__builtin_bit_cast(uint16_t, b);
}

// Two floats -> two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32; lo in bits 0-15.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// Unpack one 16-byte chunk of 8 bf16 into fp32.
__device__ __forceinline__ void unpack8(const uint4& c, float* out) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& c) {
  return __builtin_bit_cast(bf16x8_t, c);
}

// ---- buffer loads ------------------------------------------------------------
// A raw buffer resource over [base, base + bytes): loads whose byte range lies
// beyond `bytes` return zeros in hardware, which pads ragged last blocks
// without branches.  Offsets are 32-bit, so one resource covers one slice.
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint4 buf_load16(rsrc_t r, uint32_t byte_off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
  return uint4{v[0], v[1], v[2], v[3]};
}

// Bounds-checked direct load into LDS (buffer_load_dwordx4 ... lds): lane l's
// 16 bytes at byte_off land at lds_addr + 16*l (lds_addr wave-uniform); lanes
// whose range lies outside the resource write zeros.  Issued as inline assembly,
// for schedules that manage vmcnt themselves: the compiler then does not track
// these loads, so it neither drains them before unrelated LDS reads nor counts
// them in its own waits (which remain correct, as extra loads in flight only make
// them conservative).  m0 is a reserved register, so naming it as a clobber has
// no effect (the compiler warns and ignores it); what keeps this safe is that no
// kernel using this load contains a compiler-generated m0 user (its own LDS-direct
// builtin, s_sendmsg, v_movrel ...) whose hoisted m0 value this would overwrite.
// tests/test_m0_usage.py checks the compiled kernels for exactly that.
// rsrc: buffer descriptor words; lds_addr: LDS byte address (wave-uniform).
__device__ __forceinline__ void dma_load16_lds(u32x4_t rsrc, uint32_t lds_addr, uint32_t byte_off,
                                               uint32_t soff) {
  // m0 is set here on every use; it is a reserved register (the compiler keeps no
  // value in it across this statement), and the kernels calling this issue no
  // compiler-generated LDS-direct loads.  An LDS-direct load that reads m0 right
  // after an SALU write of it needs one wait state on gfx9-family chips (the compiler
  // pads its own such pairs with s_nop 0, but cannot see inside inline assembly):
  // without it the load may take the previous m0 and write its data over the
  // previous load's LDS destination when the wave issues unimpeded.
  // lds_addr and soff must be wave-uniform; readfirstlane puts them in SGPRs.
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(byte_off), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory");
}

// The same load with the nontemporal cache policy (nt), for data read exactly once: it
// streams through L2 instead of displacing lines other kernels or workgroups reuse.
__device__ __forceinline__ void dma_load16_lds_nt(u32x4_t rsrc, uint32_t lds_addr, uint32_t byte_off,
                                                  uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen nt lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(byte_off), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory");
}

// buf_load16 with the nontemporal cache policy (cache-policy operand bit 1: nt on gfx950).
__device__ __forceinline__ uint4 buf_load16_nt(rsrc_t r, uint32_t byte_off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 2);
  return uint4{v[0], v[1], v[2], v[3]};
}

// Workgroup barrier without a memory fence, so in-flight direct-to-LDS tile loads
// are not drained (a fenced __syncthreads would wait for them).  It is used only
// where this wave's preceding LDS reads have been consumed by MFMAs, i.e. have
// completed, and where the next LDS writes are direct loads issued after it.
__device__ __forceinline__ void barrier_lds_reads_done() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads have returned
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");       // no LDS access moves across the barrier
}

// vmcnt-only wait (expcnt / lgkmcnt left unconstrained), gfx9 s_waitcnt encoding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ __forceinline__ u32x4_t make_rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return (u32x4_t){(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// ---- LDS tile layouts -----------------------------------------------------

// Padded tile of bf16 rows with COLS columns.  Row stride is COLS*2 + 16 bytes,
// so 16 consecutive rows start on 16 distinct 16-byte bank groups, and the
// 16-byte chunks of a row are stored even-first (chunk c at position
// (c & 1) * COLS/16 + c/2).  A half-wavefront (h = lane / 32) reads chunks
// h, h+2, h+4, ... over consecutive MFMA k-steps, which are therefore
// contiguous: lane base + 16 * ks, an immediate offset.
template <int COLS>
struct PadTile {
  static constexpr int ROW_BYTES = COLS * 2 + 16;
  static constexpr int HALF = COLS / 16;
  __host__ __device__ static constexpr int chunk_pos(int c) { return (c & 1) * HALF + (c >> 1); }
  __host__ __device__ static constexpr int chunk_byte(int row, int c) {
    return row * ROW_BYTES + chunk_pos(c) * 16;
  }
  __host__ __device__ static constexpr int elem_byte(int row, int col) {
    return chunk_byte(row, col >> 3) + (col & 7) * 2;
  }
  // Byte offset of the k-step-0 chunk a lane of half h reads from `row`.
  __host__ __device__ static constexpr int frag_base(int row, int h) {
    return row * ROW_BYTES + h * HALF * 16;
  }
  static constexpr int bytes(int rows) { return rows * ROW_BYTES; }
};

// Token permutation inside each 16-token group: swap bits 2 and 3.  Applied to
// the token axis of transposed tiles ([feature][token]) so that the 8 tokens a
// lane feeds to one 32x32x16 MFMA as its A-operand slots (tokens
// 16s + 4h + {0..3} and 16s + 8 + 4h + {0..3}) form one 16-byte chunk.
__host__ __device__ __forceinline__ constexpr int tok_perm(int t) {
  return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1);
}

template <typename T>
__device__ __forceinline__ T lds_ld(const unsigned char* base, int byte_off) {
  return *reinterpret_cast<const T*>(base + byte_off);
}
template <typename T>
__device__ __forceinline__ void lds_st(unsigned char* base, int byte_off, const T& v) {
  *reinterpret_cast<T*>(base + byte_off) = v;
}

// ---- MFMA -----------------------------------------------------------------

// D(32x32, fp32) += A(32x16) * B(16x32), bf16 inputs.
// A: lane l holds A[l%32][8*(l/32) .. +7]; B: lane l holds B[8*(l/32) .. +7][l%32];
// D: lane l, element r holds D[8*(r/4) + 4*(l/32) + r%4][l%32].
__device__ __forceinline__ f32x16_t mfma32(const bf16x8_t& a, const bf16x8_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row of the 32x32 D tile held by element r of a lane in half h (= lane / 32).
__device__ __forceinline__ int mfma32_row(int r, int h) { return 8 * (r >> 2) + 4 * h + (r & 3); }

// ---- 16-bit element types of the attention path --------------------------------
// The D = 128 kernels take their q, k, v (and write o and the phase-2 pack) in bf16 or
// fp16; everything else (statistics, scores, accumulation) is fp32.  Each type gives
// its 8-element MFMA operand, the 32x32x16 MFMA, round-to-nearest-even packing of two
// floats, and the widening of 8 packed values.
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

struct Bf16 {
  using vec8 = bf16x8_t;
  static constexpr uint32_t kOne2 = 0x3F803F80u;  // two 1.0s
  __device__ static __forceinline__ f32x16_t mfma(const vec8& a, const vec8& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  // D(16x16) += A(16x32) * B(32x16): lane l holds A[l%16][8(l/16) .. +7] and
  // B[8(l/16) .. +7][l%16]; element i of D is D[4(l/16) + i][l%16].
  __device__ static __forceinline__ f32x4_t mfma16(const vec8& a, const vec8& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
  __device__ static __forceinline__ uint32_t bits(float x) { return f32_to_bf16_bits(x); }
  __device__ static __forceinline__ void widen8(const uint4& c, float* out) { unpack8(c, out); }
};

struct F16 {
  using vec8 = f16x8_t;
  static constexpr uint32_t kOne2 = 0x3C003C00u;
  __device__ static __forceinline__ f32x16_t mfma(const vec8& a, const vec8& b, const f32x16_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ f32x4_t mfma16(const vec8& a, const vec8& b, const f32x4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2_t));
  }
  __device__ static __forceinline__ uint32_t bits(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
  }
  __device__ static __forceinline__ void widen8(const uint4& c, float* out) {
    const f16x8_t h = __builtin_bit_cast(f16x8_t, c);
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (float)h[i];
  }
};

template <typename E>
__device__ __forceinline__ typename E::vec8 as_vec8(const uint4& c) {
  return __builtin_bit_cast(typename E::vec8, c);
}
template <typename E>
__device__ __forceinline__ typename E::vec8 as_vec8(const u32x4_t& c) {
  return __builtin_bit_cast(typename E::vec8, c);
}

// ---- wave helpers -----------------------------------------------------------

__device__ __forceinline__ float xor32(float x) {
  return __shfl_xor(x, 32, 64);
}

// max / sum of x over lanes l and l ^ 32, identical on both lanes
// (v_permlane32_swap exchanges the two wave halves in the VALU).
__device__ __forceinline__ float halves_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// max / sum of x over the four lanes l % 16 + 16 g (g = 0 .. 3), identical on all four:
// the 32-lane swap pairs g with g ^ 2, then the 16-lane swap pairs g with g ^ 1, and each
// step combines the two values in the same order on both lanes of the pair.
__device__ __forceinline__ float quad16_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float quad16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

// No v_dot2c_f32_bf16 (or other dot instructions) in MFMA kernels: on gfx950 a dot
// instruction issues only between the MFMAs of the SIMD's other waves, so it stalls
// its own wave for the length of the other wave's MFMA stream (measured: 16 dot2c
// next to an MFMA-bound wave take 252 cycles against 140 alone, while fma, exp, max3,
// cvt_pk, mul, add and permlane32_swap overlap the MFMAs at full rate).

// ds_read_b64_tr_b16: within each group of 16 lanes, the 64-bit loads of lanes
// 4r..4r+3 form row r (16 consecutive 16-bit elements) of a 4 x 16 block, and
// lane i of the group receives column i: {row0[i], row1[i], row2[i], row3[i]}.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const unsigned char* base, int byte_off) {
  typedef __attribute__((address_space(3))) s16x4_t* lds_v4_ptr;
  const s16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4_ptr)(base + byte_off));
  return __builtin_bit_cast(uint2, r);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
  return x;
}

// The same butterfly as wave_sum (x += x[lane ^ m], m = 32, 16, ..., 1: each step adds
// the same pair of partial sums, so the result is bit-identical), with one cross-lane
// primitive per step instead of an address computation and ds_bpermute: the permlane
// swaps exchange wave halves / 16-lane rows in the VALU, ds_swizzle's bitmask mode
// xors the lane id within 32 lanes, and DPP quad_perm xors it within 4.
__device__ __forceinline__ float wave_sum_xor(float x) {
  {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), (8 << 10) | 0x1F));
  x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), (4 << 10) | 0x1F));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));  // xor 2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));  // xor 1
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One fp32 operation, rounded to nearest even and never fused with a neighbour into an
// FMA.  hipcc contracts a*b+c by default, and HIP's __fmul_rn / __fadd_rn are plain
// operators in headers compiled that way; the pragma inside these helpers keeps the
// steps apart after inlining.  __builtin_sqrtf is the correctly rounded square root
// (__fsqrt_rn lowers to the approximate v_sqrt_f32 on this toolchain).
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}
__device__ __forceinline__ float div_rn(float a, float b) {
#pragma clang fp contract(off)
  return a / b;
}
__device__ __forceinline__ float sqrt_rn(float a) { return __builtin_sqrtf(a); }

// ---- token-major view of a frame-major slice ---------------------------------
// The HunyuanVideo placement (svg/models/hyvideo/placement.py:73-100): logical row
// r = p*F + f of the first F*P rows (token p of frame f, token-major) is stored at
// row f*P + p (frame-major); rows from F*P on (the text tail) are in place.  Heads
// whose flag is 0 are stored token-major already (identity).
struct RowMap {
  int F;                    // frames
  int P;                    // tokens per frame
  float invF;               // 1 / F
  const int32_t* temporal;  // per head; nullptr: every head permuted
  int heads;                // slice s is head s % heads
};

// Stored row of logical row r (F*P <= 2^24, so p = r / F is exact up to one step).
__device__ __forceinline__ int map_row(int r, const RowMap& m) {
  if (r >= m.F * m.P) return r;
  int p = (int)((float)r * m.invF);
  int f = r - p * m.F;
  if (f < 0) {
    --p;
    f += m.F;
  } else if (f >= m.F) {
    ++p;
    f -= m.F;
  }
  return f * m.P + p;
}

// Whether slice bh is permuted (uniform: a scalar load of the head's flag).
__device__ __forceinline__ bool slice_permuted(const RowMap& m, int bh) {
  if (m.temporal == nullptr) return true;
  typedef const __attribute__((address_space(4))) int32_t* const_i32_ptr;
  return ((const_i32_ptr)m.temporal)[bh % m.heads] != 0;
}

}  // namespace pasa
