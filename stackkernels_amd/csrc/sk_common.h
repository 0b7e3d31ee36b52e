// Shared device helpers for the gfx950 attention kernels.
//
// Element storage is raw 16-bit words (bf16 or fp16) or fp32.  MFMA operands
// are 8 x 16-bit values per lane (one 128-bit register quad).  Layouts used by
// the kernels (checked on gfx950 hardware):
//
//   v_mfma_f32_32x32x16_{bf16,f16}: lane l supplies A[row l%32][k 8*(l/32)+e],
//     B[k 8*(l/32)+e][col l%32], e = 0..7; result register r of lane l is
//     C[row 8*(r/4) + 4*(l/32) + r%4][col l%32].
//   v_mfma_f32_16x16x32_{bf16,f16}: A[row l%16][k 8*(l/16)+e], B[k 8*(l/16)+e]
//     [col l%16]; result r is C[row 4*(l/16) + r][col l%16].
//   ds_read_b64_tr_b16: within each group of 16 lanes, lane j addresses 4
//     consecutive 16-bit words; lane i receives word (i%4) of lanes
//     4e + i/4 for e = 0..3.  If lane j points at row r0 + j/4, column
//     c0 + 4*(j%4) of a row-major tile, lane i receives column c0 + i of
//     rows r0..r0+3: a transposed 4 x 16 read.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// On a lambda whose callers pass it register arrays by reference: inlining
// keeps those arrays in registers.
#define SK_INLINE __attribute__((always_inline))

namespace sk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// Type tags for the two 16-bit element types.
struct BF16 {
  static constexpr int code = 2;
};
struct F16 {
  static constexpr int code = 1;
};

template <class T>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c);
template <>
__device__ __forceinline__ f32x16 mfma32<BF16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16 mfma32<F16>(u32x4 a, u32x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <class T>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c);
template <>
__device__ __forceinline__ f32x4 mfma16<BF16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4 mfma16<F16>(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// Two fp32 values -> one dword of two 16-bit values (round to nearest even).
template <class T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi);
template <>
__device__ __forceinline__ uint32_t pack2<BF16>(float lo, float hi) {
  f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}
template <>
__device__ __forceinline__ uint32_t pack2<F16>(float lo, float hi) {
  f32x2 f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
}

// 16-bit word -> fp32.
template <class T>
__device__ __forceinline__ float to_f32(uint16_t x);
template <>
__device__ __forceinline__ float to_f32<BF16>(uint16_t x) {
  return __builtin_bit_cast(float, (uint32_t)x << 16);
}
template <>
__device__ __forceinline__ float to_f32<F16>(uint16_t x) {
  return (float)__builtin_bit_cast(_Float16, x);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Online-softmax rescale threshold in log2 units: the running exponent offset
// is raised only when a score exceeds it by more than this, so unnormalised
// probabilities stay <= 2^8 (exact in bf16/fp16 range, no fp32 overflow).
constexpr float kRescaleLog2 = 8.0f;

// Work-item index for XCD-aware scheduling.  gfx950 dispatches workgroup i to
// XCD i % 8 (8 XCDs, each with its own L2); this maps the n workgroups so that
// XCD x processes the contiguous item range [start(x), start(x) + count(x)).
constexpr int kNumXcd = 8;
__device__ __forceinline__ int xcd_work_index(int bid, int n) {
  const int xcd = bid % kNumXcd;
  const int r = bid / kNumXcd;
  const int per = n / kNumXcd;
  const int rem = n % kNumXcd;
  return xcd * per + min(xcd, rem) + r;
}

// max / sum of a value across lanes l and l^32 of a wave64.  v_permlane32_swap
// with both operands x leaves, in every lane l, x[l % 32] in one result and
// x[l % 32 + 32] in the other (a VALU op, no LDS round trip).
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, x), false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, x), false, false);
  return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// Transposed 4 x 16 read from a row-major LDS tile (see header comment).
__device__ __forceinline__ u32x2 lds_read_tr(const uint16_t* p) {
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(u32x2, v);
}

__device__ __forceinline__ u32x4 lds_read_b128(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Raw buffer loads (gfx9 resource word 3 = 0x00020000: 32-bit untyped data).
// A load whose byte offset is not below the resource's num_records returns
// zero; kBufferOob is an offset that is out of range for every resource used
// here (all tiles are far smaller than 2 GiB).
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
constexpr uint32_t kBufferOob = 0x80000000u;

__device__ __forceinline__ buf_rsrc make_rsrc(const void* base, int num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, num_bytes,
                                           0x00020000);
}

// Bytes a resource must cover for `rows` rows of `d` elements at row stride
// `stride` elements (16-bit data): through the end of the last row's data.
__device__ __forceinline__ int tile_bytes(int rows, int64_t stride, int d) {
  return rows > 0 ? (int)(((int64_t)(rows - 1) * stride + d) * 2) : 0;
}

__device__ __forceinline__ u32x4 buffer_load_b128(buf_rsrc r, uint32_t offset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
}

// Buffer resource as four SGPR words, for inline asm operands.
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4 make_rsrc_words(const void* base, int num_bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  return i32x4{(int)(uint32_t)a, (int)((uint32_t)(a >> 32) & 0xffffu), num_bytes, 0x00020000};
}

// The four words with each read from the first active lane: for values that
// are wave-uniform but that the compiler cannot prove so.
__device__ __forceinline__ i32x4 uniform_words(i32x4 r) {
  return i32x4{__builtin_amdgcn_readfirstlane(r[0]), __builtin_amdgcn_readfirstlane(r[1]),
               __builtin_amdgcn_readfirstlane(r[2]), __builtin_amdgcn_readfirstlane(r[3])};
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16 bytes per lane from a buffer straight into LDS: lane i writes
// lds_wave_base + 16 * i (lds_wave_base must be wave-uniform).  Out-of-range
// lanes write zeros.  Completion is counted by vmcnt, and the caller owns the
// wait: issued as inline asm so the compiler does not add its own
// conservative vmcnt(0) before every later LDS read (its alias tracking of
// LDS DMA cannot tell the ring's stages apart).  s_nop covers the M0-write
// to LDS-DMA hazard.
__device__ __forceinline__ void buffer_load_lds_b128(i32x4 rsrc, uint32_t lds_wave_base,
                                                     uint32_t offset) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds"
      :
      : "s"(lds_wave_base), "v"(offset), "s"(rsrc)
      : "memory", "m0");
}

// buffer_load_lds_b128 with the non-temporal hint, for data read once
// (streamed past the caches' reuse).
__device__ __forceinline__ void buffer_load_lds_b128_nt(i32x4 rsrc, uint32_t lds_wave_base,
                                                        uint32_t offset) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen nt lds"
      :
      : "s"(lds_wave_base), "v"(offset), "s"(rsrc)
      : "memory", "m0");
}

// 4 bytes per lane from a buffer straight into LDS: lane i writes
// lds_wave_base + 4 * i.  Same contract as buffer_load_lds_b128.
__device__ __forceinline__ void buffer_load_lds_b32(i32x4 rsrc, uint32_t lds_wave_base,
                                                    uint32_t offset) {
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %1, %2, 0 offen lds"
      :
      : "s"(lds_wave_base), "v"(offset), "s"(rsrc)
      : "memory", "m0");
}

// s_waitcnt with vmcnt <= N and the other counters left open (gfx9 encoding:
// vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Wait until at most `ahead` tiles of LOADS vector-memory loads each are
// still in flight (ahead in [0, MAXA]; the count must be an immediate).
template <int LOADS, int MAXA>
__device__ __forceinline__ void wait_tiles(int ahead) {
  static_assert(LOADS * MAXA < 64, "vmcnt range");
  if constexpr (MAXA >= 6) { if (ahead >= 6) { wait_vmcnt<LOADS * 6>(); return; } }
  if constexpr (MAXA >= 5) { if (ahead == 5) { wait_vmcnt<LOADS * 5>(); return; } }
  if constexpr (MAXA >= 4) { if (ahead == 4) { wait_vmcnt<LOADS * 4>(); return; } }
  if constexpr (MAXA >= 3) { if (ahead == 3) { wait_vmcnt<LOADS * 3>(); return; } }
  if constexpr (MAXA >= 2) { if (ahead == 2) { wait_vmcnt<LOADS * 2>(); return; } }
  if constexpr (MAXA >= 1) { if (ahead == 1) { wait_vmcnt<LOADS>(); return; } }
  wait_vmcnt<0>();
}

__device__ __forceinline__ u32x4 ldg_b128(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 ldg_b128_cached(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

}  // namespace sk
