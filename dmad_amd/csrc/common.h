// Shared device helpers for the gfx950 (CDNA4) attention kernels.
//
// Everything here is written for one target: wave64, MFMA 32x32x16 on bf16/fp16
// operands with fp32 accumulation, buffer resources with hardware range checks,
// and direct buffer->LDS loads of 16 bytes per lane.
//
// MFMA 32x32x16 register layouts (checked on the device with a lane probe):
//   A (M x K = 32 x 16): lane l holds row l%32, k = 8*(l/32) + e, e = 0..7
//   B (K x N = 16 x 32): lane l holds col l%32, k = 8*(l/32) + e
//   C (M x N = 32 x 32): lane l holds col l%32, rows 8*(v/4) + 4*(l/32) + v%4, v = 0..15
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dmad {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kWave = 64;
constexpr unsigned kRsrcWord3 = 0x00020000u;  // raw buffer, gfx9 family

// ---------------------------------------------------------------- buffers
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kRsrcWord3);
}

// 16-byte load; bytes at or beyond the range of the resource read as zero.
__device__ __forceinline__ i32x4_t buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
}

typedef __attribute__((address_space(3))) char lds_char_t;
typedef __attribute__((address_space(3))) const i32x4_t lds_i32x4_t;
typedef __attribute__((address_space(3))) const f32x4_t lds_f32x4_t;

// 16 bytes per lane straight into LDS: lane i lands at lds_base + 16*i.
__device__ __forceinline__ void buf_load16_lds(__amdgpu_buffer_rsrc_t r, lds_char_t* lds_base, uint32_t voff,
                                               uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds_base, 16, (int)voff, (int)soff, 0, 0);
}
__device__ __forceinline__ void buf_load16_lds(__amdgpu_buffer_rsrc_t r, void* lds_base, uint32_t voff,
                                               uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds_base, 16, (int)voff, (int)soff, 0, 0);
}

__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, i32x4_t v, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)voff, (int)soff, 0);
}
// 16-byte store of data the next kernel reads once (sc0 sc1 nt: system-scope
// write-through, non-temporal). For the score tiles of the backward's key pass
// this cost the pass 15% less time than a default-policy store.
__device__ __forceinline__ void buf_store16_stream(__amdgpu_buffer_rsrc_t r, i32x4_t v, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)voff, (int)soff, 19);
}

__device__ __forceinline__ void buf_store8(__amdgpu_buffer_rsrc_t r, u32x2_t v, uint32_t voff) {
  i32x2_t w = {(int)v[0], (int)v[1]};
  __builtin_amdgcn_raw_buffer_store_b64(w, r, (int)voff, 0, 0);
}

// vmcnt(0): wait for this wave's outstanding vector-memory operations
// (including buffer->LDS transfers). expcnt and lgkmcnt are left unconstrained.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// vmcnt(N): all but this wave's N most recent vector-memory operations are done.
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Workgroup barrier for a buffer->LDS ring: first vmcnt(N) lgkmcnt(0) (this
// wave's LDS reads have returned and all but its N most recent vector-memory
// requests have landed), then s_barrier. No memory fence is emitted (a fence
// would wait for every in-flight buffer->LDS request, including the ones meant
// to stay in flight); the asm memory clobber keeps the compiler from moving
// memory accesses across the barrier.
template <int N>
__device__ __forceinline__ void ring_sync() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit field");
  __builtin_amdgcn_s_waitcnt(0x0070 | (N & 15) | ((N >> 4) << 14));
  asm volatile("s_barrier" ::: "memory");
}

// ---------------------------------------------------------------- element types
template <typename T> struct Elem;
template <> struct Elem<__bf16> {
  using vec8 = bf16x8_t;
  // two floats -> two bf16 (round to nearest even), packed low|high
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t r;
    r[0] = (__bf16)a;
    r[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ __forceinline__ static float to_f32(uint16_t bits) {
    return __uint_as_float(((uint32_t)bits) << 16);
  }
  // x rounded to bf16 (nearest even) and widened back
  __device__ __forceinline__ static float round(float x) { return (float)(__bf16)x; }
};
template <> struct Elem<_Float16> {
  using vec8 = f16x8_t;
  __device__ __forceinline__ static uint32_t pack2(float a, float b) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    f16x2_t r;
    r[0] = (_Float16)a;
    r[1] = (_Float16)b;
    return __builtin_bit_cast(uint32_t, r);
  }
  __device__ __forceinline__ static float to_f32(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
  }
  __device__ __forceinline__ static float round(float x) { return (float)(_Float16)x; }
};

__device__ __forceinline__ f32x16_t mfma32(i32x4_t a, i32x4_t b, f32x16_t c, __bf16) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}
__device__ __forceinline__ f32x16_t mfma32(i32x4_t a, i32x4_t b, f32x16_t c, _Float16) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                c, 0, 0, 0);
}

// C += A B on a 32x32x16 MFMA whose accumulator C stays in AGPRs, for kernels
// compiled with MFMAs in VGPR form: the compiler then keeps the score tiles its
// own MFMAs produce in VGPRs (no AGPR->VGPR copies before the VALU uses them)
// while these accumulators stay in AGPRs. The compiler does not insert hazard
// wait states around an inline MFMA: its operands must be written at least two
// instructions before it, and code that reads C afterwards must first wait for
// it with mfma_acc_drain().
__device__ __forceinline__ void mfma32_acc(f32x16_t& c, i32x4_t a, i32x4_t b, __bf16) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma32_acc(f32x16_t& c, i32x4_t a, i32x4_t b, _Float16) {
  asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}
// 24 wait states: more than an in-flight 32x32x16 MFMA needs before its result
// is read.
__device__ __forceinline__ void mfma_acc_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// 16x16x32 layouts: A (16 x 32): lane l holds row l%16, k = 8*(l/16) + e;
// B (32 x 16): lane l holds col l%16, k = 8*(l/16) + e;
// C (16 x 16): lane l holds col l%16, rows 4*(l/16) + v, v = 0..3.
__device__ __forceinline__ f32x4_t mfma16(i32x4_t a, i32x4_t b, f32x4_t c, __bf16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                 c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(i32x4_t a, i32x4_t b, f32x4_t c, _Float16) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                c, 0, 0, 0);
}

// ---------------------------------------------------------------- lane helpers
__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Value held by lane l^32 (the other half of the wave), via v_permlane32_swap.
__device__ __forceinline__ float other_half(float x) {
  uint32_t u = __float_as_uint(x);
  auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Row permutation inside a 32-row MFMA block: swap bits 2 and 3.
// Feeding A-operand row i from source row perm32(i) makes the C-layout values
// (v = 8..15 or 0..7 of one lane) cover 8 consecutive source rows, so the C
// tile can be reused directly as the k-operand of the next MFMA.
__device__ __forceinline__ int perm32(int i) {
  return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1);
}

// XOR swizzle of the 16-byte chunk index for an LDS tile whose rows hold C
// chunks; x is the row index modulo 16 (after any row permutation). Chosen so
// that 16 lanes reading rows x = 0..15 at one logical chunk hit 16 distinct
// 16-byte slots of the 256-byte window the 64 LDS banks serve per cycle (for
// C >= 8 also 8 lanes in 8 distinct slots of a 128-byte window).
template <int C>
__device__ __forceinline__ int swz(int x) {
  if constexpr (C >= 16) return x & 15;
  else if constexpr (C == 8) return ((x >> 1) & 7) ^ ((x & 1) << 2);
  else return (x >> 2) & (C - 1);
}

// XOR swizzle of the 16-byte chunk index for LDS tiles whose rows hold 4 chunks
// (64 bytes), read 16 B per lane with lane <-> row x (x = 0..15) at one logical
// chunk: the 16 lanes hit 16 distinct 16-byte slots of a 256-byte window and
// each 8-lane half 8 distinct slots of a 128-byte window (ds_read_b128 serves 8
// lanes per cycle; swz<4> meets only the first condition, a 2-way conflict).
__device__ __forceinline__ int swz4r(int x) { return ((x >> 2) & 1) | ((x ^ (x >> 2)) & 2); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ds_read_b64_tr_b16 (gfx950 LDS transpose read), checked on the device with a
// lane probe: in each group of 16 lanes, lane 4r + c (r, c = 0..3) points at 4
// consecutive 16-bit elements that form columns 4c..4c+3 of row r of a 4 x 16
// block; lane i of the group receives column i, i.e. (row 0..3, col i).
__device__ __forceinline__ u32x2_t lds_read_tr16(const lds_char_t* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  return __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)p));
}

// XOR swizzle of the 16-byte chunk index for LDS row tiles of 16 chunks per row
// that are read both row-wise (16 B per lane, 16 lanes on 16 consecutive rows)
// and with lds_read_tr16 (8 B per lane, 4 aligned consecutive rows x 4 aligned
// chunks per 32 lanes): a bijection on the row index modulo 16 whose upper two
// bits are the row index modulo 4, so both patterns touch 16 distinct 16-byte
// slots of the 256-byte bank window.
__device__ __forceinline__ int trswz16(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// The same for row tiles of 8 chunks per row (128-byte rows: 64-wide heads): a
// map of the row index modulo 16 to [0, 8) under which 16 lanes reading rows
// 0..15 at one logical chunk hit 16 distinct 16-byte slots of the 256-byte bank
// window, and the 32 lanes of a transposed read (4 aligned consecutive rows x 4
// aligned chunks) do too. Bits: r0 ^ r2, r3, r1 (found by exhaustive search
// against both access patterns).
__device__ __forceinline__ int trswz8(int r) { return ((r ^ (r >> 2)) & 1) | ((r >> 2) & 2) | ((r << 1) & 4); }
// Rows of 32 chunks (512 bytes, read row-wise only) take trswz16: a row starts
// on a 256-byte boundary and the XOR stays inside its 16-chunk half.
template <int CR>
__device__ __forceinline__ int trswz(int r) {
  static_assert(CR == 32 || CR == 16 || CR == 8, "row tiles of 32, 16 or 8 chunks");
  if constexpr (CR >= 16) return trswz16(r);
  else return trswz8(r);
}

// Compile-time integer as a value (for generic lambdas).
template <int K>
struct IC {
  static constexpr int value = K;
};

// Scheduling-group masks for __builtin_amdgcn_sched_group_barrier.
enum SchedMask : int { kSchedVALU = 0x2, kSchedSALU = 0x4, kSchedMFMA = 0x8, kSchedVMEM = 0x10, kSchedDSRead = 0x100,
                       kSchedDSWrite = 0x200, kSchedTrans = 0x400 };

// Block order. The hardware deals workgroups to the 8 XCDs round-robin by
// block id. When a head has at least 256 tiles (the Wan shapes), the dense
// kernels use the block id as the work item, head-major (work = head * tiles +
// tile): the 256 workgroups in flight then cover one head and all 8 XCDs
// stream that head's K/V (or Q/dO) at the same time, so their L2 misses fall
// on one head's 34 MB in the memory-side cache instead of eight heads' 268 MB.
// That measured 1-2% faster than giving each XCD its own head (xcd_remap
// below), with the same L2 fetch volume.
//
// With fewer tiles per head the workgroups in flight span several heads, and
// round-robin dealing would put each head's tiles on all 8 XCDs, each L2
// fetching the whole head. There the launcher sets xcd_order and the kernels
// use xcd_remap: each XCD takes a contiguous range of work items, so a head's
// tiles share one L2 (B=4, H=32, L=1024-4096: 2-8% faster per kernel; neutral
// from 128 tiles per head on). The block-sparse kernels always use xcd_remap:
// consecutive tasks of one query group walk the same key ranges (3-4% faster
// there than head-major order).
__device__ __forceinline__ int xcd_remap(int bid, int total) {
  const int xcd = bid & 7, slot = bid >> 3;
  const int per = total >> 3, rem = total & 7;
  return (xcd < rem) ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// This workgroup's work item of a dense kernel (the grid is exactly the work
// items): head-major, or contiguous per XCD when xcd_order is set.
__device__ __forceinline__ int work_item(int xcd_order) {
  const int bid = (int)blockIdx.x;
  return xcd_order ? xcd_remap(bid, (int)gridDim.x) : bid;
}

// Head tiles from which the dense launches keep head-major order.
constexpr int kHeadMajorMinTiles = 256;

}  // namespace dmad
