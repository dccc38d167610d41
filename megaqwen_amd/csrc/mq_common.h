// Shared device helpers for the MI355X (gfx950, CDNA4) Qwen3-0.6B kernels.
//
// Model shapes follow the reference's constants (csrc/megakernel/config.cuh:33-40).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mq {

constexpr int H = 1024;        // hidden size
constexpr int I = 3072;        // MLP intermediate size
constexpr int NQ = 16;         // query heads
constexpr int NKV = 8;         // key/value heads
constexpr int HD = 128;        // head dim
constexpr int QS = NQ * HD;    // 2048
constexpr int KVS = NKV * HD;  // 1024
constexpr int VOCAB = 151936;
constexpr int MAX_LAYERS = 32;
constexpr float EPS = 1e-6f;

// Word of the per-device library workspace where the prefill kernels flag an
// invalid input (the decode kernel's words sit below it, its exchange buffers above).
constexpr uint32_t WS_PREFILL_ERR = 96;

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x3 __attribute__((ext_vector_type(3)));
typedef short bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ bf16
__device__ __forceinline__ float bf2f(uint32_t b16) { return __uint_as_float(b16 << 16); }
__device__ __forceinline__ float bflo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bfhi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
typedef __bf16 bfv2 __attribute__((ext_vector_type(2)));
// fp32 -> bf16 bits, round to nearest even (gfx950's v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t f2bf(float f) { return __builtin_bit_cast(unsigned short, (__bf16)f); }
// Round an fp32 value to the nearest bf16 value (kept in fp32).
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// Unpack 8 bf16 (one 16-byte load) into fp32.
__device__ __forceinline__ void unpack8(const u32x4& w, float (&f)[8]) {
  f[0] = bflo(w.x); f[1] = bfhi(w.x);
  f[2] = bflo(w.y); f[3] = bfhi(w.y);
  f[4] = bflo(w.z); f[5] = bfhi(w.z);
  f[6] = bflo(w.w); f[7] = bfhi(w.w);
}

// Two bf16 values (low half first) in one word: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  const bfv2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
// Round two fp32 values to bf16 (kept in fp32) with one conversion.
__device__ __forceinline__ void rbf2(float& a, float& b) {
  const uint32_t p = pack_bf2(a, b);
  a = bflo(p);
  b = bfhi(p);
}

// acc + w.lo * x.lo + w.hi * x.hi on one word of bf16 pairs (v_dot2_f32_bf16: the
// products are exact in fp32, the sum is accumulated in fp32).
__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), __builtin_bit_cast(bf16x2, x), acc, false);
}
// acc + (8 bf16 weights) . (8 bf16 inputs), both as 16-byte chunks.
__device__ __forceinline__ float dot_chunk(const u32x4& w, const u32x4& x, float acc) {
  acc = dot2(w.x, x.x, acc);
  acc = dot2(w.y, x.y, acc);
  acc = dot2(w.z, x.z, acc);
  return dot2(w.w, x.w, acc);
}

// 16x16x32 bf16 matrix product-accumulate. For A (16 x 32) lane l holds row l % 16,
// for B (32 x 16) column l % 16, each as 8 values of the k range owned by lane group
// l / 16 (the same k order in A and B); D lane l holds rows 4 * (l / 16) + e of column l % 16.
__device__ __forceinline__ f32x4 mfma_16x16x32(const u32x4& a, const u32x4& b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                  0, 0);
}

// ------------------------------------------------------------------ wave64 reductions
// DPP row operations (16-lane rows): quad_perm [1,0,3,2] and [2,3,0,1] pair
// lanes within quads, row_half_mirror pairs lane i with 7-i, row_mirror lane i
// with 15-i; after the four steps every lane of a row holds the row's sum.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  v += dpp<0x140>(v);
  return v;
}
__device__ __forceinline__ float readlane(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Sum over the 64 lanes; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}
// wave_sum of N independent values, step by step across the values so that the DPP and
// readlane latencies of one overlap the others (same operations and order as wave_sum,
// so the results are bitwise identical).
template <int N>
__device__ __forceinline__ void wave_sum_n(float (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0xB1>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x4E>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x141>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x140>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] = (readlane(v[k], 0) + readlane(v[k], 16)) + (readlane(v[k], 32) + readlane(v[k], 48));
}
// wave_sum of N values at once (N a multiple of 4) with the same additions in the same
// order as wave_sum, so the results are bitwise identical: the 16-lane butterfly of each
// row, then rows 0 + 1 and 2 + 3 (lanes l, l + 16 meet through v_permlane16_swap, values
// k and k + N/4 trading rows), then (0 + 1) + (2 + 3) (lanes l, l + 32 meet through
// v_permlane32_swap, values k and k + N/2 trading halves). The swaps replace wave_sum's
// four readlanes and three scalar-sourced adds per value. On return lane l holds in v[k],
// k < N/4, the total of value k + (l / 16) * (N / 4).
template <int N>
__device__ __forceinline__ void wave_sum_t(float (&v)[N]) {
  static_assert(N % 4 == 0, "N must be a multiple of 4");
  constexpr int H2 = N / 2, H4 = N / 4;
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0xB1>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x4E>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x141>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x140>(v[k]);
  // values k and k + N/4 (and k + N/2 and k + 3N/4) trade rows: afterwards row 0 holds
  // value k as R0 + R1, row 1 value k + N/4 as R0 + R1, rows 2 and 3 the same as R2 + R3
#pragma unroll
  for (int k = 0; k < H4; k++)
#pragma unroll
    for (int b = 0; b < N; b += H2) {
      const auto r =
          __builtin_amdgcn_permlane16_swap(__float_as_uint(v[b + k]), __float_as_uint(v[b + k + H4]), false, false);
      v[b + k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
  // values k and k + N/2 trade halves: lanes l and l + 32 add (R0 + R1) + (R2 + R3)
#pragma unroll
  for (int k = 0; k < H4; k++) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + H2]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}
// Sums of N values (N even) over lanes 0..31 and, separately, over lanes 32..63, as
// row16_sum followed by rows 0 + 1 and 2 + 3: on return lane l holds in v[k], k < N/2,
// the total of value k + ((l / 16) & 1) * (N / 2) over lane half l / 32.
template <int N>
__device__ __forceinline__ void half_sum_t(float (&v)[N]) {
  static_assert(N % 2 == 0, "N must be even");
  constexpr int H2 = N / 2;
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0xB1>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x4E>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x141>(v[k]);
#pragma unroll
  for (int k = 0; k < N; k++) v[k] += dpp<0x140>(v[k]);
#pragma unroll
  for (int k = 0; k < H2; k++) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + H2]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}
// Wave-wide maxima of N independent values, interleaved like wave_sum_n
template <int N>
__device__ __forceinline__ void wave_max_n(float (&v)[N]) {
#pragma unroll
  for (int k = 0; k < N; k++) v[k] = fmaxf(v[k], dpp<0xB1>(v[k]));
#pragma unroll
  for (int k = 0; k < N; k++) v[k] = fmaxf(v[k], dpp<0x4E>(v[k]));
#pragma unroll
  for (int k = 0; k < N; k++) v[k] = fmaxf(v[k], dpp<0x141>(v[k]));
#pragma unroll
  for (int k = 0; k < N; k++) v[k] = fmaxf(v[k], dpp<0x140>(v[k]));
#pragma unroll
  for (int k = 0; k < N; k++)
    v[k] = fmaxf(fmaxf(readlane(v[k], 0), readlane(v[k], 16)), fmaxf(readlane(v[k], 32), readlane(v[k], 48)));
}

// ------------------------------------------------------------------ global loads
// Pointers that arrive through structs in device memory have no known address
// space; loading through an explicit global pointer gives global_load (counted in
// vmcnt only) instead of a flat load (which also counts in lgkmcnt and would make
// every LDS wait wait for the weight stream as well).
typedef const __attribute__((address_space(1))) u32x4 gu32x4;
typedef const __attribute__((address_space(1))) u32x2 gu32x2;
typedef const __attribute__((address_space(1))) uint32_t gu32;
typedef const __attribute__((address_space(1))) uint16_t gu16;
// Weights are read once per token, so their loads are non-temporal: on MI355X a 1 GiB
// stream of 16-byte non-temporal loads runs at 7.15 TB/s against 6.07 TB/s for the same
// loads with the default policy, and the weight bursts then leave the exchange lines in L2.
__device__ __forceinline__ u32x4 ldw(const uint16_t* p) { return __builtin_nontemporal_load((gu32x4*)(p)); }
__device__ __forceinline__ u32x2 ldw2(const uint16_t* p) { return __builtin_nontemporal_load((gu32x2*)(p)); }
__device__ __forceinline__ uint32_t ldw1(const uint16_t* p) { return __builtin_nontemporal_load((gu32*)(p)); }
__device__ __forceinline__ uint32_t ldraw16(const uint16_t* p) { return *(gu16*)(p); }

// A pointer that is the same in every lane, moved to scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// ------------------------------------------------------------------ device-coherent access
// Plain loads/stores of data written by other CUs during the same launch can
// hit stale L2 lines of another XCD: inter-workgroup traffic uses sc1
// (device scope) buffer operations, which the compiler tracks like ordinary
// loads for s_waitcnt.
constexpr int SC1 = 16;  // gfx940+ cache-policy bit for device scope

struct Buf {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ explicit Buf(const void* base)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000)) {}
  __device__ __forceinline__ u32x4 ld4(uint32_t byte_off) const {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, SC1);
  }
  __device__ __forceinline__ u32x2 ld2(uint32_t byte_off) const {
    return __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, SC1);
  }
  __device__ __forceinline__ uint32_t ld1(uint32_t byte_off) const {
    return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, SC1);
  }
  __device__ __forceinline__ void st1(uint32_t v, uint32_t byte_off) const {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, byte_off, 0, SC1);
  }
  __device__ __forceinline__ void st4(u32x4 v, uint32_t byte_off) const {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, byte_off, 0, SC1);
  }
};

// Wait for all of this wave's outstanding vector-memory operations (loads and
// stores; gfx9 counts both in vmcnt) to complete. simm16 = vmcnt(0),
// expcnt(7), lgkmcnt(15).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// One 16-byte LDS DMA per lane: lane l's 16 bytes at `gptr` land at LDS byte
// address lds + 16 * l. Issued as inline assembly so that the compiler's vmcnt
// bookkeeping for register loads ignores it (the waits it
// derives stay correct, at worst longer); its completion is awaited explicitly.
// M0 (which carries the LDS address) is saved and restored around it.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gptr), "s"(lds)
      : "memory");
}
// the same with the non-temporal policy
__device__ __forceinline__ void dma16_nt(const void* gptr, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off nt\n\ts_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gptr), "s"(lds)
      : "memory");
}

}  // namespace mq
