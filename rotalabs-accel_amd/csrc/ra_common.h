// Shared device helpers for the gfx950 W8A16 kernels: vector types, exact
// int8 -> fp16/bf16 dequantisation, MFMA wrappers and dtype conversions.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rotaccel.h"

namespace ra {

// 16-byte store of a uint4 through a native vector type. (Assigning the HIP
// uint4 struct through a cast pointer is lowered as a struct copy that keeps
// the source array in scratch memory.)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store16(void *p, const uint4 &v) {
  *reinterpret_cast<u32x4_t *>(p) = u32x4_t{v.x, v.y, v.z, v.w};
}
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store8(void *p, uint32_t lo, uint32_t hi) {
  *reinterpret_cast<u32x2_t *>(p) = u32x2_t{lo, hi};
}

// v as an fp32 register value: the backend otherwise folds an fp32 result
// feeding a 16-bit conversion into one mixed-precision FMA (v_fma_mix),
// which rounds once instead of to fp32 first and then to 16 bits. (volatile:
// the value is also computed where it is written, not sunk into a later
// conditional block.)
__device__ __forceinline__ float fp32_rounded(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// 16-byte global load with the non-temporal cache policy
// (`global_load_dwordx4 ... nt`), for data a kernel reads exactly once and no
// later launch expects to find in cache: the weight rows the GEMV kernels
// stream (M=1 K=4096 N=11008: 9.2 -> 8.3-8.6 us per launch) and the KV codec's
// input. Activations, which many waves re-read, keep the default policy.
typedef unsigned int u32x4_vec __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream16(const void *p) {
  const u32x4_vec v = __builtin_nontemporal_load(static_cast<const u32x4_vec *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// One 32-bit (16-bit) word through the vector memory path (a buffer load)
// although its address is wave-uniform. The decode kernels load their
// epilogue operands (scale, bias) this way: as scalar loads they share the
// lgkm counter with the kernel-argument loads, and the compiler's next wait
// for an argument (lgkmcnt(0): scalar loads return out of order) would hold
// the row's weight loads back by one memory round trip.
__device__ __forceinline__ uint32_t vload_b32(const void *p) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, 4, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 0);
}
__device__ __forceinline__ uint32_t vload_b16(const void *p) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, 2, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b16(r, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Direct-to-LDS copies (gfx950 global_load_lds_dwordx4) and explicit waits.
// LDS byte address of a __shared__ object (what M0 and ds_* addresses use).
__device__ __forceinline__ uint32_t lds_offset(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// 16 bytes per lane from global memory to LDS at M0 + OFS + 16 * lane; the
// instruction offset OFS is added to both the global and the LDS address, so
// up to four consecutive 1 KB copies share one M0 value (the caller passes
// g - OFS). NEW_M0 first writes M0; an LDS DMA that reads M0 needs one wait
// state after that SALU write.
template <int OFS, bool NEW_M0>
__device__ __forceinline__ void dma16(const void *g_minus_ofs, uint32_t m0_value) {
  if (NEW_M0)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off offset:%2" ::"s"(m0_value),
                 "v"(g_minus_ofs), "n"(OFS)
                 : "memory", "m0");
  else
    asm volatile("global_load_lds_dwordx4 %0, off offset:%1" ::"v"(g_minus_ofs), "n"(OFS) : "memory");
}

// As dma16 with the uniform part of the global address in an SGPR pair and a
// 32-bit per-lane byte offset, so a copy needs no per-lane address arithmetic.
template <int OFS, bool NEW_M0>
__device__ __forceinline__ void dma16s(const void *sbase, uint32_t voff, uint32_t m0_value) {
  if (NEW_M0)
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2 offset:%3" ::"s"(m0_value),
                 "v"(voff), "s"(sbase), "n"(OFS)
                 : "memory", "m0");
  else
    asm volatile("global_load_lds_dwordx4 %0, %1 offset:%2" ::"v"(voff), "s"(sbase), "n"(OFS) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [LO, HI).
template <int LO, int HI, typename F>
__device__ __forceinline__ void static_for_int(F &&f) {
  if constexpr (LO < HI) {
    f(std::integral_constant<int, LO>{});
    static_for_int<LO + 1, HI>(f);
  }
}


typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename To, typename From>
__device__ __forceinline__ To bitcast(const From &v) {
  static_assert(sizeof(To) == sizeof(From), "bitcast size mismatch");
  return __builtin_bit_cast(To, v);
}

// ---------------------------------------------------------------------------
// int8 -> fp16, exact. Magic-number conversion (Kim et al. 2022, "Who Says
// Elephants Can't Run: Bringing Large Scale MoE Models into Cloud Scale
// Production", also used by FasterTransformer): the fp16 whose bit pattern is
// 0x64UU equals 1024 + UU; with UU = q ^ 0x80 = q + 128 it equals 1152 + q, so
// one packed subtraction of 1152 (exact in fp16) yields q for two lanes.
// Cost: 1 xor per 4 values, 1 v_perm + 1 v_pk_add_f16 per 2 values.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t dq2_f16(uint32_t t, uint32_t sel) {
  const f16x2 magic = {(_Float16)1152.0f, (_Float16)1152.0f};
  const uint32_t biased = __builtin_amdgcn_perm(0x64646464u, t, sel);
  return bitcast<uint32_t>(bitcast<f16x2>(biased) - magic);
}

// 8 int8 (w0 = bytes 0..3, w1 = bytes 4..7) -> 8 fp16 in element order.
__device__ __forceinline__ uint4 dq8_f16(uint32_t w0, uint32_t w1) {
  const uint32_t t0 = w0 ^ 0x80808080u, t1 = w1 ^ 0x80808080u;
  uint4 r;
  r.x = dq2_f16(t0, 0x04010400u);  // bytes 0,1
  r.y = dq2_f16(t0, 0x04030402u);  // bytes 2,3
  r.z = dq2_f16(t1, 0x04010400u);
  r.w = dq2_f16(t1, 0x04030402u);
  return r;
}

// ---------------------------------------------------------------------------
// int8 -> fp16, exact, 1 VALU per value: v_cvt_f16_i16 with an SDWA
// sign-extended byte select converts one byte, and its destination select
// writes the half of the dword the value belongs to (the second write keeps
// the first: UNUSED_PRESERVE). 8 instructions per 8 values against 10 for the
// magic-number form; used by the weight-streaming kernels, where it took
// 1-4 % off (M=16 K=4096 N=11008: 10.9 -> 10.5 us). The compiler does not
// form it (it shifts the byte down first and packs the halves separately),
// hence the inline assembly; being opaque to the scheduler, it stays out of
// the tiled GEMM, whose dequantisation is interleaved with the MFMAs by
// scheduling groups (there it measured 2 % slower).
// Each pair ends with one wait state (s_nop 0) after the upper-half write:
// without it the fp16 split-K kernel with one 16-row tile, the extra row and
// two weight tiles per wave gave wrong sums in rows 0..16 (32171 of 102000
// outputs at M=17 K=16384 N=6000), while the build that differs only by these
// nops (the same instruction stream otherwise) is exact. The compiler does not
// pad after inline assembly the way it pads its own 16-bit partial writes.
// Cost of the nop: 0.3-1.7 % on the row GEMV, small-batch and 64-row tile
// kernels (M=1 K=4096 N=11008 8.31 -> 8.34 us).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t cvt2_f16_b01(uint32_t w) {
  uint32_t r;
  asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
      "v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
      "s_nop 0"
      : "=&v"(r)
      : "v"(w));
  return r;
}
__device__ __forceinline__ uint32_t cvt2_f16_b23(uint32_t w) {
  uint32_t r;
  asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
      "v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3\n\t"
      "s_nop 0"
      : "=&v"(r)
      : "v"(w));
  return r;
}
__device__ __forceinline__ uint4 dq8_f16_cvt(uint32_t w0, uint32_t w1) {
  return make_uint4(cvt2_f16_b01(w0), cvt2_f16_b23(w0), cvt2_f16_b01(w1), cvt2_f16_b23(w1));
}

// ---------------------------------------------------------------------------
// int8 -> bf16, exact. A signed byte converts to fp32 in one instruction
// (v_cvt_f32_i32 with an SDWA sign-extended byte select); |q| <= 128 needs at
// most 8 significant bits, so the fp32 value's upper half IS the bf16 value
// and packing two upper halves (one v_perm) is exact. 1.5 VALU ops per value.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

__device__ __forceinline__ uint4 dq8_bf16(uint32_t w0, uint32_t w1) {
  uint4 r;
  r.x = pack_hi16((float)(int8_t)(w0), (float)(int8_t)(w0 >> 8));
  r.y = pack_hi16((float)(int8_t)(w0 >> 16), (float)(int8_t)(w0 >> 24));
  r.z = pack_hi16((float)(int8_t)(w1), (float)(int8_t)(w1 >> 8));
  r.w = pack_hi16((float)(int8_t)(w1 >> 16), (float)(int8_t)(w1 >> 24));
  return r;
}

// ---------------------------------------------------------------------------
// Scalar conversions between fp32 and the 16-bit storage types (RNE).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float f16_to_f32(uint16_t b) { return (float)bitcast<_Float16>(b); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f32_to_f16(float v) { return bitcast<uint16_t>((_Float16)v); }
__device__ __forceinline__ uint16_t f32_to_bf16(float v) { return bitcast<uint16_t>((__bf16)v); }

__device__ __forceinline__ float load_as_f32(const void *p, int64_t i, int dt) {
  if (dt == RA_F32) return static_cast<const float *>(p)[i];
  const uint16_t b = static_cast<const uint16_t *>(p)[i];
  return dt == RA_F16 ? f16_to_f32(b) : bf16_to_f32(b);
}

__device__ __forceinline__ void store_from_f32(void *p, int64_t i, int dt, float v) {
  if (dt == RA_F32) {
    static_cast<float *>(p)[i] = v;
  } else {
    static_cast<uint16_t *>(p)[i] = dt == RA_F16 ? f32_to_f16(v) : f32_to_bf16(v);
  }
}

// Round an fp32 value to fp16 / bf16 and back (the rounding torch applies when
// an fp32 intermediate is stored in a reduced-precision tensor).
__device__ __forceinline__ float round_through(float v, int dt) {
  if (dt == RA_F16) return (float)(_Float16)v;
  if (dt == RA_BF16) return (float)(__bf16)v;
  return v;
}

// ---------------------------------------------------------------------------
// Activation-type traits: dequantiser, MFMA instructions, output conversion.
// MFMA operand layouts (gfx950, wave64):
//  16x16x32: A[i][k] from lane i + 16*(k/8), element k%8;
//            B[k][j] from lane j + 16*(k/8), element k%8;
//            D[i][j] in lane j + 16*(i/4), element i%4.
//  32x32x16: A[i][k] from lane i + 32*(k/8), element k%8;
//            B[k][j] from lane j + 32*(k/8), element k%8;
//            D[i][j] in lane j + 32*((i/4)%2), element (i%4) + 4*(i/8).
// Only the row / column mappings matter to the kernels: the sum over k is the
// same for any permutation of k applied identically to A and B.
// ---------------------------------------------------------------------------
template <int DT>
struct Act;

template <>
struct Act<RA_F16> {
  static __device__ __forceinline__ uint4 dq8(uint32_t w0, uint32_t w1) { return dq8_f16(w0, w1); }
  // the weight-streaming kernels' form (fewer VALU, opaque to the scheduler)
  static __device__ __forceinline__ uint4 dq8s(uint32_t w0, uint32_t w1) { return dq8_f16_cvt(w0, w1); }
  static __device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
  }
  // c + sum of the 8 products a[i] * b[i] (v_dot2 on element pairs, fp32 sums)
  static __device__ __forceinline__ float dot8(uint4 a, uint4 b, float c) {
    c = __builtin_amdgcn_fdot2(bitcast<f16x2>(a.x), bitcast<f16x2>(b.x), c, false);
    c = __builtin_amdgcn_fdot2(bitcast<f16x2>(a.y), bitcast<f16x2>(b.y), c, false);
    c = __builtin_amdgcn_fdot2(bitcast<f16x2>(a.z), bitcast<f16x2>(b.z), c, false);
    return __builtin_amdgcn_fdot2(bitcast<f16x2>(a.w), bitcast<f16x2>(b.w), c, false);
  }
  static __device__ __forceinline__ uint16_t out(float v) { return f32_to_f16(v); }
  static __device__ __forceinline__ float in(uint16_t b) { return f16_to_f32(b); }
  static __device__ __forceinline__ float rnd(float v) { return (float)(_Float16)v; }
};

template <>
struct Act<RA_BF16> {
  static __device__ __forceinline__ uint4 dq8(uint32_t w0, uint32_t w1) { return dq8_bf16(w0, w1); }
  static __device__ __forceinline__ uint4 dq8s(uint32_t w0, uint32_t w1) { return dq8_bf16(w0, w1); }
  static __device__ __forceinline__ f32x4 mfma16(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(uint4 a, uint4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ float dot8(uint4 a, uint4 b, float c) {
    c = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(a.x), bitcast<bf16x2>(b.x), c, false);
    c = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(a.y), bitcast<bf16x2>(b.y), c, false);
    c = __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(a.z), bitcast<bf16x2>(b.z), c, false);
    return __builtin_amdgcn_fdot2_f32_bf16(bitcast<bf16x2>(a.w), bitcast<bf16x2>(b.w), c, false);
  }
  static __device__ __forceinline__ uint16_t out(float v) { return f32_to_bf16(v); }
  static __device__ __forceinline__ float in(uint16_t b) { return bf16_to_f32(b); }
  static __device__ __forceinline__ float rnd(float v) { return (float)(__bf16)v; }
};

// Wave64 sum (all lanes receive the total).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Wave64 sum through DPP lane moves (VALU only, no LDS round trips): quad
// butterflies, half-row and row mirrors, then the row_bcast15 / row_bcast31
// carries; the total ends in lane 63 and is returned to every lane.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_moved(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_moved<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
  v += dpp_moved<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
  v += dpp_moved<0x141, 0xF>(v);  // row_half_mirror
  v += dpp_moved<0x140, 0xF>(v);  // row_mirror
  v += dpp_moved<0x142, 0xA>(v);  // row_bcast15 into rows 1 and 3
  v += dpp_moved<0x143, 0xC>(v);  // row_bcast31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// NaN-propagating maximum (torch's amax semantics; v_maximum*_f32 on gfx950).
__device__ __forceinline__ float nan_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float wave_maximum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = nan_max(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// SwiGLU of a gate/up pair with the roundings of the reference composition
// int8_gemm (gate, up stored in the activation dtype) -> swiglu_torch
// (F.silu and the product each computed in fp32 and stored in that dtype),
// src/rotalabs_accel/kernels/gemm.py:46 and kernels/activations.py:45.
template <typename A>
__device__ __forceinline__ uint16_t swiglu_out(float g32, float u32) {
  const float g = A::rnd(g32), u = A::rnd(u32);
  const float sg = A::rnd(g / (1.0f + expf(-g)));
  return A::out(sg * u);
}

// Epilogue value: fp32 accumulator * per-channel scale (+ bias), in fp32.
__device__ __forceinline__ float epilogue_value(float acc, const float *scale, const void *bias,
                                                int bias_dt, int n) {
  float v = acc * scale[n];
  if (bias) v += load_as_f32(bias, n, bias_dt);
  return v;
}

// 16-byte buffer stores and loads at device scope (cache policy sc1): written
// through to, and read from, the level all XCDs share, so partial sums pass
// between workgroups on any XCD without a cache-wide fence. Buffer
// instructions, so the compiler tracks their waits; out-of-range offsets
// read zeros and drop stores.
constexpr int kCpolSc1 = 16;
constexpr int kRsrcWord3 = 0x00020000;  // raw (untyped) buffer, gfx9 family
typedef unsigned int u32x4_dev __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void store_dev16(__amdgpu_buffer_rsrc_t r, uint32_t off, const f32x4 &v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_dev, v), r, (int)off, 0, kCpolSc1);
}
__device__ __forceinline__ f32x4 load_dev16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCpolSc1));
}

}  // namespace ra
