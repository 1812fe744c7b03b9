// Device helpers shared by the gfx950 kernels of libbzgemv.
//
// Number formats
//   bf16   raw uint16 bit patterns; widening is a 16-bit shift, narrowing
//          uses the hardware RNE conversion (v_cvt_pk_bf16_f32 on gfx950).
//   int4   two nibbles per byte, even k in the low nibble.  A dword holds
//          eight consecutive k: nibble p (bits 4p..4p+3) is k = 8d + p.
//   e4m3   OCP FP8 E4M3 codes (no infinities, max 448), decoded by the
//          gfx950 conversion instruction v_cvt_scalef32_pk_bf16_fp8.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bz {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two floats -> a bf16 pair (lo in bits 0-15), round to nearest even: one
// v_cvt_pk_bf16_f32 with both operands (converting the halves one at a time
// costs two of them plus a shift and an OR).
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef float f32x2v_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2v_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2v_t));
}

__device__ __forceinline__ bf16x2_t as_bf16x2(uint32_t v) { return __builtin_bit_cast(bf16x2_t, v); }

// fp32 += a.lo*b.lo + a.hi*b.hi  (v_dot2c_f32_bf16)
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a), as_bf16x2(b), c, false);
}

// Two nibbles -> two bf16 values 128+q.  Selects nibble p = sel (low half)
// and p = sel+4 (high half) of `v` after the caller's shift: the bf16 with
// exponent 2^7 and the nibble as the low mantissa bits is exactly 128 + q.
// Plain C++ that the compiler selects as one v_and_or_b32 (GFX9 VOP3 takes no
// literal and at most one SGPR, so the mask sits in an SGPR and the exponent
// bits in a VGPR).  It must stay visible to the compiler as a VALU
// instruction: its result feeds v_mfma B operands, and the wait states a VALU
// write needs before a matrix instruction reads the register are inserted by
// the compiler's hazard pass, which does not see through inline assembly
// (an inline-asm version gave wrong MFMA inputs when scheduled one
// instruction ahead of the MFMA).
__device__ __forceinline__ uint32_t nib2_bf16(uint32_t v) { return (v & 0x000F000Fu) | 0x43004300u; }

// Same, with the mask and exponent bits supplied by the caller from
// registers it keeps live (see NibbleConsts), so a hot loop does not
// rematerialize them.
__device__ __forceinline__ uint32_t nib2_bf16(uint32_t v, uint32_t mask_s, uint32_t magic_v) {
    return (v & mask_s) | magic_v;
}

// The two constants of nib2_bf16 in registers (an SGPR and a VGPR) whose
// values the compiler cannot fold back into literals.
struct NibbleConsts {
    uint32_t mask;   // SGPR: 0x000F000F
    uint32_t magic;  // VGPR: 0x43004300 (bf16 128.0 in both halves)
    __device__ __forceinline__ NibbleConsts() {
        asm volatile("s_mov_b32 %0, 0x000F000F" : "=s"(mask));
        asm volatile("v_mov_b32 %0, 0x43004300" : "=v"(magic));
    }
};

// Two e4m3 codes (bytes 0,1 or 2,3 of v) -> two bf16 (exact: every e4m3
// value is a bf16 value).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_bf16(uint32_t v) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, HI));
}

// DPP cross-lane moves.  update_dpp(old, src, ctrl, row_mask, bank_mask, bound_ctrl).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;          // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;          // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;   // lane i <- lane 7-i inside each 8-lane half row

// Sum over each aligned group of 8 lanes; every lane of the group gets it.
__device__ __forceinline__ float sum8(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppHalfMirror>(v);
    return v;
}

constexpr int kDppRowMirror = 0x140;     // lane i <- lane 15-i inside each 16-lane row

// Sum / max over each aligned group of 16 lanes (a DPP row); every lane of
// the group gets it.  After the quad and half-row steps each lane holds its
// 8-lane group's value; the row mirror pairs the two halves.
__device__ __forceinline__ float sum16_dpp(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppHalfMirror>(v);
    return v + dpp_f32<kDppRowMirror>(v);
}
__device__ __forceinline__ float max16_dpp(float v) {
    v = fmaxf(v, dpp_f32<kDppXor1>(v));
    v = fmaxf(v, dpp_f32<kDppXor2>(v));
    v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
    return fmaxf(v, dpp_f32<kDppRowMirror>(v));
}

// Sum of the four 16-lane rows of a wave once each row holds its own sum
// (after sum16_dpp): GFX9's DPP row broadcasts add row 0 into row 1 and row 2
// into row 3 (row_bcast:15), then lane 31 into rows 2 and 3 (row_bcast:31);
// lane 63 gets (r3 + r2) + (r1 + r0).  Two VALU operations, no LDS.
constexpr int kDppRowBcast15 = 0x142;
constexpr int kDppRowBcast31 = 0x143;
__device__ __forceinline__ float rows4_sum_lane63(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kDppRowBcast15, 0xA, 0xF,
                                                               false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kDppRowBcast31, 0xC, 0xF,
                                                               false));
    return v;
}

// Sum over each aligned quad of lanes.
__device__ __forceinline__ float sum4(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    return v;
}

// Full-wave (64 lanes) sum, every lane gets it.  Prologue use only.
__device__ __forceinline__ float wave_sum(float v) {
    v = sum8(v);
    v += __shfl_xor(v, 8, 64);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ u32x4 ldg16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
// The same with the non-temporal hint, for data read once (weights): it does
// not displace lines that other workgroups read again (x) from the L2.
__device__ __forceinline__ u32x4 ldg16_nt(const void* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Range-checked 16-byte loads through a buffer resource (V#) covering
// [p, p + bytes): an offset at or past `bytes` returns zeros and sends no
// request to memory.  Lets a kernel issue a fixed number of loads
// unconditionally (exact wait counts) without reading past a buffer or
// hammering one line with clamped indices.  Word 3 = 0x00020000 is the GFX9
// untyped-buffer format (data format 32).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
constexpr uint32_t kBufferOob = 0xFFFFFFF0u;  // an offset past any buffer_rsrc range
__device__ __forceinline__ u32x4 buffer_ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
// The same with the non-temporal hint (cache-policy operand 2 = nt on gfx950),
// for data read once.
__device__ __forceinline__ u32x4 buffer_ld16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
}
// Cache-policy operand of a buffer access with the agent-scope coherence bit
// (sc1 on gfx950): what the compiler emits for a relaxed agent-scope atomic
// load or store (__hip_atomic_load / __hip_atomic_store with
// __HIP_MEMORY_SCOPE_AGENT), for 16-byte accesses that have no atomic form.
constexpr int kCpolAgent = 16;
__device__ __forceinline__ uint32_t buffer_ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + __expf(-g)); }

// Lane placement of 16-byte pieces.  A wave instruction whose lane 4 a + b
// reads piece b of row a (a = 0..15, b = 0..3: each quad of lanes reads one
// row's 64 contiguous bytes) is moved by quad_to_mfma to lane a + 16 b, the
// placement of the bf16 MFMA operands (row = lane % 16).  `src` is
// quad_source(lane), computed once.  (Measured on MI355X: it pays for x
// rows far apart in memory, whose quads would otherwise touch four lines;
// not for the 1 KiB weight tiles of the streaming kernel, whose quads span
// two lines: int4 decode GEMVs 1% slower with it.)
__device__ __forceinline__ int quad_source(int lane) { return ((lane & 15) * 4 + (lane >> 4)) * 4; }
__device__ __forceinline__ u32x4 quad_to_mfma(u32x4 v, int src) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)v[i]);
    return r;
}

}  // namespace bz
