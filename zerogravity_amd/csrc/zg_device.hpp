// Device-side helpers shared by every zerogravity_amd kernel (gfx950 only).
// All HIP code is compiled with -ffp-contract=off: a fused multiply-add only
// appears where a kernel calls fmaf() explicitly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// IEEE binary16 -> binary32 (exact, subnormals included); the hardware
// conversion is exact for every finite code, which is all a registered
// tensor may hold (nonfinite scales are refused at registration).
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    _Float16 v;
    __builtin_memcpy(&v, &h, 2);
    return (float)v;
}

// binary32 -> binary16, round to nearest even, restated bit by bit so the
// dynamic Q8_0 activation scale rounds exactly as the CPU path does.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float value) {
    uint32_t bits = __float_as_uint(value);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int exponent = (int)((bits >> 23) & 0xff);
    uint32_t fraction = bits & 0x7fffffu;
    if (exponent == 255) return (uint16_t)(sign | 0x7c00u | (fraction ? (((fraction >> 13) & 0xffffu) | 0x200u) : 0u));
    int half_exp = exponent - 127 + 15;
    if (half_exp >= 31) return (uint16_t)(sign | 0x7c00u);
    if (half_exp <= 0) {
        if (half_exp < -10) return (uint16_t)sign;
        uint32_t mantissa = fraction | 0x800000u;
        uint32_t shift = (uint32_t)(14 - half_exp);
        uint32_t half = (mantissa + ((1u << (shift - 1)) - 1) + ((mantissa >> shift) & 1)) >> shift;
        return (uint16_t)(sign | half);
    }
    uint32_t rounded = fraction + 0x0fffu + ((fraction >> 13) & 1);
    if (rounded >= 0x800000u) return (uint16_t)(sign | ((uint32_t)(half_exp + 1) << 10));
    return (uint16_t)(sign | ((uint32_t)half_exp << 10) | (rounded >> 13));
}

__device__ __forceinline__ float f16_roundtrip(float v) { return f16_to_f32(f32_to_f16_rne(v)); }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ bool finite_f32(float v) {
    return (__float_as_uint(v) & 0x7f800000u) != 0x7f800000u;
}

template <typename T>
__device__ __forceinline__ T wave_sum_xor(T v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// DPP lane moves (VALU, no LDS round trip).  dpp_f<CTRL> returns, in each
// lane, the value of the lane CTRL selects (0 where the source lies outside
// the row and bound_ctrl applies).
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWMASK, 0xf, true));
}
constexpr int kDppXor1 = 0xb1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4e;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7 - i within 8

// Sum over groups of W consecutive lanes (W = 2..64), complete in the LAST
// lane of each group (row shifts toward higher lanes, then row broadcasts).
template <int W>
__device__ __forceinline__ float group_sum_last(float v) {
    if (W >= 2) v += dpp_f<0x111>(v);       // row_shr:1
    if (W >= 4) v += dpp_f<0x112>(v);       // row_shr:2
    if (W >= 8) v += dpp_f<0x114>(v);       // row_shr:4
    if (W >= 16) v += dpp_f<0x118>(v);      // row_shr:8
    if (W >= 32) v += dpp_f<0x142, 0xa>(v); // row_bcast:15 into rows 1 and 3
    if (W >= 64) v += dpp_f<0x143, 0xc>(v); // row_bcast:31 into rows 2 and 3
    return v;
}
__device__ __forceinline__ float group_sum_last(float v, int log2w) {
    switch (log2w) {
    case 1: return group_sum_last<2>(v);
    case 2: return group_sum_last<4>(v);
    case 3: return group_sum_last<8>(v);
    case 4: return group_sum_last<16>(v);
    case 5: return group_sum_last<32>(v);
    default: return group_sum_last<64>(v);
    }
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ double dpp_d(double v) {
    const unsigned long long u = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(u & 0xffffffffu), CTRL, ROWMASK, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(u >> 32), CTRL, ROWMASK, 0xf, true);
    return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}
template <int W>
__device__ __forceinline__ double group_sum_last(double v) {
    if (W >= 2) v += dpp_d<0x111>(v);
    if (W >= 4) v += dpp_d<0x112>(v);
    if (W >= 8) v += dpp_d<0x114>(v);
    if (W >= 16) v += dpp_d<0x118>(v);
    if (W >= 32) v += dpp_d<0x142, 0xa>(v);
    if (W >= 64) v += dpp_d<0x143, 0xc>(v);
    return v;
}
// Max over groups of W lanes complete in the last lane (lanes without a
// source keep their own value).
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float dpp_keep(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROWMASK, 0xf, false));
}
template <int W>
__device__ __forceinline__ float group_max_last(float v) {
    if (W >= 2) v = fmaxf(v, dpp_keep<0x111>(v));
    if (W >= 4) v = fmaxf(v, dpp_keep<0x112>(v));
    if (W >= 8) v = fmaxf(v, dpp_keep<0x114>(v));
    if (W >= 16) v = fmaxf(v, dpp_keep<0x118>(v));
    if (W >= 32) v = fmaxf(v, dpp_keep<0x142, 0xa>(v));
    if (W >= 64) v = fmaxf(v, dpp_keep<0x143, 0xc>(v));
    return v;
}
// Wave totals in every lane (DPP to lane 63, then a scalar broadcast).
__device__ __forceinline__ float wave_sum_all(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(group_sum_last<64>(v)), 63));
}
__device__ __forceinline__ float wave_max_all(float v) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(group_max_last<64>(v)), 63));
}
__device__ __forceinline__ double wave_sum_all(double v) {
    const unsigned long long u = __double_as_longlong(group_sum_last<64>(v));
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(u & 0xffffffffu), 63);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(u >> 32), 63);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}
__device__ __forceinline__ double group8_sum_all(double v) {
    v += dpp_d<0xb1>(v);
    v += dpp_d<0x4e>(v);
    return v + dpp_d<0x141>(v);
}

// The XOR-4/2/1 tree of 8 lanes, ((l0+l4)+(l2+l6)) + ((l1+l5)+(l3+l7)),
// complete in the LAST lane of each group of 8 (row shifts by 4, 2, 1;
// f32 addition is commutative, so the operand swaps change no bit).
__device__ __forceinline__ float group8_tree_last(float v) {
    v += dpp_f<0x114>(v);  // row_shr:4
    v += dpp_f<0x112>(v);  // row_shr:2
    return v + dpp_f<0x111>(v);  // row_shr:1
}

// Max / sum over aligned groups of 8 lanes, the result in every lane.
__device__ __forceinline__ float group8_max_all(float v) {
    v = fmaxf(v, dpp_f<kDppXor1>(v));
    v = fmaxf(v, dpp_f<kDppXor2>(v));
    return fmaxf(v, dpp_f<kDppHalfMirror>(v));
}
__device__ __forceinline__ float group8_sum_all(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    return v + dpp_f<kDppHalfMirror>(v);
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS
// operations, not for its outstanding global loads, which stay in flight
// across it (__syncthreads waits for those too).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ float wave_max(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// Streaming 16-byte load that bypasses cache retention (weights are read
// exactly once per launch).
__device__ __forceinline__ v4i load_nt(const void* p) {
    return __builtin_nontemporal_load((const v4i*)p);
}

// Q4_K device layout: tiles of 16 rows in the int8 MFMA operand order.  The
// 64 bytes of unit q (elements 128q .. 128q+127) of rows 16t .. 16t+15 form
// 1 KB at (t * K/128 + q) * 1024, with the 16-byte piece s (bytes 16s ..
// 16s+15 of the unit) of row 16t + j at (j + 16 s) * 16 inside it, so one
// wave instruction (lane j + 16 s) reads 1 KB contiguously; rows past N up
// to the tile are zero.  Within a row the GGUF payload order is kept: byte e
// of 64-element chunk c holds element 64c + e in its low nibble and
// 64c + 32 + e in its high nibble.  Byte offset of bytes 0..15 of chunk c of
// `row` (bytes 16..31 follow 256 bytes later):
__host__ __device__ __forceinline__ size_t q4k_chunk_offset(size_t row, size_t c, size_t K) {
    return (((row >> 4) * (K >> 7) + (c >> 1)) * 64 + (row & 15) + 32 * (c & 1)) * 16;
}
// Headers [tiles][K/256 blocks][16 rows] x 16 bytes: index of (row, block).
__host__ __device__ __forceinline__ size_t q4k_hdr_index(size_t row, size_t blk, size_t nbk) {
    return ((row >> 4) * nbk + blk) * 16 + (row & 15);
}

// Q8_0 device layout: tiles of 8 rows x 4 blocks, one 16-byte slot per
// (row % 8, lane-of-block l) holding bytes 4l..4l+3 of the 4 blocks, so the
// 64 lanes of a wavefront read one contiguous 1 KB tile.  Byte offset of
// the 4-byte group l of block b of row `row`:
__device__ __forceinline__ size_t q8_tile_offset(size_t row, size_t b, int l, size_t nbc) {
    return (((row >> 3) * nbc + (b >> 2)) * 64 + (row & 7) * 8 + l) * 16 + (b & 3) * 4;
}

// Q4_1 device layout.  Rows in tiles of 8, blocks in chunks of 8: lane
// (row % 8) * 8 + l of a tile holds, per chunk, 16 bytes = eight 16-bit
// words, word bi = the four nibbles of elements 4l..4l+3 of block 8c+bi
// (element e of a GGUF block is the low nibble of byte e for e < 16, else
// the high nibble of byte e-16), nibble j in bits 4j..4j+3.  A wavefront
// reads one contiguous 1 KB run per chunk.  Headers: uint32 d | m << 16 per
// (row, block), rows padded to 8 blocks.  nbc8 = ceil(K/32 / 8).
__host__ __device__ __forceinline__ size_t q41_word_index(size_t row, size_t b, int l, size_t nbc8) {
    return (((row >> 3) * nbc8 + (b >> 3)) * 64 + (row & 7) * 8 + l) * 8 + (b & 7);
}

// Q6_K device layout.  Rows in tiles of 8; per superblock lane (row % 8) * 8
// + L holds the bits of the 32 elements whose position in their 32-group is
// 4L..4L+3 (the reference's Q6_K x Q8_K lane):
//   plane A, 4 dwords: ql bytes 4L.., 32+4L.. (first half), 64+4L..,
//     96+4L.. (second half) -- low nibble = group 0/1, high = group 2/3;
//   plane B, 2 dwords: qh bytes 4L.. (first half), 32+4L.. (second half),
//     2 bits per group.
// Headers: the 16 int8 local scales per (row, superblock), then f32 d.
__host__ __device__ __forceinline__ size_t q6k_a_index(size_t row, size_t sb, int L, size_t nsb) {
    return (((row >> 3) * nsb + sb) * 64 + (row & 7) * 8 + L) * 4;  // in dwords
}
__host__ __device__ __forceinline__ size_t q6k_b_index(size_t row, size_t sb, int L, size_t nsb) {
    return (((row >> 3) * nsb + sb) * 64 + (row & 7) * 8 + L) * 2;  // in dwords
}
__host__ __device__ __forceinline__ size_t q6k_b_offset(size_t N, size_t K) {  // plane B after plane A, in dwords
    return (N + 7) / 8 * (K / 256) * 64 * 4;
}

// Exact element decoders over the layouts above (codecs/q4.rs:22-36 Q4_1:
// fma(q, d, m); codecs/q6.rs:6-34 Q6_K: (d * scale) * (code - 32)).
__device__ __forceinline__ float q41_element(const uint16_t* qs, const uint32_t* hdr, size_t row, size_t e, size_t K) {
    const size_t nb = K / 32, nbc8 = (nb + 7) / 8, b = e / 32;
    const int i = (int)(e % 32);
    const uint32_t word = qs[q41_word_index(row, b, i >> 2, nbc8)];
    const float q = (float)((word >> (4 * (i & 3))) & 15u);
    const uint32_t h = hdr[row * nbc8 * 8 + b];
    return fmaf(q, f16_to_f32((uint16_t)(h & 0xffffu)), f16_to_f32((uint16_t)(h >> 16)));
}

__device__ __forceinline__ float q6k_element(const uint32_t* qs, const uint8_t* scales, const float* d, size_t row,
                                             size_t e, size_t N, size_t K) {
    const size_t nsb = K / 256, sb = e / 256;
    const int at = (int)(e % 256), half = at >> 7, group = (at >> 5) & 3, l32 = at & 31;
    const int L = l32 >> 2, j = l32 & 3;
    const uint32_t a = qs[q6k_a_index(row, sb, L, nsb) + half * 2 + (group & 1)];
    const uint32_t hb = qs[q6k_b_offset(N, K) + q6k_b_index(row, sb, L, nsb) + half];
    const uint32_t lo = (a >> (8 * j + (group >= 2 ? 4 : 0))) & 15u;
    const uint32_t hi = (hb >> (8 * j + 2 * group)) & 3u;
    const int code = (int)(lo | (hi << 4)) - 32;
    const float sc = (float)(int8_t)scales[(row * nsb + sb) * 16 + half * 8 + group * 2 + l32 / 16];
    return (d[row * nsb + sb] * sc) * (float)code;
}

// Q4_K header relayout.  GGUF packs 8 six-bit scales and 8 six-bit mins into
// 12 bytes (codecs/q4.rs:58-65), which forces a lane-dependent multi-byte
// gather per group.  The device header keeps d and dmin (bytes 0-3) and
// stores the four values of group pair p (sc[2p], mn[2p], sc[2p+1],
// mn[2p+1]) in byte p of dwords 1..3:
//   dw1.byte[p] = sc[2p]   | (mn[2p+1] & 3) << 6
//   dw2.byte[p] = mn[2p]   | ((mn[2p+1] >> 2) & 3) << 6
//   dw3.byte[p] = sc[2p+1] | ((mn[2p+1] >> 4) & 3) << 6
// so a lane decodes its pair with three fixed-offset byte extracts.  The
// mapping is a bijection of the same 96 bits: no information is added or lost.
__device__ __forceinline__ void q4k_dev_scale_min(const v4u h, int g, uint32_t& sc, uint32_t& mn) {
    const int sh = 8 * (g >> 1);
    const uint32_t b1 = (h.y >> sh) & 0xffu, b2 = (h.z >> sh) & 0xffu, b3 = (h.w >> sh) & 0xffu;
    if ((g & 1) == 0) {
        sc = b1 & 63;
        mn = b2 & 63;
    } else {
        sc = b3 & 63;
        mn = (b1 >> 6) | ((b2 >> 6) << 2) | ((b3 >> 6) << 4);
    }
}

}  // namespace zg
