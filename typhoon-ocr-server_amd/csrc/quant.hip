// quant.hip -- per-row symmetric int8 quantization and weight tile packing.
//
// quantize_rows_kernel restates the reference quantizers on the GPU, bit for
// bit (kernel/w8a32_kernel.c:63-108 w8a32_quantize, :139-178
// _quantize_activation_i8; kernel/w8a8_kernel.c:54-100 _quantize_rows;
// kernel/w8a16_kernel.c:44-65 w8a16_quantize_weights):
//   absmax = max|x|     (NaN-propagating over the 16-aligned prefix, a
//                        NaN-ignoring scan over the K%16 tail)
//   scale  = absmax > 0 ? fl(absmax/127) : 1,   inv = fl(1/scale)
//   code   = k < K&~15 ? rne(fl(x*inv)) : round-half-away(fl(x*inv)),
//            clamped to [-127,127] (the activation quantizer of the M=1 GEMV
//            only saturates to [-128,127]; |x*inv| <= 127(1+3 eps) makes the
//            two identical)
// One work-group of 256 threads per row: pass 1 reduces the absmax, pass 2
// re-reads the (L2-resident) row and writes codes.
//
// quantize_rows_tiled_kernel does the same with one wave per row and writes
// the codes straight into the 16x64 tile layout used as the int8 MFMA A
// operand.
//
// pack_tiles_kernel re-lays a row-major int8 matrix into 16x64 tiles.
#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

__global__ __launch_bounds__(256) void quantize_rows_kernel(const float* __restrict__ src,
                                                            int8_t* __restrict__ dst,
                                                            float* __restrict__ scales, int cols,
                                                            int clamp127) {
  __shared__ uint32_t s_mx[4];
  __shared__ float s_tail[4];
  const int r = blockIdx.x;
  const float* row = src + (size_t)r * cols;
  int8_t* out = dst + (size_t)r * cols;
  const int main_end = cols & ~15;
  const bool vec = ((cols & 3) == 0) && ((((uintptr_t)row) & 15) == 0);

  uint32_t mx = 0;
  float tail = 0.0f;
  if (vec) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    for (int i = threadIdx.x; i < (main_end >> 2); i += 256) {
      float4 v = r4[i];
      uint32_t a = max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w)));
      mx = a > mx ? a : mx;
    }
  } else {
    for (int k = threadIdx.x; k < main_end; k += 256) {
      uint32_t a = abs_bits(row[k]);
      mx = a > mx ? a : mx;
    }
  }
  for (int k = main_end + threadIdx.x; k < cols; k += 256) {
    float a = fabsf(row[k]);
    tail = (a > tail) ? a : tail;
  }
  const float absmax = block_absmax_256(mx, tail, s_mx, s_tail);
  const float scale = quant_scale(absmax);
  const float inv = quant_inv(scale);
  if (threadIdx.x == 0) scales[r] = scale;

  const bool c127 = clamp127 != 0;
  if (vec && ((((uintptr_t)out) & 3) == 0)) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    uint32_t* o4 = reinterpret_cast<uint32_t*>(out);
    for (int i = threadIdx.x; i < (cols >> 2); i += 256) {
      float4 v = r4[i];
      int k = i << 2;
      o4[i] = pack4(code_at(v.x, inv, k, cols, c127), code_at(v.y, inv, k + 1, cols, c127),
                    code_at(v.z, inv, k + 2, cols, c127), code_at(v.w, inv, k + 3, cols, c127));
    }
  } else {
    for (int k = threadIdx.x; k < cols; k += 256)
      out[k] = (int8_t)code_at(row[k], inv, k, cols, c127);
  }
}

// One wave per row, 4 rows per work-group; codes are written straight into
// the 16x64 tile layout (row r -> tile lanes (r & 15) + 16 lg), zero beyond K.
// Lane l owns the 16-wide chunks c = l + 64 j of the row (64 contiguous bytes
// of x each): with CH > 0 all CH chunks are loaded at once and kept in
// registers, so the row is read once; CH == 0 is the generic two-pass loop.
template <int CH>
__global__ __launch_bounds__(256) void quantize_rows_tiled_kernel(const float* __restrict__ src,
                                                                  int rows, int cols, int KB,
                                                                  uint8_t* __restrict__ tiles,
                                                                  float* __restrict__ scales,
                                                                  int clamp127) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int MG = cdiv(rows, 16);
  if (r >= rows) return;
  const float* row = src + (size_t)r * cols;
  const int main_end = cols & ~15;
  const bool c127 = clamp127 != 0;
  uint4* t4 = reinterpret_cast<uint4*>(tiles) + (size_t)(r >> 4) * 64 + (r & 15);

  auto store_chunk = [&](int c, const float* x, float inv) {
    const int k0 = c * 16;
    int q[16];
#pragma unroll
    for (int j = 0; j < 16; j++) q[j] = (k0 + j < cols) ? code_at(x[j], inv, k0 + j, cols, c127) : 0;
    uint4 o;
    o.x = pack4(q[0], q[1], q[2], q[3]);
    o.y = pack4(q[4], q[5], q[6], q[7]);
    o.z = pack4(q[8], q[9], q[10], q[11]);
    o.w = pack4(q[12], q[13], q[14], q[15]);
    t4[(size_t)(c >> 2) * MG * 64 + 16 * (c & 3)] = o;
  };

  if constexpr (CH > 0) {
    // cols == 1024 * CH, row 16-byte aligned
    float4 v[CH][4];
#pragma unroll
    for (int j = 0; j < CH; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) v[j][e] = reinterpret_cast<const float4*>(row)[(lane + 64 * j) * 4 + e];
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < CH; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float4 f = v[j][e];
        const uint32_t m4 = max(max(abs_bits(f.x), abs_bits(f.y)), max(abs_bits(f.z), abs_bits(f.w)));
        mx = m4 > mx ? m4 : mx;
      }
    mx = wave_max_u32(mx);
    const float scale = quant_scale(__uint_as_float(mx));
    const float inv = quant_inv(scale);
    if (lane == 0) scales[r] = scale;
#pragma unroll
    for (int j = 0; j < CH; j++) {
      float x[16];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        x[4 * e] = v[j][e].x; x[4 * e + 1] = v[j][e].y; x[4 * e + 2] = v[j][e].z; x[4 * e + 3] = v[j][e].w;
      }
      store_chunk(lane + 64 * j, x, inv);
    }
  } else {
    uint32_t mx = 0;
    float tail = 0.0f;
    for (int k = lane; k < main_end; k += 64) {
      const uint32_t a = abs_bits(row[k]);
      mx = a > mx ? a : mx;
    }
    for (int k = main_end + lane; k < cols; k += 64) {
      const float a = fabsf(row[k]);
      tail = (a > tail) ? a : tail;
    }
    mx = wave_max_u32(mx);
    tail = wave_maxf_nonnan(tail);
    const float vmax = __uint_as_float(mx);
    const float absmax = (tail > vmax) ? tail : vmax;
    const float scale = quant_scale(absmax);
    const float inv = quant_inv(scale);
    if (lane == 0) scales[r] = scale;
    for (int c = lane; c < KB * 4; c += 64) {
      const int k0 = c * 16;
      float x[16];
#pragma unroll
      for (int j = 0; j < 16; j++) x[j] = (k0 + j < cols) ? row[k0 + j] : 0.0f;
      store_chunk(c, x, inv);
    }
  }
}

// One wave per row, 4 rows per work-group, for rows of cols == 256 NV floats
// (16-byte aligned): lane l loads float4 l + 64 j (every load instruction
// reads 1 KiB contiguous), the absmax is reduced with DPP, and each lane
// writes the 4 codes of each of its float4 as one dword at its place in the
// 16x64 tile layout (4 consecutive lanes fill one 16-byte tile lane).
template <int NV>
__global__ __launch_bounds__(256) void quantize_rows_tiled_vec_kernel(const float* __restrict__ src, int rows,
                                                                      int cols, int MG,
                                                                      uint8_t* __restrict__ tiles,
                                                                      float* __restrict__ scales, int clamp127) {
  const int lane = threadIdx.x & 63;
  // rows 4 quad .. 4 quad + 3; the two quads whose codes share each 128-byte
  // tile line (8 rows) run on one XCD (work-group b on XCD b % 8), so their
  // partial-line stores merge in its L2; a bijection of [0, 16 n) work-groups
  const int x = blockIdx.x & 7, jj = blockIdx.x >> 3;
  const int quad = 16 * (jj >> 1) + 2 * x + (jj & 1);
  const int r = quad * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;
  const float4* row = reinterpret_cast<const float4*>(src + (size_t)r * cols);
  float4 v[NV];
#pragma unroll
  for (int j = 0; j < NV; j++) v[j] = row[lane + 64 * j];
  uint32_t mx = 0;
#pragma unroll
  for (int j = 0; j < NV; j++)
    mx = max(mx, max(max(abs_bits(v[j].x), abs_bits(v[j].y)), max(abs_bits(v[j].z), abs_bits(v[j].w))));
  mx = wave_umax(mx);
  const float scale = quant_scale(__uint_as_float(mx));
  const float inv = quant_inv(scale);
  if (lane == 0) scales[r] = scale;
  const bool fast = mx < 0x7f800000u && (__float_as_uint(inv) & 0x7f800000u) != 0x7f800000u;
  const bool c127 = clamp127 != 0;
  uint32_t* t32 = reinterpret_cast<uint32_t*>(tiles) + ((size_t)(r >> 4) * 64 + (r & 15)) * 4;
#pragma unroll
  for (int j = 0; j < NV; j++) {
    const int f = lane + 64 * j;          // float4 index: k = 4f .. 4f+3
    // finite absmax and reciprocal: |x * inv| <= 127 (1 + 2^-22), so the
    // codes lie in [-127, 127] and the weight clamp changes nothing
    const uint32_t code = fast ? codes4_rne(v[j], inv)
                               : pack4(code_rne(v[j].x * inv, c127), code_rne(v[j].y * inv, c127),
                                       code_rne(v[j].z * inv, c127), code_rne(v[j].w * inv, c127));
    // chunk c = f >> 2 (16 k): tile kb = f >> 4, lane group (f >> 2) & 3,
    // dword f & 3 of that tile lane
    t32[((size_t)(f >> 4) * MG) * 256 + ((f >> 2) & 3) * 64 + (f & 3)] = code;
  }
}

// fp32 token rows -> four int8 planes each (the A operand of W8A32 batches on
// the int8 MFMA).  One wave per token t:
//   e = frexp exponent of the row's absmax - 6, v = x 2^-e (exact), |v| < 64;
//   q0 = rint(v), r0 = v - q0 (exact), then q_p = rint(254 r_{p-1}) with
//   r_p = 254 r_{p-1} - q_p for p = 1..3 (|254 r| <= 127: every q fits int8).
// So x = 2^e (q0 + q1/254 + q2/254^2 + q3/254^3 + d) with |d| below
// 2^-26 of 64 (the rounding of 254 r and the last residual): about 2^-32 of
// the row's absmax.  Plane p of token t is code row 4t + p of the 16x64 tile
// array (each lane writes one dword per plane for its 4 consecutive k; k past
// K inside the last k-block gets zero codes).  A row holding Inf or NaN gets
// xe = kXeNonFinite and zero codes.
__global__ __launch_bounds__(256) void split_i8x4_kernel(const float* __restrict__ X, int ldx, int M, int K,
                                                         int KB, int MG, uint8_t* __restrict__ tiles,
                                                         int* __restrict__ xe) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= M) return;
  const float* row = X + (size_t)t * ldx;
  const bool vec = ((((uintptr_t)row) & 15) == 0);
  const int nf = KB * 16;                      // float4 groups in the padded row
  uint32_t mx = 0;
  for (int f = lane; f < nf; f += 64) {
    const int k = 4 * f;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (vec && k + 4 <= K) {
      v = *reinterpret_cast<const float4*>(row + k);
    } else {
      if (k < K) v.x = row[k];
      if (k + 1 < K) v.y = row[k + 1];
      if (k + 2 < K) v.z = row[k + 2];
      if (k + 3 < K) v.w = row[k + 3];
    }
    mx = max(mx, max(max(abs_bits(v.x), abs_bits(v.y)), max(abs_bits(v.z), abs_bits(v.w))));
  }
  mx = wave_umax(mx);
  const bool finite = mx < 0x7f800000u;
  const int ee = planes_exponent(mx);
  const int e = finite ? ee : 0;
  if (lane == 0) xe[t] = ee;
  // tile dword of plane p for float4 group f: row 4t + p of group (4t + p) >> 4
  uint32_t* t32 = reinterpret_cast<uint32_t*>(tiles);
  const int r0 = 4 * t;
  for (int f = lane; f < nf; f += 64) {
    const int k = 4 * f;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (finite) {
      if (vec && k + 4 <= K) {
        const float4 u = *reinterpret_cast<const float4*>(row + k);
        v[0] = u.x; v[1] = u.y; v[2] = u.z; v[3] = u.w;
      } else {
#pragma unroll
        for (int q = 0; q < 4; q++) v[q] = (k + q < K) ? row[k + q] : 0.0f;
      }
    }
    uint32_t code[4];
    planes4_i8(v, e, code);
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int rr = r0 + p;
      // k-block f >> 4, tile lane (rr & 15) + 16 ((f >> 2) & 3), dword f & 3
      t32[(((size_t)(f >> 4) * MG + (rr >> 4)) * 64 + (rr & 15) + 16 * ((f >> 2) & 3)) * 4 + (f & 3)] = code[p];
    }
  }
}

hipError_t launch_split_i8x4(const float* X, int ldx, int M, int K, uint8_t* tiles, int* xe, hipStream_t st) {
  if (M <= 0 || K <= 0 || ldx < K || !X || !tiles || !xe) return hipErrorInvalidValue;
  const int KB = cdiv(K, 64), MG = cdiv(4 * M, 16);
  hipLaunchKernelGGL(split_i8x4_kernel, dim3(cdiv(M, 4)), dim3(256), 0, st, X, ldx, M, K, KB, MG, tiles, xe);
  return hipGetLastError();
}

// one thread per (tile, lane): 16 bytes of W[16g + (l&15)][64kb + 16(l>>4) ..]
// for the row groups of rows [0, rows) of w, written as row groups g0 .. of a
// tile array with NGt row groups per k-block (g0 = 0, NGt = NG for a whole
// matrix; a row chunk starting at row 16 g0 of a larger one otherwise)
__global__ __launch_bounds__(256) void pack_tiles_kernel(const int8_t* __restrict__ w, int rows,
                                                         int cols, int KB, long long total, int NGt,
                                                         int g0, uint8_t* __restrict__ tiles) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const int lane = (int)(t & 63);
  const long long tile = t >> 6;               // k-block-major: tile = kb * NG + g
  const int NG = (rows + 15) / 16;
  const int g = (int)(tile % NG);
  const int kb = (int)(tile / NG);
  const int r = g * 16 + (lane & 15);
  const int k0 = kb * 64 + (lane >> 4) * 16;
  uint4 q = make_uint4(0, 0, 0, 0);
  if (r < rows) {
    const int8_t* p = w + (size_t)r * cols + k0;
    if (k0 + 16 <= cols && ((((uintptr_t)p) & 15) == 0)) {
      q = *reinterpret_cast<const uint4*>(p);
    } else {
      uint8_t b[16];
#pragma unroll
      for (int j = 0; j < 16; j++) b[j] = (k0 + j < cols) ? (uint8_t)p[j] : 0;
      q.x = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
      q.y = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
      q.z = b[8] | (b[9] << 8) | (b[10] << 16) | ((uint32_t)b[11] << 24);
      q.w = b[12] | (b[13] << 8) | (b[14] << 16) | ((uint32_t)b[15] << 24);
    }
  }
  reinterpret_cast<uint4*>(tiles)[((size_t)kb * NGt + g0 + g) * 64 + lane] = q;
}

// inverse of pack_tiles_kernel over a whole matrix: tiles -> row-major codes
__global__ __launch_bounds__(256) void unpack_tiles_kernel(const uint8_t* __restrict__ tiles, int rows,
                                                           int cols, int KB, long long total,
                                                           int8_t* __restrict__ w) {
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const int lane = (int)(t & 63);
  const long long tile = t >> 6;
  const int NG = (rows + 15) / 16;
  const int g = (int)(tile % NG);
  const int kb = (int)(tile / NG);
  const int r = g * 16 + (lane & 15);
  const int k0 = kb * 64 + (lane >> 4) * 16;
  if (r >= rows || k0 >= cols) return;
  const uint4 q = reinterpret_cast<const uint4*>(tiles)[t];
  int8_t* p = w + (size_t)r * cols + k0;
  if (k0 + 16 <= cols && ((((uintptr_t)p) & 15) == 0)) {
    *reinterpret_cast<uint4*>(p) = q;
  } else {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    for (int j = 0; j < 16 && k0 + j < cols; j++) p[j] = (int8_t)((d[j >> 2] >> (8 * (j & 3))) & 0xff);
  }
}

// Word copy, used to bring a small host-resident (pinned, device-mapped)
// vector into HBM with one kernel instead of a DMA transfer: 16 bytes per
// thread where both sides are 16-byte aligned, 4 bytes otherwise.
__global__ __launch_bounds__(256) void copy_words_kernel(const uint32_t* __restrict__ src,
                                                         uint32_t* __restrict__ dst, long long n, int vec) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (vec) {
    const long long n4 = n >> 2;
    if (i < n4) reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    const long long t = (n4 << 2) + i;
    if (i < (n & 3)) dst[t] = src[t];
  } else if (i < n) {
    dst[i] = src[i];
  }
}

// Byte copy with zero padding: dst[i] = src[i] for i < n, 0 for n <= i < npad
// (src may be null when n == 0).  Clears or pads a small code vector inside
// the stream's kernel order, so that a caller capturing the call into a HIP
// graph records a kernel node rather than a memset node.
__global__ __launch_bounds__(256) void copy_pad_bytes_kernel(const uint8_t* __restrict__ src, long long n,
                                                             uint8_t* __restrict__ dst, long long npad) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i < npad) dst[i] = i < n ? src[i] : (uint8_t)0;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_copy_pad_bytes(const void* src, size_t n, void* dst, size_t npad, hipStream_t st) {
  if (npad == 0) return hipSuccess;
  if (!dst || n > npad || (n > 0 && !src)) return hipErrorInvalidValue;
  const long long blocks = ((long long)npad + 255) / 256;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(copy_pad_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                     static_cast<const uint8_t*>(src), (long long)n, static_cast<uint8_t*>(dst), (long long)npad);
  return hipGetLastError();
}

hipError_t launch_copy_words(const void* src, void* dst, size_t bytes, hipStream_t st) {
  if (bytes == 0) return hipSuccess;
  if (bytes & 3) return hipErrorInvalidValue;
  const long long n = (long long)(bytes >> 2);
  const int vec = ((((uintptr_t)src) | ((uintptr_t)dst)) & 15) == 0 ? 1 : 0;
  const long long threads = vec ? ((n >> 2) > 4 ? (n >> 2) : 4) : n;
  const long long blocks = (threads + 255) / 256;
  hipLaunchKernelGGL(copy_words_kernel, dim3((unsigned)blocks), dim3(256), 0, st,
                     static_cast<const uint32_t*>(src), static_cast<uint32_t*>(dst), n, vec);
  return hipGetLastError();
}

hipError_t launch_quantize_rows(const float* src, int8_t* dst, float* scales, int rows, int cols,
                                bool clamp127, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  hipLaunchKernelGGL(quantize_rows_kernel, dim3(rows), dim3(256), 0, st, src, dst, scales, cols,
                     clamp127 ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_quantize_rows_tiled(const float* src, int rows, int cols, uint8_t* tiles,
                                      float* scales, bool clamp127, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  const int KB = cdiv(cols, 64);
  const dim3 grid(cdiv(rows, 4)), block(256);
  const int c = clamp127 ? 1 : 0;
  const bool aligned = (((uintptr_t)src) & 15) == 0;
  const int MG = cdiv(rows, 16);
  const dim3 vgrid(cdiv(rows, 64) * 16);   // whole groups of 16 quads of rows
  if (aligned && cols == 2048)
    hipLaunchKernelGGL(quantize_rows_tiled_vec_kernel<8>, vgrid, block, 0, st, src, rows, cols, MG, tiles, scales, c);
  else if (aligned && cols == 6144)
    hipLaunchKernelGGL(quantize_rows_tiled_vec_kernel<24>, vgrid, block, 0, st, src, rows, cols, MG, tiles, scales, c);
  else if (aligned && cols == 1024)
    hipLaunchKernelGGL(quantize_rows_tiled_vec_kernel<4>, vgrid, block, 0, st, src, rows, cols, MG, tiles, scales, c);
  else if (aligned && cols == 4096)
    hipLaunchKernelGGL(quantize_rows_tiled_vec_kernel<16>, vgrid, block, 0, st, src, rows, cols, MG, tiles, scales, c);
  else
    hipLaunchKernelGGL(quantize_rows_tiled_kernel<0>, grid, block, 0, st, src, rows, cols, KB, tiles, scales, c);
  return hipGetLastError();
}

hipError_t launch_pack_tiles_rows(const int8_t* w, int rows, int cols, int NGt, int g0, uint8_t* tiles,
                                  hipStream_t st) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  if (g0 < 0 || g0 + cdiv(rows, 16) > NGt) return hipErrorInvalidValue;
  const int KB = cdiv(cols, 64);
  const long long total = (long long)cdiv(rows, 16) * KB * 64;
  const long long blocks = (total + 255) / 256;
  hipLaunchKernelGGL(pack_tiles_kernel, dim3((unsigned)blocks), dim3(256), 0, st, w, rows, cols, KB,
                     total, NGt, g0, tiles);
  return hipGetLastError();
}

hipError_t launch_pack_tiles(const int8_t* w, int rows, int cols, uint8_t* tiles, hipStream_t st) {
  return launch_pack_tiles_rows(w, rows, cols, cdiv(rows, 16), 0, tiles, st);
}

hipError_t launch_unpack_tiles(const uint8_t* tiles, int rows, int cols, int8_t* w, hipStream_t st) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  const int KB = cdiv(cols, 64);
  const long long total = (long long)cdiv(rows, 16) * KB * 64;
  const long long blocks = (total + 255) / 256;
  hipLaunchKernelGGL(unpack_tiles_kernel, dim3((unsigned)blocks), dim3(256), 0, st, tiles, rows, cols, KB,
                     total, w);
  return hipGetLastError();
}

}  // namespace tl

// ---------------------------------------------------------------------------
// C ABI of the launchers above (tl_kernels.h)
// ---------------------------------------------------------------------------
extern "C" {
hipError_t tlk_launch_quantize_rows(const float* src, int8_t* dst, float* scales, int rows, int cols,
                                    bool clamp127, hipStream_t st) {
  return tl::launch_quantize_rows(src, dst, scales, rows, cols, clamp127, st);
}
hipError_t tlk_launch_quantize_rows_tiled(const float* src, int rows, int cols, uint8_t* tiles, float* scales,
                                          bool clamp127, hipStream_t st) {
  return tl::launch_quantize_rows_tiled(src, rows, cols, tiles, scales, clamp127, st);
}
hipError_t tlk_launch_pack_tiles(const int8_t* w, int rows, int cols, uint8_t* tiles, hipStream_t st) {
  return tl::launch_pack_tiles(w, rows, cols, tiles, st);
}
hipError_t tlk_launch_pack_tiles_rows(const int8_t* w, int rows, int cols, int NGt, int g0, uint8_t* tiles,
                                      hipStream_t st) {
  return tl::launch_pack_tiles_rows(w, rows, cols, NGt, g0, tiles, st);
}
hipError_t tlk_launch_unpack_tiles(const uint8_t* tiles, int rows, int cols, int8_t* w, hipStream_t st) {
  return tl::launch_unpack_tiles(tiles, rows, cols, w, st);
}
hipError_t tlk_launch_split_i8x4(const float* X, int ldx, int M, int K, uint8_t* tiles, int* xe, hipStream_t st) {
  return tl::launch_split_i8x4(X, ldx, M, K, tiles, xe, st);
}
hipError_t tlk_launch_copy_words(const void* src, void* dst, size_t bytes, hipStream_t st) {
  return tl::launch_copy_words(src, dst, bytes, st);
}
hipError_t tlk_launch_copy_pad_bytes(const void* src, size_t n, void* dst, size_t npad, hipStream_t st) {
  return tl::launch_copy_pad_bytes(src, n, dst, npad, st);
}
}  // extern "C"
