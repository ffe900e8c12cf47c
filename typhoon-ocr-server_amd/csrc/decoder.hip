// decoder.hip -- the decode-step kernels around the linear layers.
//
// Reference: kernel/decoder.c:33-157 (decoder_layer_forward, DECODE_MODE).
// The linear layers run on gemv_i8_kernel with the layer's other steps fused
// around them (RMSNorm prologues, the residual add as the GEMV bias, SwiGLU
// as an epilogue); what remains for this file is
//   attn_decode_kernel   per-head QK RMSNorm (q_norm / k_norm), M-RoPE at the
//                        decode position, the KV cache append of the new
//                        token, and split-sequence GQA attention partials
//                        (kernel/ops.c:233-289, kernel/kv_cache.c:53-64,
//                        kernel/attention.c:172-224);
//   attn_combine_kernel  the softmax-weighted merge of the partials;
//   step_end_kernel      greedy token from the lm_head argmax keys, the next
//                        step's embedding row, the position advance
//                        (decoder.py:463-464 and :501-504, kv_cache.c:108-112).
//
// Decode state lives in device memory (int32): [0] positions in the cache
// (the new K/V go there), [1] rotary position, [2] generated-token counter.
// Every kernel reads it at run time, so one captured step replays for every
// token.
//
// KV cache: per layer and kv head [max_seq][128] fp32 (head-first, as the
// reference's kv_cache.c), K and V in separate arrays.
#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

constexpr int HD = 128;          // head dim
constexpr int ATT_T = 64;        // positions per attention work-group

// RMSNorm of one 128-wide head held one element per thread by the 128
// threads [g*128, g*128 + 128) (two waves): sum of squares through DPP and
// LDS, rsqrt as the reference computes it (FRSQRTE + two Newton steps),
// x * r * w.  s_two: 2 floats of LDS per head slot.  Called by all threads of
// the work-group (it has a barrier).
__device__ __forceinline__ float head_rmsnorm(float v, float w, float* s_two, float eps) {
  float sq = __fmul_rn(v, v);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sq = __fadd_rn(sq, __shfl_xor(sq, o, 64));
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_two[wv] = sq;
  __syncthreads();
  const int w0 = wv & ~1;
  const float tot = __fadd_rn(s_two[w0], s_two[w0 + 1]);
  const float r = ref_rsqrt(__fadd_rn(__fdiv_rn(tot, (float)HD), eps));
  return __fmul_rn(__fmul_rn(v, r), w);
}

// rotate_half at one position: element d of a head held in s_head[0..127]
__device__ __forceinline__ float rope_at(const float* s_head, int d, const float* co, const float* si) {
  const int j = d & 63;
  const float lo = s_head[j], hi = s_head[j + 64];
  const float c = co[j], s = si[j];
  return d < 64 ? __fsub_rn(__fmul_rn(lo, c), __fmul_rn(hi, s)) : __fadd_rn(__fmul_rn(hi, c), __fmul_rn(lo, s));
}

// Work-group (c, h): kv head h, positions [64 c, 64 c + 64) of the S = len + 1
// that the new token attends to; two q heads (GQA group 2).  256 threads:
// thread t holds element t & 127 of q head 2h + (t >> 7).
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecodeArgs a) {
  const int c = blockIdx.x, h = blockIdx.y;
  const int p = a.state[0];                 // position of the new token
  const int S = p + 1;
  const int t0 = c * ATT_T;
  if (t0 >= S) return;                      // uniform: the whole work-group leaves
  const int t1 = min(t0 + ATT_T, S);
  const int rp = a.state[1];
  const float* co = a.cos_tab + (size_t)rp * 64;
  const float* si = a.sin_tab + (size_t)rp * 64;

  __shared__ float s_x[2][HD];              // normalised heads before the rotation
  __shared__ float s_q[2][HD];              // rotated q heads
  __shared__ float s_k[HD], s_v[HD];        // the new token's k (rotated) and v
  __shared__ float s_red[4];
  __shared__ float s_p[2][ATT_T];           // scores, then probabilities

  const int tid = threadIdx.x, g = tid >> 7, d = tid & 127;
  const int lane = tid & 63, wv = tid >> 6;
  const bool has_new = p < t1;              // this chunk holds position p

  // q: RMSNorm with q_norm, then the rotation
  const float qn = head_rmsnorm(a.qkv[(2 * h + g) * HD + d], a.q_norm[d], s_red, a.eps);
  s_x[g][d] = qn;
  __syncthreads();
  s_q[g][d] = rope_at(s_x[g], d, co, si);
  __syncthreads();

  if (has_new) {
    // threads 0-127: k of kv head h (k_norm, rotation); 128-255: v
    const float* kv_src = a.qkv + a.nq * HD + (g == 0 ? h * HD : a.nkv * HD + h * HD);
    const float raw = kv_src[d];
    const float kn = head_rmsnorm(raw, a.k_norm[d], s_red, a.eps);   // all threads; g == 1 unused
    if (g == 0) s_x[0][d] = kn;
    __syncthreads();
    const size_t off = ((size_t)h * a.max_seq + p) * HD + d;
    if (g == 0) {
      const float kr = rope_at(s_x[0], d, co, si);
      s_k[d] = kr;
      a.kc[off] = kr;
    } else {
      s_v[d] = raw;
      a.vc[off] = raw;
    }
    __syncthreads();
  }

  // scores: 16 lanes per position (8 elements each), 4 positions per wave
  // instruction, wave w takes positions t0 + 16 w .. t0 + 16 w + 15
  const int seg = lane & 15;
  float q0[8], q1[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    q0[i] = s_q[0][seg * 8 + i];
    q1[i] = s_q[1][seg * 8 + i];
  }
  const float* kbase = a.kc + (size_t)h * a.max_seq * HD;
#pragma unroll
  for (int it = 0; it < 4; it++) {
    const int t = t0 + wv * 16 + it * 4 + (lane >> 4);
    float kv8[8];
    if (t < t1 && t != p) {
      const float4* kp = reinterpret_cast<const float4*>(kbase + (size_t)t * HD + seg * 8);
      const float4 k0 = kp[0], k1 = kp[1];
      kv8[0] = k0.x; kv8[1] = k0.y; kv8[2] = k0.z; kv8[3] = k0.w;
      kv8[4] = k1.x; kv8[5] = k1.y; kv8[6] = k1.z; kv8[7] = k1.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) kv8[i] = (t == p) ? s_k[seg * 8 + i] : 0.0f;
    }
    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      d0 = __fmaf_rn(q0[i], kv8[i], d0);
      d1 = __fmaf_rn(q1[i], kv8[i], d1);
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      d0 = __fadd_rn(d0, __shfl_xor(d0, o, 64));
      d1 = __fadd_rn(d1, __shfl_xor(d1, o, 64));
    }
    if (seg == 0 && t < t1) {
      s_p[0][t - t0] = __fmul_rn(d0, a.scale);
      s_p[1][t - t0] = __fmul_rn(d1, a.scale);
    }
  }
  __syncthreads();

  // chunk softmax statistics: wave g for q head 2h + g
  const int n = t1 - t0;
  if (wv < 2) {
    const float sc = lane < n ? s_p[wv][lane] : -3.0e38f;
    float m = sc;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    const float e = lane < n ? expf(__fsub_rn(sc, m)) : 0.0f;
    float l = e;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) l = __fadd_rn(l, __shfl_xor(l, o, 64));
    if (lane < n) s_p[wv][lane] = e;
    if (lane == 0) {
      const int qh = 2 * h + wv;
      a.pm[qh * a.C + c] = m;
      a.pl[qh * a.C + c] = l;
    }
  }
  __syncthreads();

  // unnormalised output of the chunk: thread (g, d) over the chunk's positions
  const float* vbase = a.vc + (size_t)h * a.max_seq * HD + d;
  float o = 0.0f;
  int t = t0;
  for (; t + 4 <= t1; t += 4) {
    float v4[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v4[i] = (t + i == p) ? s_v[d] : vbase[(size_t)(t + i) * HD];
#pragma unroll
    for (int i = 0; i < 4; i++) o = __fmaf_rn(s_p[g][t + i - t0], v4[i], o);
  }
  for (; t < t1; t++) {
    const float v = (t == p) ? s_v[d] : vbase[(size_t)t * HD];
    o = __fmaf_rn(s_p[g][t - t0], v, o);
  }
  a.po[((size_t)(2 * h + g) * a.C + c) * HD + d] = o;
}

// one work-group per q head: out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c
__global__ __launch_bounds__(128) void attn_combine_kernel(const float* __restrict__ pm, const float* __restrict__ pl,
                                                           const float* __restrict__ po, const int* __restrict__ state,
                                                           int C, float* __restrict__ out) {
  const int qh = blockIdx.x, d = threadIdx.x;
  const int nc = cdiv(state[0] + 1, ATT_T);
  float M = -3.0e38f;
  for (int c = 0; c < nc; c++) M = fmaxf(M, pm[qh * C + c]);
  float L = 0.0f, o = 0.0f;
  for (int c = 0; c < nc; c++) {
    const float w = expf(__fsub_rn(pm[qh * C + c], M));
    L = __fmaf_rn(w, pl[qh * C + c], L);
    o = __fmaf_rn(w, po[((size_t)qh * C + c) * HD + d], o);
  }
  out[qh * HD + d] = __fmul_rn(o, __fdiv_rn(1.0f, L));
}

// greedy token (largest argmax key: largest logit, lowest index on ties),
// recorded at tokens[state[2]]; hidden <- embed[token]; positions advance
__global__ __launch_bounds__(1024) void step_end_kernel(const uint64_t* __restrict__ keys, int n,
                                                        const float* __restrict__ embed, int H,
                                                        float* __restrict__ hidden, int* __restrict__ state,
                                                        int32_t* __restrict__ tokens, int max_tokens) {
  __shared__ uint64_t s_k[16];
  __shared__ int s_tok;
  uint64_t k = 0;
  for (int i = threadIdx.x; i < n; i += 1024) k = keys[i] > k ? keys[i] : k;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t t = __shfl_xor(k, o, 64);
    k = t > k ? t : k;
  }
  if ((threadIdx.x & 63) == 0) s_k[threadIdx.x >> 6] = k;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 16; i++) k = s_k[i] > k ? s_k[i] : k;
    const int tok = argmax_key_index(k);
    s_tok = tok;
    const int step = state[2];
    if (tokens && step < max_tokens) tokens[step] = tok;
  }
  __syncthreads();
  const int tok = s_tok;
  if (embed)
    for (int i = threadIdx.x; i < H; i += 1024) hidden[i] = embed[(size_t)tok * H + i];
  if (threadIdx.x == 0) {
    state[0] += 1;
    state[1] += 1;
    state[2] += 1;
  }
}

hipError_t launch_attn_decode(const AttnDecodeArgs& a, hipStream_t st) {
  if (a.nq != 2 * a.nkv || a.C * ATT_T < a.max_seq) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attn_decode_kernel, dim3(a.C, a.nkv), dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_attn_combine(const AttnDecodeArgs& a, float* out, hipStream_t st) {
  hipLaunchKernelGGL(attn_combine_kernel, dim3(a.nq), dim3(HD), 0, st, a.pm, a.pl, a.po, a.state, a.C, out);
  return hipGetLastError();
}

hipError_t launch_step_end(const uint64_t* keys, int n, const float* embed, int H, float* hidden, int* state,
                           int32_t* tokens, int max_tokens, hipStream_t st) {
  hipLaunchKernelGGL(step_end_kernel, dim3(1), dim3(1024), 0, st, keys, n, embed, H, hidden, state, tokens,
                     max_tokens);
  return hipGetLastError();
}

int attn_chunks(int max_seq) { return cdiv(max_seq, ATT_T); }

}  // namespace tl
