// decoder.hip -- the decode-step kernels around the linear layers.
//
// Reference: kernel/decoder.c:33-157 (decoder_layer_forward, DECODE_MODE).
// The linear layers run on gemv_i8_kernel with the layer's other steps fused
// around them (RMSNorm prologues, the residual add as the GEMV bias, SwiGLU
// as an epilogue); what remains for this file is
//   attn_decode_kernel   per-head QK RMSNorm (q_norm / k_norm), M-RoPE at the
//                        decode position, the KV cache append of the new
//                        token, split-sequence GQA attention partials and,
//                        in the last work-group of each kv head to finish,
//                        the softmax-weighted merge of the partials
//                        (kernel/ops.c:233-289, kernel/kv_cache.c:53-64,
//                        kernel/attention.c:172-224);
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




// out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c over the nc live chunks
// of q head qh, element d; chunks in batches of 32 (all loads of a batch in
// flight together), each batch rescaling what the earlier ones accumulated.
__device__ __forceinline__ float merge_chunks(const float* pm, const float* pl, const float* po, int C, int nc,
                                              int qh, int d) {
  float L = 0.0f, acc = 0.0f, M = -3.0e38f;
  for (int c0 = 0; c0 < nc; c0 += 32) {
    float v[32], m[32], l[32];
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const bool ok = c0 + i < nc;
      const int cc = min(c0 + i, nc - 1);
      v[i] = ld_agent(po + ((size_t)qh * C + cc) * HD + d);
      m[i] = ok ? ld_agent(pm + qh * C + cc) : -3.0e38f;
      l[i] = ld_agent(pl + qh * C + cc);
    }
    float Mb = M;
#pragma unroll
    for (int i = 0; i < 32; i++) Mb = fmaxf(Mb, m[i]);
    const float r = expf(__fsub_rn(M, Mb));
    L = __fmul_rn(L, r);
    acc = __fmul_rn(acc, r);
#pragma unroll
    for (int i = 0; i < 32; i++) {
      if (c0 + i < nc) {
        const float w = expf(__fsub_rn(m[i], Mb));
        L = __fmaf_rn(w, l[i], L);
        acc = __fmaf_rn(w, v[i], acc);
      }
    }
    M = Mb;
  }
  return __fmul_rn(acc, __fdiv_rn(1.0f, L));
}

// Work-group (c, h): kv head h, positions [64 c, 64 c + 64) of the S = len + 1
// that the new token attends to; two q heads (GQA group 2).  256 threads.
// Every load of the chunk (its K and V rows, the q/k/v rows of the QKV
// output, norm weights, rope row) is issued first, so the norm/rotation
// prologue runs while they are in flight.  Positions past the chunk end read
// a clamped valid row and are masked; position p (the new token, whose cache
// row this work-group writes) is taken from LDS instead of memory.
//
// Merge without a second launch: every work-group stores its partials with
// agent-scope atomic stores, waits until they are acknowledged (vmcnt 0: the
// stores bypass the non-coherent L2 path, so no L2 write-back is needed, which
// a device-scope fence would do), then bumps the kv head's arrival counter.
// The work-group that brings the counter to the number of live chunks merges
// the two q heads and resets the counter for the next launch.  Nothing waits
// on another work-group.
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecodeArgs a) {
  const int c = blockIdx.x, h = blockIdx.y;
  const int p = a.state[0];                 // position of the new token
  const int S = p + 1;
  const int t0 = c * ATT_T;
  if (t0 >= S) return;                      // uniform: the whole work-group leaves
  const int t1 = min(t0 + ATT_T, S);
  const int rp = a.state[1];

  __shared__ float s_x[2][HD];              // normalised q heads before the rotation
  __shared__ float s_xk[HD];                // normalised new k before the rotation
  __shared__ float s_q[2][HD];              // rotated q heads
  __shared__ float s_k[HD], s_v[HD];        // the new token's k (rotated) and v
  __shared__ float s_red[8];
  __shared__ float s_p[2][ATT_T];           // scores, then probabilities
  __shared__ float4 s_o[8][2][HD / 4];      // V partial sums of the 8 position groups

  const int tid = threadIdx.x, g = tid >> 7, d = tid & 127;
  const int lane = tid & 63, wv = tid >> 6;
  const bool has_new = p < t1;              // this chunk holds position p

  // ---- loads ---------------------------------------------------------------
  // scores: 16 lanes per position (8 elements each), wave w takes positions
  // t0 + 16 w + 4 it + (lane >> 4), it = 0..3
  const int seg = lane & 15;
  const float* kbase = a.kc + (size_t)h * a.max_seq * HD;
  float4 kr[4][2];
#pragma unroll
  for (int it = 0; it < 4; it++) {
    const int t = min(t0 + wv * 16 + it * 4 + (lane >> 4), t1 - 1);
    const float4* kp = reinterpret_cast<const float4*>(kbase + (size_t)t * HD + seg * 8);
    kr[it][0] = kp[0];
    kr[it][1] = kp[1];
  }
  // V: thread (pg = tid >> 5, d4 = tid & 31) reads float4 d4 of positions
  // t0 + pg + 8 i, i = 0..7
  const int pg = tid >> 5, d4 = tid & 31;
  const float4* vbase = reinterpret_cast<const float4*>(a.vc + (size_t)h * a.max_seq * HD) + d4;
  float4 vr[8];
#pragma unroll
  for (int i = 0; i < 8; i++) vr[i] = vbase[(size_t)min(t0 + pg + 8 * i, t1 - 1) * (HD / 4)];
  const float qraw = a.qkv[(2 * h + g) * HD + d];
  const float qw = a.q_norm[d];
  const float* kv_src = a.qkv + a.nq * HD + (g == 0 ? h * HD : a.nkv * HD + h * HD);
  const float kvraw = has_new ? kv_src[d] : 0.0f;
  const float kw = a.k_norm[d];
  const int j = d & 63;
  const float co = a.cos_tab[(size_t)rp * 64 + j], si = a.sin_tab[(size_t)rp * 64 + j];

  // ---- q and the new k: RMSNorm (q_norm / k_norm) in one reduction pass, then
  //      the rotation; threads 0-127 also hold element d of k, 128-255 of v
  {
    float sq = __fmul_rn(qraw, qraw), sk = __fmul_rn(kvraw, kvraw);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      sq = __fadd_rn(sq, __shfl_xor(sq, o, 64));
      sk = __fadd_rn(sk, __shfl_xor(sk, o, 64));
    }
    if (lane == 0) {
      s_red[wv] = sq;
      s_red[4 + wv] = sk;
    }
    __syncthreads();
    const int w0 = wv & ~1;
    const float rq = ref_rsqrt(__fadd_rn(__fdiv_rn(__fadd_rn(s_red[w0], s_red[w0 + 1]), (float)HD), a.eps));
    s_x[g][d] = __fmul_rn(__fmul_rn(qraw, rq), qw);
    if (has_new && g == 0) {
      const float rk = ref_rsqrt(__fadd_rn(__fdiv_rn(__fadd_rn(s_red[4], s_red[5]), (float)HD), a.eps));
      s_xk[d] = __fmul_rn(__fmul_rn(kvraw, rk), kw);
    }
    __syncthreads();
    const float lo = s_x[g][j], hi = s_x[g][j + 64];
    s_q[g][d] = d < 64 ? __fsub_rn(__fmul_rn(lo, co), __fmul_rn(hi, si)) : __fadd_rn(__fmul_rn(hi, co), __fmul_rn(lo, si));
    if (has_new) {
      const size_t off = ((size_t)h * a.max_seq + p) * HD + d;
      if (g == 0) {
        const float klo = s_xk[j], khi = s_xk[j + 64];
        const float kr_ = d < 64 ? __fsub_rn(__fmul_rn(klo, co), __fmul_rn(khi, si))
                                 : __fadd_rn(__fmul_rn(khi, co), __fmul_rn(klo, si));
        s_k[d] = kr_;
        a.kc[off] = kr_;
      } else {
        s_v[d] = kvraw;
        a.vc[off] = kvraw;
      }
    }
    __syncthreads();
  }

  // ---- scores ----------------------------------------------------------------
  float q0[8], q1[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    q0[i] = s_q[0][seg * 8 + i];
    q1[i] = s_q[1][seg * 8 + i];
  }
#pragma unroll
  for (int it = 0; it < 4; it++) {
    const int t = t0 + wv * 16 + it * 4 + (lane >> 4);
    float kv8[8] = {kr[it][0].x, kr[it][0].y, kr[it][0].z, kr[it][0].w,
                    kr[it][1].x, kr[it][1].y, kr[it][1].z, kr[it][1].w};
    if (t == p) {
#pragma unroll
      for (int i = 0; i < 8; i++) kv8[i] = s_k[seg * 8 + i];
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

  // ---- chunk softmax statistics: wave g for q head 2h + g ---------------------
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
    s_p[wv][lane] = e;                      // zero past the chunk end
    if (lane == 0) {
      const int qh = 2 * h + wv;
      st_agent(a.pm + qh * a.C + c, m);
      st_agent(a.pl + qh * a.C + c, l);
    }
  }
  __syncthreads();

  // ---- unnormalised output of the chunk ------------------------------------------
  float4 o0 = make_float4(0.f, 0.f, 0.f, 0.f), o1 = o0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int t = t0 + pg + 8 * i;
    float4 v = vr[i];
    if (t == p) v = reinterpret_cast<const float4*>(s_v)[d4];
    if (t >= t1) v = make_float4(0.f, 0.f, 0.f, 0.f);
    const float w0 = s_p[0][pg + 8 * i], w1 = s_p[1][pg + 8 * i];
    o0.x = __fmaf_rn(w0, v.x, o0.x); o0.y = __fmaf_rn(w0, v.y, o0.y);
    o0.z = __fmaf_rn(w0, v.z, o0.z); o0.w = __fmaf_rn(w0, v.w, o0.w);
    o1.x = __fmaf_rn(w1, v.x, o1.x); o1.y = __fmaf_rn(w1, v.y, o1.y);
    o1.z = __fmaf_rn(w1, v.z, o1.z); o1.w = __fmaf_rn(w1, v.w, o1.w);
  }
  s_o[pg][0][d4] = o0;
  s_o[pg][1][d4] = o1;
  __syncthreads();
  const float* so = reinterpret_cast<const float*>(&s_o[0][0][0]);
  float o = 0.0f;
#pragma unroll
  for (int q = 0; q < 8; q++) o = __fadd_rn(o, so[(q * 2 + g) * HD + d]);
  st_agent(a.po + ((size_t)(2 * h + g) * a.C + c) * HD + d, o);

  // ---- arrival; the last work-group of kv head h merges ----------------------
  __shared__ int s_last;
  asm volatile("" ::: "memory");
  wait_vm<0>();                             // this thread's partial stores are acknowledged
  asm volatile("" ::: "memory");
  __syncthreads();
  const int nc = cdiv(S, ATT_T);
  if (tid == 0) s_last = __hip_atomic_fetch_add(a.count + h, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nc - 1;
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) __hip_atomic_store(a.count + h, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  a.out[(2 * h + g) * HD + d] = merge_chunks(a.pm, a.pl, a.po, a.C, nc, 2 * h + g, d);
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
  if (a.nq != 2 * a.nkv || a.C * ATT_T < a.max_seq || !a.count || !a.out) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attn_decode_kernel, dim3(a.C, a.nkv), dim3(256), 0, st, a);
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
