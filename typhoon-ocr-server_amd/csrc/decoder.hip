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
#include <atomic>

#include "tl_common.h"
#include "tl_kernels.h"

namespace tl {

constexpr int HD = 128;          // head dim
constexpr int kMergeRound = 32;  // chunks whose partials the merger loads at once

// Work-group (c, h): kv head h, positions [T c, T c + T) of the S = p + 1 that
// the new token attends to; its two q heads (GQA group 2).  256 threads.
// The loads are issued in the order the work-group consumes them (the memory
// counter retires loads in issue order): the q/k/v row, norm weights and rope
// row, then the K rows, then the V rows; the norm and rotation prologue
// starts when the first ones land and each score step waits only for its own
// K rows.  Positions past the chunk end read a clamped valid row and are
// masked; position p (the new token, whose cache row this work-group writes)
// is taken from LDS instead of memory.  Lane sums are DPP row and wave
// reductions (no LDS permutes).
//
// Merge without a second launch: every work-group stores its partials (m, l
// and o of each q head) with agent-scope atomic stores, waits until they are
// acknowledged (vmcnt 0: the stores bypass the non-coherent L2 path, so no L2
// write-back is needed, which a device-scope fence would do), then bumps the
// kv head's arrival counter.  The work-group that brings the counter to the
// number of live chunks merges the two q heads: every partial of a round of
// chunks is loaded at once (each thread its o values, the m and l values one
// per lane of a wave and shared through LDS), merged in chunk order, and the
// counter is reset for the next launch.  Nothing waits on another work-group.
// The state pointer and the q/k/v row come first among the arguments, so
// that they arrive in SGPRs at wave launch (kernarg preload in the build) and
// the state read, the first link of the kernel's dependent chain, waits for
// no kernarg fetch.
template <int T>
__global__ __launch_bounds__(256) void attn_decode_kernel(const int* __restrict__ state, const float* __restrict__ qkv,
                                                          AttnDecodeArgs a) {
  constexpr int NK = T / 16;                // K iterations: 16 positions (4 waves x 4) each
  constexpr int NV = T / 8;                 // V float4 per thread: positions pg + 8 i
  const int c = blockIdx.x, h = blockIdx.y;
  const int p = state[0];                   // position of the new token
  const int S = p + 1;
  const int t0 = c * T;
  if (t0 >= S) return;                      // uniform: the whole work-group leaves, no ticket
  const int t1 = min(t0 + T, S);
  const int rp = state[1];

  __shared__ float s_x[2][HD];              // normalised q heads before the rotation
  __shared__ float s_xk[HD];                // normalised new k before the rotation
  __shared__ float s_q[2][HD];              // rotated q heads
  __shared__ float s_k[HD], s_v[HD];        // the new token's k (rotated) and v
  __shared__ float s_red[8];
  __shared__ float s_p[2][T];               // scores, then probabilities
  __shared__ float s_ml[2][2];              // chunk max and sum per q head
  __shared__ float4 s_o[8][2][HD / 4];      // V partial sums of the 8 position groups

  const int tid = threadIdx.x, g = tid >> 7, d = tid & 127;
  const int lane = tid & 63, wv = tid >> 6;
  const bool has_new = p < t1;              // this chunk holds position p

  // ---- loads, in the order they are needed ----------------------------------
  const float qraw = qkv[(2 * h + g) * HD + d];
  const float qw = a.q_norm[d];
  const float* kv_src = qkv + a.nq * HD + (g == 0 ? h * HD : a.nkv * HD + h * HD);
  const float kvraw = has_new ? kv_src[d] : 0.0f;
  const float kw = a.k_norm[d];
  const int j = d & 63;
  const float co = a.cos_tab[(size_t)rp * 64 + j], si = a.sin_tab[(size_t)rp * 64 + j];
  // scores: 16 lanes per position, lane seg holds dimensions 4 seg .. 4 seg + 3
  // and 64 + 4 seg .. + 3 (each load instruction reads four 256-byte row halves);
  // wave w takes positions t0 + 16 it + 4 w + (lane >> 4)
  const int seg = lane & 15;
  const float* kbase = a.kc + (size_t)h * a.max_seq * HD;
  float4 kr[NK][2];
#pragma unroll
  for (int it = 0; it < NK; it++) {
    const int t = min(t0 + it * 16 + wv * 4 + (lane >> 4), t1 - 1);
    const float4* kp = reinterpret_cast<const float4*>(kbase + (size_t)t * HD);
    kr[it][0] = kp[seg];
    kr[it][1] = kp[16 + seg];
  }
  // V: thread (pg = tid >> 5, d4 = tid & 31) reads float4 d4 of positions
  // t0 + pg + 8 i
  const int pg = tid >> 5, d4 = tid & 31;
  const float4* vbase = reinterpret_cast<const float4*>(a.vc + (size_t)h * a.max_seq * HD) + d4;
  float4 vr[NV];
#pragma unroll
  for (int i = 0; i < NV; i++) vr[i] = vbase[(size_t)min(t0 + pg + 8 * i, t1 - 1) * (HD / 4)];

  // ---- q and the new k: RMSNorm (q_norm / k_norm) in one reduction pass, then
  //      the rotation; threads 0-127 also hold element d of k, 128-255 of v
  {
    const float sq = wave_sum(__fmul_rn(qraw, qraw)), sk = wave_sum(__fmul_rn(kvraw, kvraw));
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
  for (int i = 0; i < 4; i++) {
    q0[i] = s_q[0][4 * seg + i];
    q1[i] = s_q[1][4 * seg + i];
    q0[4 + i] = s_q[0][64 + 4 * seg + i];
    q1[4 + i] = s_q[1][64 + 4 * seg + i];
  }
#pragma unroll
  for (int it = 0; it < NK; it++) {
    const int t = t0 + it * 16 + wv * 4 + (lane >> 4);
    float kv8[8] = {kr[it][0].x, kr[it][0].y, kr[it][0].z, kr[it][0].w,
                    kr[it][1].x, kr[it][1].y, kr[it][1].z, kr[it][1].w};
    if (t == p) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        kv8[i] = s_k[4 * seg + i];
        kv8[4 + i] = s_k[64 + 4 * seg + i];
      }
    }
    float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      d0 = __fmaf_rn(q0[i], kv8[i], d0);
      d1 = __fmaf_rn(q1[i], kv8[i], d1);
    }
    d0 = row16_sum(d0);                     // the 16 lanes of a position are one DPP row
    d1 = row16_sum(d1);
    if (seg == 0 && t < t1) {
      s_p[0][t - t0] = __fmul_rn(d0, a.scale);
      s_p[1][t - t0] = __fmul_rn(d1, a.scale);
    }
  }
  __syncthreads();

  // ---- chunk softmax statistics: wave g for q head 2h + g ---------------------
  const int n = t1 - t0;
  if (wv < 2) {
    constexpr int PL = T >= 64 ? T / 64 : 1;   // scores per lane
    float sc[PL];
    float m = -3.0e38f;
#pragma unroll
    for (int i = 0; i < PL; i++) {
      const int t = lane + 64 * i;
      sc[i] = t < n ? s_p[wv][t] : -3.0e38f;
      m = fmaxf(m, sc[i]);
    }
    m = wave_fmax(m);
    float l = 0.0f;
#pragma unroll
    for (int i = 0; i < PL; i++) {
      const int t = lane + 64 * i;
      const float e = t < n ? expf(__fsub_rn(sc[i], m)) : 0.0f;
      if (t < T) s_p[wv][t] = e;            // zero past the chunk end
      l = __fadd_rn(l, e);
    }
    l = wave_sum(l);
    if (lane == 0) {
      s_ml[wv][0] = m;
      s_ml[wv][1] = l;
    }
  }
  __syncthreads();

  // ---- unnormalised output of the chunk ------------------------------------------
  float4 o0 = make_float4(0.f, 0.f, 0.f, 0.f), o1 = o0;
#pragma unroll
  for (int i = 0; i < NV; i++) {
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
  const int qh = 2 * h + g;
  const int nc = cdiv(S, T);
  if (d < 2) st_agent((d == 0 ? a.pm : a.pl) + (size_t)qh * a.C + c, s_ml[g][d]);
  st_agent(a.po + ((size_t)qh * a.C + c) * HD + d, o);

  // ---- arrival; the last work-group of kv head h merges ----------------------
  __shared__ int s_last;
  asm volatile("" ::: "memory");
  wait_vm<0>();                             // this thread's partial stores are acknowledged
  asm volatile("" ::: "memory");
  __syncthreads();
  if (tid == 0) s_last = __hip_atomic_fetch_add(a.count + h, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nc - 1;
  __syncthreads();
  if (!s_last) return;
  // the merger's acquire: the chunks' partials are read after the counter
  // showed them all arrived (agent scope; once per kv head and token)
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

  // out = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c, M = max_c m_c, in
  // chunk order over rounds of kMergeRound chunks (one round up to 2048
  // positions at 64 per chunk), each round rescaling the earlier ones
  // The round's maximum and the chunk weights e^(m_c - M) are made once per
  // chunk (lane c of the wave that loaded the m values) and shared through
  // LDS; every thread then folds them in chunk order (the values and the
  // order of the sequential fold, without its serial exponentials).
  __shared__ float s_w[2][2][kMergeRound];  // m and l of q heads 2h, 2h + 1
  __shared__ float s_e[2][kMergeRound + 1]; // e^(m_c - M) of the round, then e^(M_prev - M)
  __shared__ float s_mb[2];                 // the running maximum M of each q head
  const int wg = wv >> 1, ww = wv & 1;      // wave: q head 2h + wg, word ww (m or l)
  const float* src_w = (ww == 0 ? a.pm : a.pl) + (size_t)(2 * h + wg) * a.C;
  float M = -3.0e38f, L = 0.0f, acc = 0.0f;
  for (int c0 = 0; c0 < nc; c0 += kMergeRound) {
    float wm = -3.0e38f;                    // this lane's m (wave ww == 0 of head wg)
    if (lane < kMergeRound) {
      wm = ld_agent(src_w + min(c0 + lane, nc - 1));
      s_w[wg][ww][lane] = wm;
    }
    float v[kMergeRound];
#pragma unroll
    for (int i = 0; i < kMergeRound; i++) v[i] = ld_agent(a.po + ((size_t)qh * a.C + min(c0 + i, nc - 1)) * HD + d);
    if (ww == 0) {                          // wave-uniform: the wave holding the m values
      const float mb = fmaxf(M, wave_fmax(lane < kMergeRound && c0 + lane < nc ? wm : -3.0e38f));
      if (lane < kMergeRound) s_e[wg][lane] = expf(__fsub_rn(wm, mb));
      if (lane == 0) {
        s_e[wg][kMergeRound] = expf(__fsub_rn(M, mb));
        s_mb[wg] = mb;
      }
    }
    __syncthreads();
    const float Mb = s_mb[g];
    const float r = s_e[g][kMergeRound];
    L = __fmul_rn(L, r);
    acc = __fmul_rn(acc, r);
#pragma unroll
    for (int i = 0; i < kMergeRound; i++) {
      if (c0 + i < nc) {
        const float w = s_e[g][i];
        L = __fmaf_rn(w, s_w[g][1][i], L);
        acc = __fmaf_rn(w, v[i], acc);
      }
    }
    M = Mb;
    __syncthreads();                        // s_w and s_e are rewritten by the next round
  }
  // written through to device scope: the O projection reads it on every XCD
  // next (a plain store leaves the line dirty in this XCD's L2 for the
  // kernel-end write-back; 1,145 -> 1,154 tok/s, tokens identical)
  st_agent(a.out + qh * HD + d, __fmul_rn(acc, __fdiv_rn(1.0f, L)));
  if (tid == 0) __hip_atomic_store(a.count + h, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
  // keys in pairs, eight 16-byte loads in flight per thread (the keys buffer
  // is 16-byte aligned); an odd last key separately
  const int n2 = n >> 1;
  const ulonglong2* k2 = reinterpret_cast<const ulonglong2*>(keys);
  for (int i0 = threadIdx.x; i0 < n2; i0 += 1024 * 8) {
    ulonglong2 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = i0 + 1024 * u;
      v[u] = i < n2 ? k2[i] : make_ulonglong2(0, 0);
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      k = v[u].x > k ? v[u].x : k;
      k = v[u].y > k ? v[u].y : k;
    }
  }
  if ((n & 1) && threadIdx.x == 0) k = keys[n - 1] > k ? keys[n - 1] : k;
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
    for (int i = threadIdx.x; i < H; i += 1024) st_agent(hidden + i, embed[(size_t)tok * H + i]);
  if (threadIdx.x == 0) {
    state[0] += 1;
    state[1] += 1;
    state[2] += 1;
  }
}

// positions per work-group override (tuning), 0 = planner; atomic, since a
// setter may run while other threads plan launches
static std::atomic<int> g_attn_t{0};

void attn_set_chunk(int t) { g_attn_t.store((t == 32 || t == 64 || t == 128) ? t : 0, std::memory_order_relaxed); }

int attn_chunk_size(int max_seq) {
  (void)max_seq;
  const int t = g_attn_t.load(std::memory_order_relaxed);
  return t ? t : 64;
}

int attn_chunks(int max_seq) { return cdiv(max_seq, 32); }   // records per q head for the smallest chunks

hipError_t launch_attn_decode(const AttnDecodeArgs& a, hipStream_t st) {
  if (a.nq != 2 * a.nkv || a.T * a.C < a.max_seq || a.max_seq < 1 || !a.pm || !a.pl || !a.po || !a.count ||
      !a.out)
    return hipErrorInvalidValue;
  const dim3 grid(cdiv(a.max_seq, a.T), a.nkv);
  switch (a.T) {
    case 32: hipLaunchKernelGGL(attn_decode_kernel<32>, grid, dim3(256), 0, st, a.state, a.qkv, a); break;
    case 64: hipLaunchKernelGGL(attn_decode_kernel<64>, grid, dim3(256), 0, st, a.state, a.qkv, a); break;
    case 128: hipLaunchKernelGGL(attn_decode_kernel<128>, grid, dim3(256), 0, st, a.state, a.qkv, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_step_end(const uint64_t* keys, int n, const float* embed, int H, float* hidden, int* state,
                           int32_t* tokens, int max_tokens, hipStream_t st) {
  if (n < 1 || (((uintptr_t)keys) & 15) != 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(step_end_kernel, dim3(1), dim3(1024), 0, st, keys, n, embed, H, hidden, state, tokens,
                     max_tokens);
  return hipGetLastError();
}

}  // namespace tl

// ---------------------------------------------------------------------------
// C ABI of the launchers above (tl_kernels.h)
// ---------------------------------------------------------------------------
extern "C" {
int tlk_attn_chunks(int max_seq) { return tl::attn_chunks(max_seq); }
int tlk_attn_chunk_size(int max_seq) { return tl::attn_chunk_size(max_seq); }
void tlk_attn_set_chunk(int t) { tl::attn_set_chunk(t); }
hipError_t tlk_launch_attn_decode(const AttnDecodeArgs* a, hipStream_t st) { return tl::launch_attn_decode(*a, st); }
hipError_t tlk_launch_step_end(const uint64_t* keys, int n, const float* embed, int H, float* hidden, int* state,
                               int32_t* tokens, int max_tokens, hipStream_t st) {
  return tl::launch_step_end(keys, n, embed, H, hidden, state, tokens, max_tokens, st);
}
}  // extern "C"
