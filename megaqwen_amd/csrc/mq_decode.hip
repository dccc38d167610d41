// Persistent cooperative decode kernel for Qwen3-0.6B on MI355X (gfx950).
//
// One launch = one greedy decode step of the whole model (embedding, 28
// decoder layers, final norm, tied LM head, argmax), the role of the
// reference's ldg_decode_kernel + ldg_lm_head_phase1/2
// (csrc/megakernel/fused_decode_ldg.cu:617-887).
//
// Layout on the chip: 256 workgroups x 256 threads (4 waves of 64), one per
// CU. A cooperative launch places workgroup w on XCD w % 8, so KV head g is
// owned by XCD g: its 32 workgroups compute the 512 q/k/v rows of that head
// group and split its attention over positions. Every other matvec is
// split evenly over all 256 workgroups by output rows, so each workgroup
// streams the same number of weight bytes per stage.
//
// Inter-workgroup data moves through a small device workspace as "tagged
// words": each 32-bit word holds a bf16 value in its low half and a 16-bit
// tag (launch epoch x 32 + layer) in its high half, written and read with
// device-scope (sc1) buffer operations. A consumer polls the words it needs
// until every tag matches, so one exchange costs one memory round trip and
// no separate barrier. A watchdog bounds every poll.
//
// Numerics follow HF Qwen3 in bf16 (transformers/models/qwen3/modeling_qwen3.py):
// every Linear / norm / RoPE op / residual add / SiLU / product result is
// rounded to bf16 where HF rounds it, dot products accumulate in fp32, the
// logits are rounded to bf16 and the argmax takes the lowest index on ties.

#include "mq_common.h"

#include <math.h>
#include <mutex>
#include <string.h>

#include "../../include/megaqwen_amd.h"

namespace mq {

constexpr int NWG = 256;
constexpr int NT = 256;
constexpr int NXCD = 8;
constexpr int WG_PER_XCD = NWG / NXCD;  // 32
constexpr int CH_MIN = 32;              // minimum positions per attention split

// Workspace layout, in 32-bit words.
constexpr uint32_t WS_EPOCH = 0;
constexpr uint32_t WS_ERR = 32;
constexpr uint32_t WS_FINAL_TICKET = 64;
constexpr uint32_t WS_ATTN_TICKET = 1024;  // [MAX_LAYERS][NKV], 32 words apart
constexpr uint32_t WS_XH = WS_ATTN_TICKET + MAX_LAYERS * NKV * 32;
constexpr uint32_t WS_XQKV = WS_XH + H;           // [NKV][512]
constexpr uint32_t WS_XATTN = WS_XQKV + NKV * 512;  // [2048]
constexpr uint32_t WS_XH1 = WS_XATTN + QS;        // [1024]
constexpr uint32_t WS_XM = WS_XH1 + H;            // [3072]
constexpr uint32_t APART = 132;                   // m, l, o[128], pad
constexpr uint32_t WS_APART = WS_XM + I;          // [NKV][32][2][APART] fp32
constexpr uint32_t WS_LMPART = WS_APART + NKV * WG_PER_XCD * 2 * APART;  // [NWG][2]
constexpr uint32_t WS_WORDS = WS_LMPART + NWG * 2;
constexpr size_t WS_BYTES = ((WS_WORDS * 4 + 65535) / 65536) * 65536;

constexpr uint32_t POLL_LIMIT = 1u << 21;  // ~1 s of polling before the watchdog fires
constexpr uint32_t ERR_POLL = 1u;
constexpr uint32_t ERR_TICKET = 2u;

enum : int { MODE_INPUT_HIDDEN = 1, MODE_NO_LMHEAD = 2, MODE_LOGITS = 4 };

struct DecodeParams {
  const LDGLayerWeights* layers;
  const uint16_t* embed;
  const uint16_t* final_norm;
  const uint16_t* lm_head;
  const uint16_t* cos_tab;
  const uint16_t* sin_tab;
  uint16_t* k_cache;
  uint16_t* v_cache;
  const uint16_t* hidden_in;
  uint16_t* hidden_out;
  float* normed_out;
  float* logits_out;
  int* out_token;
  uint32_t* ws;
  int token;
  int num_layers;
  int position;
  int max_seq_len;
  float attn_scale;
  int mode;
};

__device__ __forceinline__ uint32_t tag_of(uint32_t epoch, int layer) {
  return 1u + ((epoch * 32u + (uint32_t)layer) % 65535u);
}
__device__ __forceinline__ uint32_t tagged(uint32_t tag, float bfval) { return (tag << 16) | f2bf(bfval); }

__device__ __forceinline__ bool tags_ok(const u32x4& v, uint32_t tag) {
  return ((v.x >> 16) == tag) & ((v.y >> 16) == tag) & ((v.z >> 16) == tag) & ((v.w >> 16) == tag);
}

__device__ __noinline__ void raise_error(uint32_t* ws, uint32_t code) {
  __hip_atomic_fetch_or(ws + WS_ERR, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll 4 tagged words at word offset `word` until all carry `tag`.
__device__ __forceinline__ u32x4 poll4(const Buf& wsb, uint32_t* ws, uint32_t word, uint32_t tag) {
  u32x4 v = wsb.ld4(word * 4u);
  uint32_t spins = 0;
  while (!tags_ok(v, tag)) {
    ++spins;
    if ((spins & 1023u) == 0) {
      if (spins > POLL_LIMIT || wsb.ld1(WS_ERR * 4u) != 0) {
        raise_error(ws, ERR_POLL);
        break;
      }
    }
    __builtin_amdgcn_s_sleep(1);
    v = wsb.ld4(word * 4u);
  }
  return v;
}

// Weight pointers arrive through the LDGLayerWeights array, so the compiler
// cannot infer their address space; load through an explicit global pointer
// (global_load, vmcnt only) rather than a flat load (which also counts in
// lgkmcnt and would make every LDS wait also wait for the weight stream).
typedef const __attribute__((address_space(1))) u32x4 gu32x4;
typedef const __attribute__((address_space(1))) u32x2 gu32x2;
typedef const __attribute__((address_space(1))) uint16_t gu16;
__device__ __forceinline__ u32x4 ldw(const uint16_t* p) { return *(gu32x4*)(p); }
__device__ __forceinline__ u32x2 ldw2(const uint16_t* p) { return *(gu32x2*)(p); }
__device__ __forceinline__ float ldbf(const uint16_t* p) { return bf2f(*(gu16*)(p)); }

// Block-wide RMSNorm of s_x[H] (bf16 values held as fp32) with bf16 weight w:
// HF Qwen3RMSNorm (modeling_qwen3.py:59-64): y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))).
__device__ __forceinline__ void block_rmsnorm(const float* s_x, const uint16_t* __restrict__ w, float* s_y,
                                              float* s_red) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float x[4];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    x[i] = s_x[tid * 4 + i];
    ss += x[i] * x[i];
  }
  ss = wave_sum(ss);
  if (lane == 0) s_red[wave] = ss;
  __syncthreads();
  const float tot = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  const float rstd = 1.0f / sqrtf(tot * (1.0f / H) + EPS);
  const u32x2 wv = ldw2(w + tid * 4);
  const float wf[4] = {bflo(wv.x), bfhi(wv.x), bflo(wv.y), bfhi(wv.y)};
#pragma unroll
  for (int i = 0; i < 4; i++) s_y[tid * 4 + i] = rbf(wf[i] * rbf(x[i] * rstd));
  __syncthreads();
}

// Gather `n` tagged words (n a multiple of 4*NT or <= 4*NT) into s_dst as fp32.
__device__ __forceinline__ void gather_lds(const Buf& wsb, uint32_t* ws, uint32_t base, int n, uint32_t tag,
                                           float* s_dst) {
  for (int i = threadIdx.x * 4; i < n; i += NT * 4) {
    const u32x4 v = poll4(wsb, ws, base + i, tag);
    s_dst[i + 0] = bflo(v.x);
    s_dst[i + 1] = bflo(v.y);
    s_dst[i + 2] = bflo(v.z);
    s_dst[i + 3] = bflo(v.w);
  }
}

// ---------------------------------------------------------------- the kernel
__global__ void __launch_bounds__(NT, 1) mq_decode_kernel(DecodeParams P) {
  __shared__ float s_h[H];    // layer input h (residual stream)
  __shared__ float s_h1[H];   // residual after attention
  __shared__ float s_y[H];    // normalized vector
  __shared__ float s_qkv[4 * HD];
  __shared__ float s_red[4][16];
  __shared__ float s_att[4][2][APART];
  __shared__ uint32_t s_flag;
  __shared__ float s_bestv[4];
  __shared__ int s_besti[4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int w = blockIdx.x, g = w & (NXCD - 1), j = w / NXCD;
  uint32_t* ws = P.ws;
  const Buf wsb(ws);
  const uint32_t epoch = wsb.ld1(WS_EPOCH * 4u);

  const int p = P.position;
  const int n_ctx = p + 1;
  int CH = (n_ctx + WG_PER_XCD - 1) / WG_PER_XCD;
  CH = CH < CH_MIN ? CH_MIN : CH;
  CH = (CH + 3) & ~3;
  const int nsplit = (n_ctx + CH - 1) / CH;

  const size_t kv_layer_stride = (size_t)NKV * P.max_seq_len * HD;

  for (int layer = 0; layer < P.num_layers; layer++) {
    const LDGLayerWeights& LW = P.layers[layer];
    const uint32_t tag = tag_of(epoch, layer);

    // ============ stage 1: input RMSNorm + q/k/v rows of KV group g ============
    // workgroup (g, j) owns rows r = 16j + 4*wave + k of [q_{2g}; q_{2g+1}; k_g; v_g].
    {
      const uint16_t* rows[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int r = 16 * j + 4 * wave + k;
        const uint16_t* base;
        if (r < 256) base = (const uint16_t*)LW.q_proj_weight + (size_t)(256 * g + r) * H;
        else if (r < 384) base = (const uint16_t*)LW.k_proj_weight + (size_t)(128 * g + r - 256) * H;
        else base = (const uint16_t*)LW.v_proj_weight + (size_t)(128 * g + r - 384) * H;
        rows[k] = base;
      }
      u32x4 wq[4][2];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        wq[k][0] = ldw(rows[k] + 8 * lane);
        wq[k][1] = ldw(rows[k] + 512 + 8 * lane);
      }
      if (layer == 0) {
        const uint16_t* src = (P.mode & MODE_INPUT_HIDDEN) ? P.hidden_in : P.embed + (size_t)P.token * H;
        const u32x2 v = ldw2(src + tid * 4);
        s_h[tid * 4 + 0] = bflo(v.x);
        s_h[tid * 4 + 1] = bfhi(v.x);
        s_h[tid * 4 + 2] = bflo(v.y);
        s_h[tid * 4 + 3] = bfhi(v.y);
      } else {
        gather_lds(wsb, ws, WS_XH, H, tag_of(epoch, layer - 1), s_h);
      }
      __syncthreads();
      block_rmsnorm(s_h, (const uint16_t*)LW.input_layernorm_weight, s_y, &s_red[0][0]);
      float x0[8], x1[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        x0[i] = s_y[8 * lane + i];
        x1[i] = s_y[512 + 8 * lane + i];
      }
      float acc[4];
#pragma unroll
      for (int k = 0; k < 4; k++) acc[k] = wave_sum(dot8(wq[k][0], x0) + dot8(wq[k][1], x1));
#pragma unroll
      for (int k = 0; k < 4; k++) {
        if (lane == k) wsb.st1(tagged(tag, rbf(acc[k])), (WS_XQKV + 512 * g + 16 * j + 4 * wave + k) * 4u);
      }
    }

    // ============ stage 2: QK-norm, RoPE, KV append, split-K attention ============
    if (j < nsplit) {
      gather_lds(wsb, ws, WS_XQKV + 512 * g, 512, tag, s_qkv);
      __syncthreads();
      if (wave < 3) {
        // HF: q_norm/k_norm over 128 (modeling_qwen3.py:252-253), then apply_rotary_pos_emb (:147-170).
        float a = s_qkv[wave * HD + lane], b = s_qkv[wave * HD + 64 + lane];
        const float ss = wave_sum(a * a + b * b);
        const float rstd = 1.0f / sqrtf(ss * (1.0f / HD) + EPS);
        const uint16_t* nw = (const uint16_t*)(wave < 2 ? LW.q_norm_weight : LW.k_norm_weight);
        a = rbf(ldbf(nw + lane) * rbf(a * rstd));
        b = rbf(ldbf(nw + 64 + lane) * rbf(b * rstd));
        const uint16_t* ct = P.cos_tab + (size_t)p * HD;
        const uint16_t* st = P.sin_tab + (size_t)p * HD;
        const float c0 = ldbf(ct + lane), s0 = ldbf(st + lane);
        const float c1 = ldbf(ct + 64 + lane), s1 = ldbf(st + 64 + lane);
        const float ra = rbf(rbf(a * c0) - rbf(b * s0));
        const float rb = rbf(rbf(b * c1) + rbf(a * s1));
        s_qkv[wave * HD + lane] = ra;
        s_qkv[wave * HD + 64 + lane] = rb;
      }
      __syncthreads();
      if (j == p / CH && wave >= 2) {
        // KV-cache append at slot p (bf16 [L][8][max_seq][128]).
        uint16_t* dst = (wave == 2 ? P.k_cache : P.v_cache) + layer * kv_layer_stride + ((size_t)g * P.max_seq_len + p) * HD;
        const float* src = &s_qkv[wave * HD];
        dst[lane] = (uint16_t)f2bf(src[lane]);
        dst[64 + lane] = (uint16_t)f2bf(src[64 + lane]);
      }
      // ---- this workgroup's chunk of positions
      const int c_begin = j * CH;
      const int c_end = min(n_ctx, c_begin + CH);
      const int grp = lane >> 4, d0 = (lane & 15) * 8;
      float q0[8], q1[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        q0[i] = s_qkv[d0 + i];
        q1[i] = s_qkv[HD + d0 + i];
      }
      const uint16_t* kc = P.k_cache + layer * kv_layer_stride + (size_t)g * P.max_seq_len * HD;
      const uint16_t* vc = P.v_cache + layer * kv_layer_stride + (size_t)g * P.max_seq_len * HD;
      float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;
      float a0[8], a1[8];
#pragma unroll
      for (int i = 0; i < 8; i++) a0[i] = a1[i] = 0.f;
      const float scale = P.attn_scale;
      for (int pos = c_begin + wave * 4 + grp; pos < c_end; pos += 16) {
        float kf[8], vf[8];
        if (pos == p) {
#pragma unroll
          for (int i = 0; i < 8; i++) {
            kf[i] = s_qkv[2 * HD + d0 + i];
            vf[i] = s_qkv[3 * HD + d0 + i];
          }
        } else {
          unpack8(ldw(kc + (size_t)pos * HD + d0), kf);
          unpack8(ldw(vc + (size_t)pos * HD + d0), vf);
        }
        float d0s = 0.f, d1s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          d0s = fmaf(q0[i], kf[i], d0s);
          d1s = fmaf(q1[i], kf[i], d1s);
        }
        const float s0 = group16_sum(d0s) * scale;
        const float s1 = group16_sum(d1s) * scale;
        const float n0 = fmaxf(m0, s0), n1 = fmaxf(m1, s1);
        const float al0 = expf(m0 - n0), al1 = expf(m1 - n1);
        const float p0 = expf(s0 - n0), p1 = expf(s1 - n1);
        l0 = fmaf(l0, al0, p0);
        l1 = fmaf(l1, al1, p1);
#pragma unroll
        for (int i = 0; i < 8; i++) {
          a0[i] = fmaf(a0[i], al0, p0 * vf[i]);
          a1[i] = fmaf(a1[i], al1, p1 * vf[i]);
        }
        m0 = n0;
        m1 = n1;
      }
      // merge the 4 position groups of this wave (lanes 16 apart)
#pragma unroll
      for (int off = 16; off < 64; off <<= 1) {
        const float om0 = __shfl_xor(m0, off, 64), om1 = __shfl_xor(m1, off, 64);
        const float ol0 = __shfl_xor(l0, off, 64), ol1 = __shfl_xor(l1, off, 64);
        const float n0 = fmaxf(m0, om0), n1 = fmaxf(m1, om1);
        const float e0a = n0 == -INFINITY ? 0.f : expf(m0 - n0), e0b = n0 == -INFINITY ? 0.f : expf(om0 - n0);
        const float e1a = n1 == -INFINITY ? 0.f : expf(m1 - n1), e1b = n1 == -INFINITY ? 0.f : expf(om1 - n1);
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float o0 = __shfl_xor(a0[i], off, 64), o1 = __shfl_xor(a1[i], off, 64);
          a0[i] = a0[i] * e0a + o0 * e0b;
          a1[i] = a1[i] * e1a + o1 * e1b;
        }
        l0 = l0 * e0a + ol0 * e0b;
        l1 = l1 * e1a + ol1 * e1b;
        m0 = n0;
        m1 = n1;
      }
      if (lane < 16) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
          s_att[wave][0][2 + d0 + i] = a0[i];
          s_att[wave][1][2 + d0 + i] = a1[i];
        }
        if (lane == 0) {
          s_att[wave][0][0] = m0;
          s_att[wave][0][1] = l0;
          s_att[wave][1][0] = m1;
          s_att[wave][1][1] = l1;
        }
      }
      __syncthreads();
      // merge the 4 waves: thread t -> (head t / 128, dim t % 128)
      const int hh = tid >> 7, dim = tid & 127;
      float M = -INFINITY;
#pragma unroll
      for (int v = 0; v < 4; v++) M = fmaxf(M, s_att[v][hh][0]);
      float L = 0.f, O = 0.f;
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const float e = M == -INFINITY ? 0.f : expf(s_att[v][hh][0] - M);
        L = fmaf(s_att[v][hh][1], e, L);
        O = fmaf(s_att[v][hh][2 + dim], e, O);
      }
      const uint32_t out_word = WS_XATTN + (2 * g + hh) * HD + dim;
      if (nsplit == 1) {
        wsb.st1(tagged(tag, rbf(O * (1.0f / L))), out_word * 4u);
      } else {
        const uint32_t pbase = WS_APART + ((g * WG_PER_XCD + j) * 2 + hh) * APART;
        wsb.st1(__float_as_uint(O), (pbase + 2 + dim) * 4u);
        if (dim == 0) {
          wsb.st1(__float_as_uint(M), (pbase + 0) * 4u);
          wsb.st1(__float_as_uint(L), (pbase + 1) * 4u);
        }
        wait_vmem();
        __syncthreads();
        if (tid == 0) {
          const uint32_t old = __hip_atomic_fetch_add(ws + WS_ATTN_TICKET + (layer * NKV + g) * 32, 1u,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          s_flag = (old == (uint32_t)(nsplit - 1)) ? 1u : 0u;
        }
        __syncthreads();
        if (s_flag) {
          // last arriving split combines all partials of this KV group
          float Mc = -INFINITY;
          for (int c = 0; c < nsplit; c++) {
            const uint32_t pb = WS_APART + ((g * WG_PER_XCD + c) * 2 + hh) * APART;
            Mc = fmaxf(Mc, __uint_as_float(wsb.ld1(pb * 4u)));
          }
          float Lc = 0.f, Oc = 0.f;
          for (int c = 0; c < nsplit; c++) {
            const uint32_t pb = WS_APART + ((g * WG_PER_XCD + c) * 2 + hh) * APART;
            const float mc = __uint_as_float(wsb.ld1(pb * 4u));
            const float lc = __uint_as_float(wsb.ld1((pb + 1) * 4u));
            const float oc = __uint_as_float(wsb.ld1((pb + 2 + dim) * 4u));
            const float e = mc == -INFINITY ? 0.f : expf(mc - Mc);
            Lc = fmaf(lc, e, Lc);
            Oc = fmaf(oc, e, Oc);
          }
          wsb.st1(tagged(tag, rbf(Oc * (1.0f / Lc))), out_word * 4u);
        }
      }
    }

    // ============ stage 3: o_proj rows 4w..4w+3, residual ============
    {
      const uint16_t* wo = (const uint16_t*)LW.o_proj_weight;
      u32x4 wv[4];
#pragma unroll
      for (int k = 0; k < 4; k++) wv[k] = ldw(wo + (size_t)(4 * w + k) * QS + 8 * tid);
      const u32x4 va = poll4(wsb, ws, WS_XATTN + 8 * tid, tag);
      const u32x4 vb = poll4(wsb, ws, WS_XATTN + 8 * tid + 4, tag);
      const float x[8] = {bflo(va.x), bflo(va.y), bflo(va.z), bflo(va.w),
                          bflo(vb.x), bflo(vb.y), bflo(vb.z), bflo(vb.w)};
      float acc[4];
#pragma unroll
      for (int k = 0; k < 4; k++) acc[k] = wave_sum(dot8(wv[k], x));
      if (lane == 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) s_red[wave][k] = acc[k];
      }
      __syncthreads();
      if (tid < 4) {
        const float o = rbf((s_red[0][tid] + s_red[1][tid]) + (s_red[2][tid] + s_red[3][tid]));
        const float h1 = rbf(s_h[4 * w + tid] + o);
        wsb.st1(tagged(tag, h1), (WS_XH1 + 4 * w + tid) * 4u);
      }
    }

    // ============ stage 4: post-attention RMSNorm, gate/up rows, SiLU * up ============
    {
      const int cc = tid & 127, half = tid >> 7;
      const uint16_t* wm = (const uint16_t*)(half == 0 ? LW.gate_proj_weight : LW.up_proj_weight);
      u32x4 wv[12];
#pragma unroll
      for (int r = 0; r < 12; r++) wv[r] = ldw(wm + (size_t)(12 * w + r) * H + 8 * cc);
      gather_lds(wsb, ws, WS_XH1, H, tag, s_h1);
      __syncthreads();
      block_rmsnorm(s_h1, (const uint16_t*)LW.post_attn_layernorm_weight, s_y, &s_red[0][0]);
      float x[8];
#pragma unroll
      for (int i = 0; i < 8; i++) x[i] = s_y[8 * cc + i];
      float acc[12];
#pragma unroll
      for (int r = 0; r < 12; r++) acc[r] = wave_sum(dot8(wv[r], x));
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < 12; r++) s_red[wave][r] = acc[r];
      }
      __syncthreads();
      if (tid < 12) {
        // HF Qwen3MLP (modeling_qwen3.py:81-83): bf16(bf16(silu(gate)) * up)
        const float gt = rbf(s_red[0][tid] + s_red[1][tid]);
        const float up = rbf(s_red[2][tid] + s_red[3][tid]);
        const float sl = rbf(gt / (1.0f + expf(-gt)));
        wsb.st1(tagged(tag, rbf(sl * up)), (WS_XM + 12 * w + tid) * 4u);
      }
    }

    // ============ stage 5: down_proj rows 4w..4w+3, residual ============
    {
      const uint16_t* wd = (const uint16_t*)LW.down_proj_weight;
      const bool two = tid < 128;
      u32x4 wv[4], wv2[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        wv[k] = ldw(wd + (size_t)(4 * w + k) * I + 8 * tid);
        if (two) wv2[k] = ldw(wd + (size_t)(4 * w + k) * I + 2048 + 8 * tid);
      }
      const u32x4 ma = poll4(wsb, ws, WS_XM + 8 * tid, tag);
      const u32x4 mb = poll4(wsb, ws, WS_XM + 8 * tid + 4, tag);
      const float x[8] = {bflo(ma.x), bflo(ma.y), bflo(ma.z), bflo(ma.w),
                          bflo(mb.x), bflo(mb.y), bflo(mb.z), bflo(mb.w)};
      float x2[8];
      if (two) {
        const u32x4 mc = poll4(wsb, ws, WS_XM + 2048 + 8 * tid, tag);
        const u32x4 md = poll4(wsb, ws, WS_XM + 2048 + 8 * tid + 4, tag);
        x2[0] = bflo(mc.x); x2[1] = bflo(mc.y); x2[2] = bflo(mc.z); x2[3] = bflo(mc.w);
        x2[4] = bflo(md.x); x2[5] = bflo(md.y); x2[6] = bflo(md.z); x2[7] = bflo(md.w);
      }
      float acc[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        float s = dot8(wv[k], x);
        if (two) s += dot8(wv2[k], x2);
        acc[k] = wave_sum(s);
      }
      __syncthreads();  // s_red reuse
      if (lane == 0) {
#pragma unroll
        for (int k = 0; k < 4; k++) s_red[wave][k] = acc[k];
      }
      __syncthreads();
      if (tid < 4) {
        const float d = rbf((s_red[0][tid] + s_red[1][tid]) + (s_red[2][tid] + s_red[3][tid]));
        const float hn = rbf(s_h1[4 * w + tid] + d);
        wsb.st1(tagged(tag, hn), (WS_XH + 4 * w + tid) * 4u);
      }
    }
  }

  // ============ final norm + tied LM head + argmax ============
  const int last = P.num_layers - 1;
  gather_lds(wsb, ws, WS_XH, H, tag_of(epoch, last), s_h);
  __syncthreads();
  // The single-block entry (MODE_NO_LMHEAD) passes no final-norm weight.
  const bool lm = !(P.mode & MODE_NO_LMHEAD);
  if (lm) block_rmsnorm(s_h, P.final_norm, s_y, &s_red[0][0]);
  if (w == 0) {
    for (int i = tid; i < H; i += NT) {
      P.hidden_out[i] = (uint16_t)f2bf(s_h[i]);
      if (lm && P.normed_out) P.normed_out[i] = s_y[i];
    }
  }
  float bestv = -INFINITY;
  int besti = 0x7fffffff;
  if (!(P.mode & MODE_NO_LMHEAD)) {
    const int r0 = w < 128 ? w * 594 : 128 * 594 + (w - 128) * 593;
    const int r1 = r0 + (w < 128 ? 594 : 593);
    float x0[8], x1[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      x0[i] = s_y[8 * lane + i];
      x1[i] = s_y[512 + 8 * lane + i];
    }
    const bool want_logits = (P.mode & MODE_LOGITS) != 0;
    int r = r0 + wave;
    for (; r + 12 < r1; r += 16) {
      u32x4 wv[4][2];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const uint16_t* row = P.lm_head + (size_t)(r + 4 * u) * H;
        wv[u][0] = ldw(row + 8 * lane);
        wv[u][1] = ldw(row + 512 + 8 * lane);
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float v = rbf(wave_sum(dot8(wv[u][0], x0) + dot8(wv[u][1], x1)));
        if (want_logits && lane == 0) P.logits_out[r + 4 * u] = v;
        if (v > bestv) {
          bestv = v;
          besti = r + 4 * u;
        }
      }
    }
    for (; r < r1; r += 4) {
      const uint16_t* row = P.lm_head + (size_t)r * H;
      const float v = rbf(wave_sum(dot8(ldw(row + 8 * lane), x0) + dot8(ldw(row + 512 + 8 * lane), x1)));
      if (want_logits && lane == 0) P.logits_out[r] = v;
      if (v > bestv) {
        bestv = v;
        besti = r;
      }
    }
    if (lane == 0) {
      s_bestv[wave] = bestv;
      s_besti[wave] = besti;
    }
    __syncthreads();
    if (tid == 0) {
      for (int v = 1; v < 4; v++) {
        if (s_bestv[v] > bestv || (s_bestv[v] == bestv && s_besti[v] < besti)) {
          bestv = s_bestv[v];
          besti = s_besti[v];
        }
      }
      wsb.st1(__float_as_uint(bestv), (WS_LMPART + 2 * w) * 4u);
      wsb.st1((uint32_t)besti, (WS_LMPART + 2 * w + 1) * 4u);
    }
  }
  // ---- completion ticket: the last workgroup reduces and resets the workspace
  wait_vmem();
  __syncthreads();
  if (tid == 0) {
    const uint32_t old =
        __hip_atomic_fetch_add(ws + WS_FINAL_TICKET, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_flag = (old == (uint32_t)(NWG - 1)) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_flag) return;
  int tok = 0;
  if (!(P.mode & MODE_NO_LMHEAD)) {
    float v = __uint_as_float(wsb.ld1((WS_LMPART + 2 * tid) * 4u));
    int i = (int)wsb.ld1((WS_LMPART + 2 * tid + 1) * 4u);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(v, off, 64);
      const int oi = __shfl_xor(i, off, 64);
      if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
      }
    }
    if (lane == 0) {
      s_bestv[wave] = v;
      s_besti[wave] = i;
    }
    __syncthreads();
    float bv = s_bestv[0];
    int bi = s_besti[0];
    for (int q = 1; q < 4; q++) {
      if (s_bestv[q] > bv || (s_bestv[q] == bv && s_besti[q] < bi)) {
        bv = s_bestv[q];
        bi = s_besti[q];
      }
    }
    tok = bi;
  }
  if (tid == 0) {
    const uint32_t err = wsb.ld1(WS_ERR * 4u);
    *P.out_token = err ? -(int)(1u + err) : tok;
    wsb.st1(0u, WS_ERR * 4u);
    wsb.st1(0u, WS_FINAL_TICKET * 4u);
    wsb.st1(epoch + 1u, WS_EPOCH * 4u);
  }
  for (int i = tid; i < P.num_layers * NKV; i += NT) wsb.st1(0u, (WS_ATTN_TICKET + i * 32) * 4u);
}

// ---------------------------------------------------------------- host side
struct DeviceState {
  bool init = false;
  int status = MQ_OK;
  uint32_t* ws = nullptr;
};
static std::mutex g_mu;
static DeviceState g_dev[64];

static int ensure_device(int dev) {
  if (dev < 0 || dev >= 64) return MQ_ERR_DEVICE;
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState& d = g_dev[dev];
  if (d.init) return d.status;
  d.init = true;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return d.status = MQ_ERR_HIP;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0 || !prop.cooperativeLaunch) return d.status = MQ_ERR_DEVICE;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(mq_decode_kernel), NT,
                                                   0) != hipSuccess)
    return d.status = MQ_ERR_HIP;
  if (per_cu * prop.multiProcessorCount < NWG) return d.status = MQ_ERR_DEVICE;
  void* p = nullptr;
  if (hipMalloc(&p, WS_BYTES) != hipSuccess) return d.status = MQ_ERR_ALLOC;
  if (hipMemset(p, 0, WS_BYTES) != hipSuccess) return d.status = MQ_ERR_HIP;
  if (hipDeviceSynchronize() != hipSuccess) return d.status = MQ_ERR_HIP;
  d.ws = static_cast<uint32_t*>(p);
  return d.status = MQ_OK;
}

static int launch(DecodeParams& P, hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MQ_ERR_HIP;
  const int st = ensure_device(dev);
  if (st != MQ_OK) return st;
  P.ws = g_dev[dev].ws;
  void* args[] = {&P};
  const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(mq_decode_kernel), dim3(NWG),
                                                  dim3(NT), args, 0, stream);
  return e == hipSuccess ? MQ_OK : MQ_ERR_HIP;
}

static bool bad_scale(float s) { return !(s > 0.f) || !isfinite(s); }

}  // namespace mq

using namespace mq;

extern "C" int launch_ldg_decode_with_logits(int input_token_id, int* output_token_id, float* logits_output,
                                             const void* embed_weight, const LDGLayerWeights* layer_weights,
                                             const void* final_norm_weight, const void* lm_head_weight,
                                             const void* cos_table, const void* sin_table, void* k_cache,
                                             void* v_cache, void* hidden_buffer, void* g_activations, void* g_residual,
                                             void* g_q, void* g_k, void* g_v, void* g_attn_out,
                                             void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
                                             void* block_max_idxs, int num_layers, int position, int cache_len,
                                             int max_seq_len, float attn_scale, hipStream_t stream) {
  (void)g_activations; (void)g_residual; (void)g_q; (void)g_k; (void)g_v; (void)g_attn_out;
  (void)g_mlp_intermediate; (void)block_max_vals; (void)block_max_idxs;
  if (!output_token_id || !embed_weight || !layer_weights || !final_norm_weight || !lm_head_weight || !cos_table ||
      !sin_table || !k_cache || !v_cache || !hidden_buffer)
    return MQ_ERR_ARG;
  if (num_layers < 1 || num_layers > MAX_LAYERS || max_seq_len < 1 || position < 0 || position >= max_seq_len ||
      cache_len != position + 1 || input_token_id < 0 || input_token_id >= VOCAB || bad_scale(attn_scale))
    return MQ_ERR_ARG;
  DecodeParams P{};
  P.layers = layer_weights;
  P.embed = static_cast<const uint16_t*>(embed_weight);
  P.final_norm = static_cast<const uint16_t*>(final_norm_weight);
  P.lm_head = static_cast<const uint16_t*>(lm_head_weight);
  P.cos_tab = static_cast<const uint16_t*>(cos_table);
  P.sin_tab = static_cast<const uint16_t*>(sin_table);
  P.k_cache = static_cast<uint16_t*>(k_cache);
  P.v_cache = static_cast<uint16_t*>(v_cache);
  P.hidden_out = static_cast<uint16_t*>(hidden_buffer);
  P.normed_out = static_cast<float*>(g_normalized);
  P.logits_out = logits_output;
  P.out_token = output_token_id;
  P.token = input_token_id;
  P.num_layers = num_layers;
  P.position = position;
  P.max_seq_len = max_seq_len;
  P.attn_scale = attn_scale;
  P.mode = logits_output ? MODE_LOGITS : 0;
  return launch(P, stream);
}

extern "C" int launch_ldg_decode(int input_token_id, int* output_token_id, const void* embed_weight,
                                 const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                                 const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                 void* k_cache, void* v_cache, void* hidden_buffer, void* g_activations,
                                 void* g_residual, void* g_q, void* g_k, void* g_v, void* g_attn_out,
                                 void* g_mlp_intermediate, void* g_normalized, void* block_max_vals,
                                 void* block_max_idxs, int num_layers, int position, int cache_len, int max_seq_len,
                                 float attn_scale, hipStream_t stream) {
  return launch_ldg_decode_with_logits(input_token_id, output_token_id, nullptr, embed_weight, layer_weights,
                                       final_norm_weight, lm_head_weight, cos_table, sin_table, k_cache, v_cache,
                                       hidden_buffer, g_activations, g_residual, g_q, g_k, g_v, g_attn_out,
                                       g_mlp_intermediate, g_normalized, block_max_vals, block_max_idxs, num_layers,
                                       position, cache_len, max_seq_len, attn_scale, stream);
}

extern "C" int mq_decode_layer(const void* hidden_in, void* hidden_out, const LDGLayerWeights* layer_weights,
                               const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
                               int position, int max_seq_len, float attn_scale, hipStream_t stream) {
  if (!hidden_in || !hidden_out || !layer_weights || !cos_table || !sin_table || !k_cache || !v_cache)
    return MQ_ERR_ARG;
  if (max_seq_len < 1 || position < 0 || position >= max_seq_len || bad_scale(attn_scale)) return MQ_ERR_ARG;
  DecodeParams P{};
  P.layers = layer_weights;
  P.cos_tab = static_cast<const uint16_t*>(cos_table);
  P.sin_tab = static_cast<const uint16_t*>(sin_table);
  P.k_cache = static_cast<uint16_t*>(k_cache);
  P.v_cache = static_cast<uint16_t*>(v_cache);
  P.hidden_in = static_cast<const uint16_t*>(hidden_in);
  P.hidden_out = static_cast<uint16_t*>(hidden_out);
  P.num_layers = 1;
  P.position = position;
  P.max_seq_len = max_seq_len;
  P.attn_scale = attn_scale;
  P.mode = MODE_INPUT_HIDDEN | MODE_NO_LMHEAD;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MQ_ERR_HIP;
  if (ensure_device(dev) != MQ_OK) return g_dev[dev].status;
  // The kernel reports watchdog errors through the token slot; this entry has
  // no token output, so it uses a word of the workspace tail.
  P.out_token = reinterpret_cast<int*>(g_dev[dev].ws + WS_WORDS);
  return launch(P, stream);
}

extern "C" int mq_reset_workspace(int device) {
  const int st = ensure_device(device);
  if (st != MQ_OK) return st;
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return MQ_ERR_HIP;
  if (hipSetDevice(device) != hipSuccess) return MQ_ERR_HIP;
  hipError_t e = hipMemset(g_dev[device].ws, 0, WS_BYTES);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (hipSetDevice(cur) != hipSuccess) return MQ_ERR_HIP;
  return e == hipSuccess ? MQ_OK : MQ_ERR_HIP;
}

extern "C" const char* mq_strerror(int status) {
  switch (status) {
    case MQ_OK: return "ok";
    case MQ_ERR_ARG: return "invalid argument";
    case MQ_ERR_HIP: return "HIP runtime error";
    case MQ_ERR_DEVICE: return "device cannot run the 256-workgroup cooperative gfx950 kernel";
    case MQ_ERR_ALLOC: return "workspace allocation failed";
    default: return "unknown status";
  }
}
