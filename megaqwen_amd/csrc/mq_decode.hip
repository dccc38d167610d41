// Persistent cooperative decode kernel for Qwen3-0.6B on MI355X (gfx950).
//
// One launch = one greedy decode step of the whole model (embedding, 28
// decoder layers, final norm, tied LM head, argmax), the role of the
// reference's ldg_decode_kernel + ldg_lm_head_phase1/2
// (csrc/megakernel/fused_decode_ldg.cu:617-887).
//
// Layout on the chip: 256 workgroups x 256 threads (4 waves of 64), one per
// CU. A cooperative launch places workgroup w on XCD g = w % 8 as its j = w / 8
// -th member. XCD g owns KV group g end to end:
//   * the 512 q/k/v rows of group g (16 rows per workgroup),
//   * the attention of its two query heads (split over positions),
//   * the o_proj columns of those two heads (all 1024 rows, 32 per workgroup),
//   * MLP units [384g, 384g+384): their gate/up rows and down_proj columns.
// Every workgroup streams the same 120 KB of weights per layer. The only
// data that crosses XCDs are the o_proj and down_proj partial sums: workgroup
// (g, j) owns residual-stream rows [32j, 32j+32) and reduces them from the 8
// XCDs' partials, so each XCD keeps a full copy of the residual stream.
//
// Exchanges use "tagged words": a bf16 value in the low half of a 32-bit word
// and a 16-bit tag (launch epoch x 32 + layer) in the high half, or an fp32
// value with a 32-bit tag in a 64-bit word. A consumer issues all its loads at
// once and re-polls only words with a stale tag, so an exchange costs one
// memory round trip and no barrier. Inside an XCD, producers use plain stores
// and consumers non-temporal loads, which bypass the per-CU L1 and are served
// by the XCD's shared L2; across XCDs both sides use device-scope (sc1)
// accesses. A watchdog bounds every poll.
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
constexpr int ROWS = H / WG_PER_XCD;    // residual rows owned per workgroup: 32
constexpr int UNITS = I / NWG;          // MLP units per workgroup: 12
constexpr int XUNITS = I / NXCD;        // MLP units per XCD: 384
// Attention: one workgroup per KV group up to CH_MIN positions; longer contexts
// are split over up to 32 workgroups of the owning XCD. The first PF rounds
// of 16 positions are prefetched while the q/k/v rows are still in flight.
constexpr int CH_MIN = 128;
constexpr int PF = 8;

// Workspace layout, in 32-bit words.
constexpr uint32_t WS_EPOCH = 0;
constexpr uint32_t WS_ERR = 32;
constexpr uint32_t WS_FINAL_TICKET = 64;
// per-XCD regions (128 KB apart), written and read only by that XCD's workgroups
constexpr uint32_t WS_LOCAL = 1024;
constexpr uint32_t LOCAL_WORDS = 32768;
constexpr uint32_t LX_H = 0;        // [1024] tagged bf16: residual stream h (layer input)
constexpr uint32_t LX_H1 = 1024;    // [1024] tagged bf16: residual after attention
constexpr uint32_t LX_M = 2048;     // [384]  tagged bf16: SiLU(gate) * up of this XCD's units
constexpr uint32_t LX_ATTN = 2432;  // [256]  tagged bf16: attention output of the two heads
constexpr uint32_t LX_QKV = 2688;   // [512]  tagged bf16: raw q0, q1, k, v rows
constexpr uint32_t APART = 130;     // split partial: m, l, o[128]
constexpr uint32_t LX_PART = 4096;  // [32 splits][2 heads][APART] (fp32, tag) pairs
// cross-XCD partial sums: [j][row][g] (fp32, tag) pairs
constexpr uint32_t WS_OPART = WS_LOCAL + NXCD * LOCAL_WORDS;
constexpr uint32_t WS_DPART = WS_OPART + 2 * WG_PER_XCD * ROWS * NXCD;
constexpr uint32_t WS_LMPART = WS_DPART + 2 * WG_PER_XCD * ROWS * NXCD;  // [NWG][2]
constexpr uint32_t WS_WORDS = WS_LMPART + NWG * 2;
constexpr size_t WS_BYTES = ((WS_WORDS * 4 + 4 + 65535) / 65536) * 65536;

constexpr uint32_t POLL_LIMIT = 1u << 21;  // ~1 s of polling before the watchdog fires
constexpr uint32_t ERR_POLL = 1u;

constexpr int NT_LD = 2;  // non-temporal cache policy: bypasses the CU's L1, served by the XCD's L2

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

// The error word is written and read with sc1 buffer operations only.
__device__ __noinline__ void raise_error(uint32_t* ws, uint32_t code) {
  __builtin_amdgcn_raw_buffer_store_b32(code, __builtin_amdgcn_make_buffer_rsrc(ws, 0, 0x7fffffff, 0x00020000),
                                        WS_ERR * 4u, 0, SC1);
}

__device__ __forceinline__ bool watchdog(const Buf& wsb, uint32_t* ws, uint32_t spins) {
  if ((spins & 1023u) == 0 && (spins > POLL_LIMIT || wsb.ld1(WS_ERR * 4u) != 0)) {
    raise_error(ws, ERR_POLL);
    return true;
  }
  return false;
}

// ---- XCD-local exchange: plain stores, non-temporal loads (L2)
__device__ __forceinline__ u32x4 ldl4(const Buf& b, uint32_t word) {
  return __builtin_amdgcn_raw_buffer_load_b128(b.r, word * 4u, 0, NT_LD);
}
__device__ __forceinline__ u32x2 ldl64(const Buf& b, uint32_t word) {
  return __builtin_amdgcn_raw_buffer_load_b64(b.r, word * 4u, 0, NT_LD);
}
__device__ __forceinline__ void stl1(const Buf& b, uint32_t word, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, b.r, word * 4u, 0, 0);
}
__device__ __forceinline__ void stl64(const Buf& b, uint32_t word, float v, uint32_t tag) {
  u32x2 x;
  x.x = __float_as_uint(v);
  x.y = tag;
  __builtin_amdgcn_raw_buffer_store_b64(x, b.r, word * 4u, 0, 0);
}
__device__ __forceinline__ u32x4 repoll_l4(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag, u32x4 v) {
  uint32_t spins = 0;
  while (!tags_ok(v, tag)) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    v = ldl4(b, word);
  }
  return v;
}
__device__ __forceinline__ float repoll_l64(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag, u32x2 v) {
  uint32_t spins = 0;
  while (v.y != tag) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    v = ldl64(b, word);
  }
  return __uint_as_float(v.x);
}

// ---- cross-XCD exchange: device-scope (sc1) stores and loads of (fp32, tag) pairs;
// aligned 8-byte accesses are single-copy atomic
__device__ __forceinline__ u32x2 ldx64(const Buf& b, uint32_t word) {
  return __builtin_amdgcn_raw_buffer_load_b64(b.r, word * 4u, 0, SC1);
}
__device__ __forceinline__ void stx64(const Buf& b, uint32_t word, float v, uint32_t tag) {
  u32x2 x;
  x.x = __float_as_uint(v);
  x.y = tag;
  __builtin_amdgcn_raw_buffer_store_b64(x, b.r, word * 4u, 0, SC1);
}
__device__ __forceinline__ float repoll_x64(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag, u32x2 v) {
  uint32_t spins = 0;
  while (v.y != tag) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    v = ldx64(b, word);
  }
  return __uint_as_float(v.x);
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
__device__ __forceinline__ uint32_t ldraw16(const uint16_t* p) { return *(gu16*)(p); }

// Block-wide RMSNorm of s_x[H] (bf16 values held as fp32) with bf16 weight w:
// HF Qwen3RMSNorm (modeling_qwen3.py:59-64): y = bf16(w * bf16(x * rsqrt(mean(x^2) + eps))).
// `wv` holds this thread's 4 weights (elements 4*tid .. 4*tid+3), loaded by the
// caller ahead of time so that no global load sits on the reduction's path.
__device__ __forceinline__ void block_rmsnorm(const float* s_x, const u32x2 wv, float* s_y, float* s_red) {
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
  const float wf[4] = {bflo(wv.x), bfhi(wv.x), bflo(wv.y), bfhi(wv.y)};
#pragma unroll
  for (int i = 0; i < 4; i++) s_y[tid * 4 + i] = rbf(wf[i] * rbf(x[i] * rstd));
  __syncthreads();
}

// Gather the 1024 tagged words of an XCD-local vector into s_dst as fp32.
__device__ __forceinline__ void gather_local_h(const Buf& b, uint32_t* ws, uint32_t base, uint32_t tag,
                                               float* s_dst) {
  const int i = threadIdx.x * 4;
  const u32x4 x = repoll_l4(b, ws, base + i, tag, ldl4(b, base + i));
  s_dst[i + 0] = bflo(x.x);
  s_dst[i + 1] = bflo(x.y);
  s_dst[i + 2] = bflo(x.z);
  s_dst[i + 3] = bflo(x.w);
}

// Gather 8 consecutive XCD-local tagged words starting at `word`.
__device__ __forceinline__ void gather8_local(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag,
                                              float (&x)[8]) {
  u32x4 a = ldl4(b, word);
  u32x4 c = ldl4(b, word + 4);
  a = repoll_l4(b, ws, word, tag, a);
  c = repoll_l4(b, ws, word + 4, tag, c);
  x[0] = bflo(a.x); x[1] = bflo(a.y); x[2] = bflo(a.z); x[3] = bflo(a.w);
  x[4] = bflo(c.x); x[5] = bflo(c.y); x[6] = bflo(c.z); x[7] = bflo(c.w);
}

// Residual rows [32j, 32j+32) of this workgroup: r_out = bf16(r_in + bf16(sum over the 8
// XCDs' partials in XCD order)); thread r < 32 handles row r. Returns the new row value.
__device__ __forceinline__ float reduce_rows(const Buf& wsb, uint32_t* ws, uint32_t part_base, int j, int r,
                                             uint32_t tag64, float r_in) {
  const uint32_t base = part_base + 2 * ((j * ROWS + r) * NXCD);
  u32x2 v[NXCD];
#pragma unroll
  for (int q = 0; q < NXCD; q++) v[q] = ldx64(wsb, base + 2 * q);
  float s = 0.f;
#pragma unroll
  for (int q = 0; q < NXCD; q++) s += repoll_x64(wsb, ws, base + 2 * q, tag64, v[q]);
  return rbf(r_in + rbf(s));
}

// ---------------------------------------------------------------- the kernel
__global__ void __launch_bounds__(NT, 1) mq_decode_kernel(DecodeParams P) {
  __shared__ float s_h[H];      // a full residual-stream vector (h or h1)
  __shared__ float s_y[H];      // its RMSNorm output
  __shared__ float s_rh[ROWS];  // this workgroup's rows of h (layer input)
  __shared__ float s_rh1[ROWS]; // this workgroup's rows of h1
  __shared__ float s_qkv[4 * HD];
  __shared__ float s_red[4][16];
  __shared__ float s_att[16][2][APART];
  __shared__ float s_part[WG_PER_XCD * 2 * APART];
  __shared__ uint32_t s_flag;
  __shared__ const uint16_t* s_lw[MAX_LAYERS][11];  // weight pointers, copied once per launch
  __shared__ float s_bestv[4];
  __shared__ int s_besti[4];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int w = blockIdx.x, g = w & (NXCD - 1), j = w / NXCD;
  uint32_t* ws = P.ws;
  const Buf wsb(ws);
  const uint32_t epoch = wsb.ld1(WS_EPOCH * 4u);
  const uint32_t lb = WS_LOCAL + g * LOCAL_WORDS;  // this XCD's exchange region

  const int p = P.position;
  const int n_ctx = p + 1;
  int CH = (n_ctx + WG_PER_XCD - 1) / WG_PER_XCD;
  CH = CH < CH_MIN ? CH_MIN : CH;
  CH = (CH + 15) & ~15;
  const int nsplit = (n_ctx + CH - 1) / CH;

  const size_t kv_layer_stride = (size_t)NKV * P.max_seq_len * HD;

  // The pointer table lives in device memory the kernel also writes to, so the
  // compiler cannot fetch it with scalar loads; fetch it once into LDS instead of
  // paying a dependent global round trip before every stage's weight stream.
  for (int i = tid; i < P.num_layers * 11; i += NT)
    s_lw[i / 11][i % 11] = reinterpret_cast<const uint16_t* const*>(P.layers)[i];
  __syncthreads();

  for (int layer = 0; layer < P.num_layers; layer++) {
    const uint16_t* const* LW = s_lw[layer];
    enum { W_IN = 0, W_Q, W_K, W_V, W_QN, W_KN, W_O, W_POST, W_G, W_U, W_D };
    const uint32_t tag = tag_of(epoch, layer);
    const uint32_t tag64 = epoch * 32u + (uint32_t)layer + 1u;

    // ============ stage 1: input RMSNorm + q/k/v rows of KV group g ============
    // workgroup (g, j) owns rows r = 16j + 4*wave + k of [q_{2g}; q_{2g+1}; k_g; v_g].
    {
      const uint16_t* rows[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int r = 16 * j + 4 * wave + k;
        const uint16_t* base;
        if (r < 256) base = LW[W_Q] + (size_t)(256 * g + r) * H;
        else if (r < 384) base = LW[W_K] + (size_t)(128 * g + r - 256) * H;
        else base = LW[W_V] + (size_t)(128 * g + r - 384) * H;
        rows[k] = base;
      }
      const u32x2 wln = ldw2(LW[W_IN] + tid * 4);
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
        __syncthreads();
        if (tid < ROWS) s_rh[tid] = s_h[ROWS * j + tid];
      } else {
        gather_local_h(wsb, ws, lb + LX_H, tag_of(epoch, layer - 1), s_h);
      }
      __syncthreads();
      block_rmsnorm(s_h, wln, s_y, &s_red[0][0]);
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
        if (lane == k) stl1(wsb, lb + LX_QKV + 16 * j + 4 * wave + k, tagged(tag, rbf(acc[k])));
      }
    }

    // ============ stage 2: QK-norm, RoPE, KV append, attention ============
    if (j < nsplit) {
      // ---- this workgroup's chunk of positions: lane group grp (16 lanes, 8 dims each)
      // takes positions c_begin + 4*wave + grp + 16*r.
      const int c_begin = j * CH;
      const int c_end = min(n_ctx, c_begin + CH);
      const int grp = lane >> 4, d0 = (lane & 15) * 8;
      const int pos0 = c_begin + wave * 4 + grp;
      const int nround = (c_end - c_begin + 15) >> 4;
      const uint16_t* kc = P.k_cache + layer * kv_layer_stride + (size_t)g * P.max_seq_len * HD + d0;
      const uint16_t* vc = P.v_cache + layer * kv_layer_stride + (size_t)g * P.max_seq_len * HD + d0;
      // QK-norm weights and this position's cos/sin first (the in-order load queue would
      // otherwise put them behind the K/V stream), then K/V of positions < p, which do
      // not depend on this layer's q/k/v.
      // (unconditional: a load merged from a branch would be waited for at the merge)
      const uint16_t* nw = wave < 2 ? LW[W_QN] : LW[W_KN];
      const uint16_t* ct = P.cos_tab + (size_t)p * HD;
      const uint16_t* st = P.sin_tab + (size_t)p * HD;
      const uint32_t rnw0 = ldraw16(nw + lane), rnw1 = ldraw16(nw + 64 + lane);
      const uint32_t rc0 = ldraw16(ct + lane), rs0 = ldraw16(st + lane);
      const uint32_t rc1 = ldraw16(ct + 64 + lane), rs1 = ldraw16(st + 64 + lane);
      u32x4 KP[PF], VP[PF];
#pragma unroll
      for (int u = 0; u < PF; u++) {
        const int pos = pos0 + 16 * u;
        if (pos < c_end && pos != p) {
          KP[u] = ldw(kc + (size_t)pos * HD);
          VP[u] = ldw(vc + (size_t)pos * HD);
        }
      }
      if (tid < 128) {
        const u32x4 v = repoll_l4(wsb, ws, lb + LX_QKV + 4 * tid, tag, ldl4(wsb, lb + LX_QKV + 4 * tid));
        s_qkv[4 * tid + 0] = bflo(v.x);
        s_qkv[4 * tid + 1] = bflo(v.y);
        s_qkv[4 * tid + 2] = bflo(v.z);
        s_qkv[4 * tid + 3] = bflo(v.w);
      }
      __syncthreads();
      if (wave < 3) {
        // HF: q_norm/k_norm over 128 (modeling_qwen3.py:252-253), then apply_rotary_pos_emb (:147-170).
        float a = s_qkv[wave * HD + lane], b = s_qkv[wave * HD + 64 + lane];
        const float ss = wave_sum(a * a + b * b);
        const float rstd = 1.0f / sqrtf(ss * (1.0f / HD) + EPS);
        const float c0 = bf2f(rc0), s0 = bf2f(rs0), c1 = bf2f(rc1), s1 = bf2f(rs1);
        a = rbf(bf2f(rnw0) * rbf(a * rstd));
        b = rbf(bf2f(rnw1) * rbf(b * rstd));
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
      float q0[8], q1[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        q0[i] = s_qkv[d0 + i];
        q1[i] = s_qkv[HD + d0 + i];
      }
      float m0 = -INFINITY, m1 = -INFINITY, l0 = 0.f, l1 = 0.f;
      float a0[8], a1[8];
#pragma unroll
      for (int i = 0; i < 8; i++) a0[i] = a1[i] = 0.f;
      const float scale = P.attn_scale;
      auto step = [&](int pos, const u32x4& Kw, const u32x4& Vw) {
        float kf[8], vf[8];
        if (pos == p) {
#pragma unroll
          for (int i = 0; i < 8; i++) {
            kf[i] = s_qkv[2 * HD + d0 + i];
            vf[i] = s_qkv[3 * HD + d0 + i];
          }
        } else {
          unpack8(Kw, kf);
          unpack8(Vw, vf);
        }
        float d0s = 0.f, d1s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          d0s = fmaf(q0[i], kf[i], d0s);
          d1s = fmaf(q1[i], kf[i], d1s);
        }
        const float s0 = row16_sum(d0s) * scale;
        const float s1 = row16_sum(d1s) * scale;
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
      };
#pragma unroll
      for (int u = 0; u < PF; u++) {
        const int pos = pos0 + 16 * u;
        if (pos < c_end) step(pos, KP[u], VP[u]);
      }
      // rounds beyond the prefetch window: two batches of 4 rounds in flight
      auto load_batch = [&](int r0, u32x4 (&K)[4], u32x4 (&V)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int pos = pos0 + 16 * (r0 + u);
          if (pos < c_end && pos != p) {
            K[u] = ldw(kc + (size_t)pos * HD);
            V[u] = ldw(vc + (size_t)pos * HD);
          }
        }
      };
      auto run_batch = [&](int r0, const u32x4 (&K)[4], const u32x4 (&V)[4]) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const int pos = pos0 + 16 * (r0 + u);
          if (pos < c_end) step(pos, K[u], V[u]);
        }
      };
      if (nround > PF) {
        u32x4 KA[4], VA[4], KB[4], VB[4];
        load_batch(PF, KA, VA);
        for (int r = PF; r < nround; r += 8) {
          load_batch(r + 4, KB, VB);
          run_batch(r, KA, VA);
          load_batch(r + 8, KA, VA);
          run_batch(r + 4, KB, VB);
        }
      }
      // merge the 16 partial states (4 waves x 4 lane groups) through LDS:
      // thread t -> (head t / 128, dim t % 128)
      {
        const int st = wave * 4 + grp;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          s_att[st][0][2 + d0 + i] = a0[i];
          s_att[st][1][2 + d0 + i] = a1[i];
        }
        if ((lane & 15) == 0) {
          s_att[st][0][0] = m0;
          s_att[st][0][1] = l0;
          s_att[st][1][0] = m1;
          s_att[st][1][1] = l1;
        }
      }
      __syncthreads();
      const int hh = tid >> 7, dim = tid & 127;
      float M = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; v++) M = fmaxf(M, s_att[v][hh][0]);
      float L = 0.f, O = 0.f;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const float e = M == -INFINITY ? 0.f : expf(s_att[v][hh][0] - M);
        L = fmaf(s_att[v][hh][1], e, L);
        O = fmaf(s_att[v][hh][2 + dim], e, O);
      }
      const uint32_t out_word = lb + LX_ATTN + hh * HD + dim;
      if (nsplit == 1) {
        stl1(wsb, out_word, tagged(tag, rbf(O * (1.0f / L))));
      } else {
        // split partial as (fp32, tag) pairs; workgroup (g, 0) combines them
        const uint32_t pb = lb + LX_PART + 2 * ((j * 2 + hh) * APART);
        stl64(wsb, pb + 2 * (2 + dim), O, tag64);
        if (dim == 0) {
          stl64(wsb, pb + 0, M, tag64);
          stl64(wsb, pb + 2, L, tag64);
        }
        if (j == 0) {
          // thread t gathers pairs t, t + NT, ... of the nsplit * 2 * APART partial values
          const int total = nsplit * 2 * APART;
          constexpr int MAXL = (WG_PER_XCD * 2 * APART + NT - 1) / NT;  // 33
          u32x2 v[MAXL];
#pragma unroll
          for (int k = 0; k < MAXL; k++) {
            const int i = tid + NT * k;
            if (i < total) v[k] = ldl64(wsb, lb + LX_PART + 2 * i);
          }
#pragma unroll
          for (int k = 0; k < MAXL; k++) {
            const int i = tid + NT * k;
            if (i < total) s_part[i] = repoll_l64(wsb, ws, lb + LX_PART + 2 * i, tag64, v[k]);
          }
          __syncthreads();
          float Mc = -INFINITY;
          for (int c = 0; c < nsplit; c++) Mc = fmaxf(Mc, s_part[(c * 2 + hh) * APART]);
          float Lc = 0.f, Oc = 0.f;
          for (int c = 0; c < nsplit; c++) {
            const float* pc = &s_part[(c * 2 + hh) * APART];
            const float e = pc[0] == -INFINITY ? 0.f : expf(pc[0] - Mc);
            Lc = fmaf(pc[1], e, Lc);
            Oc = fmaf(pc[2 + dim], e, Oc);
          }
          stl1(wsb, out_word, tagged(tag, rbf(Oc * (1.0f / Lc))));
        }
      }
    }

    // ============ stage 3: o_proj columns of heads 2g, 2g+1 for rows [32j, 32j+32) ============
    // thread t: 16-byte column chunk c = t & 31 (columns 256g + 8c ..), rows rg + 8i with
    // rg = t >> 5 (so wave v holds rows 2v, 2v+1 (+8i)).
    {
      const int c = tid & 31, rg = tid >> 5;
      const uint16_t* wo = LW[W_O] + 256 * g + 8 * c;
      u32x4 wv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) wv[i] = ldw(wo + (size_t)(ROWS * j + rg + 8 * i) * QS);
      float x[8];
      gather8_local(wsb, ws, lb + LX_ATTN + 8 * c, tag, x);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float s = row16_sum(dot8(wv[i], x));
        // lanes 0-31 hold row 2*wave + 8i (rows 0, 1 of the wave), lanes 32-63 row 2*wave+1 + 8i
        const float lo = readlane(s, 0) + readlane(s, 16);
        const float hi = readlane(s, 32) + readlane(s, 48);
        const int r0 = 2 * wave + 8 * i;
        if (lane == 0) stx64(wsb, WS_OPART + 2 * ((j * ROWS + r0) * NXCD + g), lo, tag64);
        if (lane == 32) stx64(wsb, WS_OPART + 2 * ((j * ROWS + r0 + 1) * NXCD + g), hi, tag64);
      }
      // residual rows: h1 = bf16(h + bf16(o)), o summed over the 8 XCDs
      if (tid < ROWS) {
        const float h1 = reduce_rows(wsb, ws, WS_OPART, j, tid, tag64, s_rh[tid]);
        s_rh1[tid] = h1;
        stl1(wsb, lb + LX_H1 + ROWS * j + tid, tagged(tag, h1));
      }
    }

    // ============ stage 4: post-attention RMSNorm, gate/up rows, SiLU * up ============
    // units u0 + [0, 12) with u0 = 384g + 12j; threads 0-127 gate rows, 128-255 up rows.
    {
      const int cc = tid & 127, half = tid >> 7;
      const int u0 = XUNITS * g + UNITS * j;
      const uint16_t* wm = half == 0 ? LW[W_G] : LW[W_U];
      const u32x2 wln = ldw2(LW[W_POST] + tid * 4);
      u32x4 wv[UNITS];
#pragma unroll
      for (int r = 0; r < UNITS; r++) wv[r] = ldw(wm + (size_t)(u0 + r) * H + 8 * cc);
      gather_local_h(wsb, ws, lb + LX_H1, tag, s_h);
      __syncthreads();
      block_rmsnorm(s_h, wln, s_y, &s_red[0][0]);
      float x[8];
#pragma unroll
      for (int i = 0; i < 8; i++) x[i] = s_y[8 * cc + i];
      float acc[UNITS];
#pragma unroll
      for (int r = 0; r < UNITS; r++) acc[r] = wave_sum(dot8(wv[r], x));
      if (lane == 0) {
#pragma unroll
        for (int r = 0; r < UNITS; r++) s_red[wave][r] = acc[r];
      }
      __syncthreads();
      if (tid < UNITS) {
        // HF Qwen3MLP (modeling_qwen3.py:81-83): bf16(bf16(silu(gate)) * up)
        const float gt = rbf(s_red[0][tid] + s_red[1][tid]);
        const float up = rbf(s_red[2][tid] + s_red[3][tid]);
        const float sl = rbf(gt / (1.0f + expf(-gt)));
        stl1(wsb, lb + LX_M + UNITS * j + tid, tagged(tag, rbf(sl * up)));
      }
    }

    // ============ stage 5: down_proj columns of this XCD's units for rows [32j, 32j+32) ============
    // wave v: rows 8v + i (i < 8); lane l < 48: 16-byte column chunk l (columns 384g + 8l ..).
    {
      const bool act = lane < 48;
      const uint16_t* wd = LW[W_D] + XUNITS * g + 8 * lane;
      u32x4 wv[8];
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if (act) wv[i] = ldw(wd + (size_t)(ROWS * j + 8 * wave + i) * I);
      }
      float x[8];
      if (act) gather8_local(wsb, ws, lb + LX_M + 8 * lane, tag, x);
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float s = wave_sum(act ? dot8(wv[i], x) : 0.f);
        if (lane == 0) stx64(wsb, WS_DPART + 2 * ((j * ROWS + 8 * wave + i) * NXCD + g), s, tag64);
      }
      // residual rows: h' = bf16(h1 + bf16(d)), d summed over the 8 XCDs
      if (tid < ROWS) {
        const float hn = reduce_rows(wsb, ws, WS_DPART, j, tid, tag64, s_rh1[tid]);
        s_rh[tid] = hn;
        stl1(wsb, lb + LX_H + ROWS * j + tid, tagged(tag, hn));
      }
    }
  }

  // ============ final norm + tied LM head + argmax ============
  const int last = P.num_layers - 1;
  // The single-block entry (MODE_NO_LMHEAD) passes no final-norm weight.
  const bool lm = !(P.mode & MODE_NO_LMHEAD);
  u32x2 wfn = {0u, 0u};
  if (lm) wfn = ldw2(P.final_norm + tid * 4);
  gather_local_h(wsb, ws, lb + LX_H, tag_of(epoch, last), s_h);
  __syncthreads();
  if (lm) block_rmsnorm(s_h, wfn, s_y, &s_red[0][0]);
  if (w == 0) {
    for (int i = tid; i < H; i += NT) {
      P.hidden_out[i] = (uint16_t)f2bf(s_h[i]);
      if (lm && P.normed_out) P.normed_out[i] = s_y[i];
    }
  }
  float bestv = -INFINITY;
  int besti = 0x7fffffff;
  if (lm) {
    const int r0 = w < 128 ? w * 594 : 128 * 594 + (w - 128) * 593;
    const int r1 = r0 + (w < 128 ? 594 : 593);
    float x0[8], x1[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      x0[i] = s_y[8 * lane + i];
      x1[i] = s_y[512 + 8 * lane + i];
    }
    const bool want_logits = (P.mode & MODE_LOGITS) != 0;
    // wave `wave` takes rows r0 + wave + 4*i, four rows per batch, two batches in flight
    auto load_rows = [&](int rb, u32x4 (&Wr)[4][2]) {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = rb + 4 * u;
        if (r < r1) {
          const uint16_t* row = P.lm_head + (size_t)r * H;
          Wr[u][0] = ldw(row + 8 * lane);
          Wr[u][1] = ldw(row + 512 + 8 * lane);
        }
      }
    };
    auto score_rows = [&](int rb, const u32x4 (&Wr)[4][2]) {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = rb + 4 * u;
        if (r < r1) {
          const float v = rbf(wave_sum(dot8(Wr[u][0], x0) + dot8(Wr[u][1], x1)));
          if (want_logits && lane == 0) P.logits_out[r] = v;
          if (v > bestv) {
            bestv = v;
            besti = r;
          }
        }
      }
    };
    u32x4 WA[4][2], WB[4][2];
    load_rows(r0 + wave, WA);
    for (int rb = r0 + wave; rb < r1; rb += 32) {
      load_rows(rb + 16, WB);
      score_rows(rb, WA);
      load_rows(rb + 32, WA);
      score_rows(rb + 16, WB);
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
  if (lm) {
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
  if (!P.out_token) P.out_token = reinterpret_cast<int*>(g_dev[dev].ws + WS_WORDS);
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
  // No token output: the kernel's status word goes to the workspace tail.
  P.out_token = nullptr;
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
