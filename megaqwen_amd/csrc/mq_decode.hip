// Persistent decode kernel for Qwen3-0.6B on MI355X (gfx950).
//
// One launch = one greedy decode step of the whole model (embedding, 28
// decoder layers, final norm, tied LM head, argmax), the role of the
// reference's ldg_decode_kernel + ldg_lm_head_phase1/2
// (csrc/megakernel/fused_decode_ldg.cu:617-887).
//
// Chip layout: 256 workgroups of 512 threads, one per CU; workgroup w serves the
// XCD g it runs on (read from the hardware XCC id) as that XCD's member j = w / 8. XCD g owns KV group g: the 512 q/k/v rows of query heads 2g, 2g+1
// and KV head g, the attention of those heads, the o_proj columns of those
// heads (a K-split of o_proj across XCDs) and MLP units 384g .. 384g+383 (a
// K-split of down_proj). Every workgroup runs four roles, one per wave kind:
//   * stream waves 0-3 hold the workgroup's weight slice of the next stage in
//     registers: as soon as a stage's dot products are done the registers are
//     refilled with the following stage (the first LM-head rows after the last
//     layer), so each weight byte is requested one stage before it is used.
//     They also copy the next layer's K/V rows into LDS (LDS DMA). Stream
//     waves only ever issue loads, so the compiler's in-order vmcnt bookkeeping
//     stays exact across the layer loop.
//   * poll waves 4-5 gather the XCD-local exchanges (h, q/k/v, attention
//     output, h1, m), normalise, apply QK-norm and RoPE, and combine attention
//     chunks.
//   * reduce wave 6 sums the eight XCDs' o_proj and down_proj partials of the
//     workgroup's 32 residual rows and applies the residual adds.
//   * store wave 7 publishes the stream waves' dot products (handed over
//     through LDS) and the K/V append. For contexts of at most 256 positions, and
//     for contexts split over at most three workgroups, the store waves of the
//     workgroups without attention also warm the XCD's L2 with the attention
//     workgroups' next K/V rows and weight rows, which they would otherwise copy
//     from HBM on their critical path.
// Per layer and workgroup (g, j):
//   q/k/v : rows 16j .. 16j+15 of the group's [q0; q1; k; v]
//   attn  : workgroups j < nsplit attend over chunk j (<= 256 positions) for the
//           group's two query heads; QK^T and PV run on MFMA from LDS
//   o_proj: partial sums of rows 32j .. 32j+31 over the group's 256 columns
//   MLP   : gate and up rows of units 384g + 12j .. +11, then down_proj
//           partial sums of rows 32j .. 32j+31 over the XCD's 384 units
// so a layer has five XCD-local all-gathers and two cross-XCD reductions. The
// kernel has two instances: SPLIT = false for contexts of at most 256
// positions (one attention workgroup per XCD, no chunk merge compiled in) and
// SPLIT = true for the rest.
//
// Exchanges use "tagged words": a bf16 value in the low half of a 32-bit word
// and a 16-bit tag (launch epoch x 32 + layer) in the high half, or an fp32
// value with a 32-bit tag in a 64-bit word. A consumer issues all its loads at
// once and re-polls only stale words, so an exchange costs one memory round
// trip and no grid barrier. Across XCDs both sides use device-scope (sc1)
// accesses; inside an XCD producers use plain stores and consumers
// non-temporal loads, served by the XCD's shared L2. A watchdog bounds every
// poll and turns a lost producer into an error code instead of a hang.
//
// Numerics follow HF Qwen3 in bf16 (transformers/models/qwen3/modeling_qwen3.py):
// every Linear / norm / RoPE op / residual add / SiLU / product result is
// rounded to bf16 where HF rounds it, dot products accumulate in fp32, the
// attention probabilities enter P.V as bf16 (torch's CPU flash kernel), the
// logits are rounded to bf16 and the argmax takes the lowest index on ties.

#include "mq_common.h"

#include <math.h>
#include <atomic>
#include <mutex>
#include <string.h>

#include "../../include/megaqwen_amd.h"

// Instrumentation hooks: MQ_STAMP(slot) marks a point of a layer's timeline
// (slot = layer * 40 + event; stream events 0..9, poll 12..24, reduce 28..32,
// store 34..38), MQ_STAMP_DUMP() runs once at the end of the kernel. Both compile
// to nothing unless a tracing build defines them before including this file.
#ifndef MQ_STAMP
#define MQ_STAMP(i) ((void)0)
#endif
#ifndef MQ_STAMP_DUMP
#define MQ_STAMP_DUMP() ((void)0)
#endif

namespace mq {

constexpr int NWG = 256;
constexpr int NT = 512;
constexpr int NSW = 4;  // stream waves 0..3
constexpr int NPW = 2;  // poll waves 4..5; wave 6 reduces the cross-XCD partial sums, wave 7 stores
constexpr int NXCD = 8;
constexpr int WG_PER_XCD = NWG / NXCD;        // 32
constexpr int ROWS = H / WG_PER_XCD;          // residual-stream rows owned per workgroup: 32
constexpr int UNITS = I / NWG;                // MLP units per workgroup: 12
constexpr int XUNITS = I / NXCD;              // MLP units per XCD: 384
constexpr int KV_CAP = 256;                       // positions per LDS pass of an attention workgroup
constexpr int MAX_CTX = 2 * WG_PER_XCD * KV_CAP;  // 16384: at most two passes per workgroup
constexpr int SPLIT_WARM_MAX = 3;  // split contexts whose next-layer rows are warmed in L2
constexpr int LM_PRE = 4;                     // LM-head rows each stream wave loads during the last layer

// Attention split of a context of n positions (the query at n - 1): nsplit chunks of at
// most `chunk` positions, chunk j on workgroup (g, j) of every XCD g, each attended in
// passes of at most KV_CAP positions (the LDS copy holds KV_CAP rows).
__host__ __device__ constexpr int plan_nsplit(int n) {
  return (n + KV_CAP - 1) / KV_CAP < WG_PER_XCD ? (n + KV_CAP - 1) / KV_CAP : WG_PER_XCD;
}
__host__ __device__ constexpr int plan_chunk(int n) { return (n + plan_nsplit(n) - 1) / plan_nsplit(n); }
// Every context length the kernel accepts (1 .. MAX_CTX) gives chunks of at most two LDS
// passes, none of them empty, covering all n positions.
constexpr bool plan_is_sound() {
  for (int n = 1; n <= MAX_CTX; n++) {
    const int ns = plan_nsplit(n), ch = plan_chunk(n);
    if (ns < 1 || ns > WG_PER_XCD || ch > 2 * KV_CAP || ch * ns < n || (ns - 1) * ch >= n) return false;
  }
  return true;
}
static_assert(plan_is_sound(), "attention chunks must fit two LDS passes and cover the context");

// Workspace layout, in 32-bit words.
constexpr uint32_t WS_RESERVED = 0;  // (words 0..31 unused)
constexpr uint32_t WS_ERR = 32;
constexpr uint32_t WS_FINAL_TICKET = 64;
// word WS_PREFILL_ERR (96) belongs to the prefill kernels
// per-XCD regions of tagged bf16 words, written and read only by that XCD's workgroups
constexpr uint32_t WS_LOCAL = 1024;
constexpr uint32_t LOCAL_WORDS = 32768;
constexpr uint32_t LX_H = 0;        // [1024] residual stream after the layer (a full copy per XCD)
constexpr uint32_t LX_H1 = 1024;    // [1024] residual stream after attention
constexpr uint32_t LX_QKV = 2048;   // [512]  raw q0, q1, k, v rows of the XCD's KV group
constexpr uint32_t LX_ATT = 2560;   // [256]  attention output of the group's two query heads
constexpr uint32_t LX_M = 2816;     // [384]  SiLU(gate) * up of the XCD's MLP units
constexpr uint32_t LX_HSS = 3200;   // [32] (fp32, tag) pairs: sum of squares of workgroup j's rows of h
constexpr uint32_t LX_H1SS = 3264;  // [32] the same for h1
constexpr uint32_t APART = 130;     // attention partial of one head: m, l, acc[128]
constexpr uint32_t LX_PART = 4096;  // [32 chunks][2 heads][APART] (fp32, tag) pairs
// cross-XCD partial sums: [j][row][xcd] (fp32, tag) pairs
constexpr uint32_t X_OPART = WS_LOCAL + NXCD * LOCAL_WORDS;
constexpr uint32_t X_DPART = X_OPART + 2 * WG_PER_XCD * ROWS * NXCD;
constexpr uint32_t WS_LMPART = X_DPART + 2 * WG_PER_XCD * ROWS * NXCD;  // [NWG][2]: best logit, index
constexpr uint32_t WS_WORDS = WS_LMPART + NWG * 2;
constexpr size_t WS_BYTES = ((WS_WORDS * 4 + 4 + 65535) / 65536) * 65536;

constexpr uint32_t POLL_LIMIT = 1u << 21;  // ~1 s of polling before the watchdog fires
constexpr uint32_t ERR_POLL = 1u;
constexpr uint32_t ERR_XCD = 2u;  // a workgroup ran on an XCD numbered 8 or above
constexpr uint32_t ERR_STEP = 4u;  // a device-resident step found an invalid token, position or count

constexpr int NT_LD = 2;  // non-temporal cache policy: bypasses the CU's L1, served by the XCD's L2

enum : int { MODE_INPUT_HIDDEN = 1, MODE_NO_LMHEAD = 2, MODE_LOGITS = 4, MODE_DEVICE_STEP = 8 };
enum { W_IN = 0, W_Q, W_K, W_V, W_QN, W_KN, W_O, W_POST, W_G, W_U, W_D };

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
  uint32_t epoch;  // launch counter of the device (the host's): tags of this launch's exchanges
  // MODE_DEVICE_STEP: token, position and epoch come from *step (advanced by the launch's
  // last workgroup), and each launch's token is appended to out_ids[step->count]
  MqDecodeStep* step;
  int* out_ids;
  int out_capacity;
};

// Workgroup barrier without a memory fence: LDS writes are complete once
// lgkmcnt reaches zero, and no vector-memory wait is implied, so the stream
// waves keep their weight loads in flight across it.
#define BAR() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")
// Keeps the compiler from issuing the loads that follow before `v` (which
// depends on every use of the registers being reloaded) is computed.
#define AFTER(v) asm volatile("" ::"v"(v) : "memory")

__device__ __forceinline__ uint32_t tag_of(uint32_t epoch, int layer) {
  return 1u + ((epoch * 32u + (uint32_t)layer) % 65535u);
}
__device__ __forceinline__ uint32_t tagged(uint32_t tag, float bfval) { return (tag << 16) | f2bf(bfval); }
__device__ __forceinline__ bool tags_ok(const u32x4& v, uint32_t tag) {
  return ((v.x >> 16) == tag) & ((v.y >> 16) == tag) & ((v.z >> 16) == tag) & ((v.w >> 16) == tag);
}
// low halves (bf16 values) of two tagged words as one bf16 pair
__device__ __forceinline__ uint32_t pair_lo(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }

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

// ---- cross-XCD exchange: device-scope (sc1) loads and stores
__device__ __forceinline__ u32x4 xld4(const Buf& b, uint32_t word) { return b.ld4(word * 4u); }
__device__ __forceinline__ void xst4(const Buf& b, uint32_t word, u32x4 v) { b.st4(v, word * 4u); }
__device__ __forceinline__ void xst1(const Buf& b, uint32_t word, uint32_t v) { b.st1(v, word * 4u); }
__device__ __forceinline__ u32x4 xrepoll4(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag, u32x4 v) {
  uint32_t spins = 0;
  while (!tags_ok(v, tag)) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    v = xld4(b, word);
  }
  return v;
}

// two (fp32, tag) pairs in one 16-byte load
__device__ __forceinline__ u32x4 xrepoll64x2(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag, u32x4 v) {
  uint32_t spins = 0;
  while ((v.y != tag) | (v.w != tag)) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    v = xld4(b, word);
  }
  return v;
}

// ---- XCD-local exchange: plain stores, non-temporal loads (L2)
__device__ __forceinline__ u32x4 ldl4(const Buf& b, uint32_t word) {
  return __builtin_amdgcn_raw_buffer_load_b128(b.r, word * 4u, 0, NT_LD);
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
__device__ __forceinline__ uint32_t ldl1(const Buf& b, uint32_t word) {
  return __builtin_amdgcn_raw_buffer_load_b32(b.r, word * 4u, 0, NT_LD);
}
__device__ __forceinline__ u32x2 ldl64(const Buf& b, uint32_t word) {
  return __builtin_amdgcn_raw_buffer_load_b64(b.r, word * 4u, 0, NT_LD);
}
__device__ __forceinline__ void stl4(const Buf& b, uint32_t word, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, b.r, word * 4u, 0, 0);
}
__device__ __forceinline__ void stl64(const Buf& b, uint32_t word, float v, uint32_t tag) {
  u32x2 x;
  x.x = __float_as_uint(v);
  x.y = tag;
  __builtin_amdgcn_raw_buffer_store_b64(x, b.r, word * 4u, 0, 0);
}
__device__ __forceinline__ uint32_t repoll_l1(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag, uint32_t v) {
  uint32_t spins = 0;
  while ((v >> 16) != tag) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    v = ldl1(b, word);
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

// L2 warm-up of the K/V rows [0, p) of (layer, group g) for the XCD's attention
// workgroup: one 4-byte LDS DMA per 64-byte line, so one instruction touches 64
// lines. Instruction t of the ceil(p / 8) needed (K lines, then V lines) goes to
// worker t % nworkers; a worker is the store wave of one of the XCD's other
// workgroups, whose LDS K/V area is otherwise unused and takes the dead data.
// The issuing wave awaits the copies before that area is reused.
__device__ __forceinline__ void kv_warm(const DecodeParams& P, int layer, int g, int p, uint32_t lds, int wk,
                                        int nworkers, int lane) {
  const size_t base = (size_t)(layer * NKV + g) * P.max_seq_len * HD;
  const uint8_t* kb = reinterpret_cast<const uint8_t*>(P.k_cache + base);
  const uint8_t* vb = reinterpret_cast<const uint8_t*>(P.v_cache + base);
  const int nlk = 4 * p;  // 64-byte lines of K rows 0 .. p-1
  const int ninst = (2 * nlk + 63) >> 6;
  for (int t = wk; t < ninst; t += nworkers) {
    const int li = 64 * t + lane;
    if (li < 2 * nlk) {
      const uint8_t* gp = li < nlk ? kb + 64 * (size_t)li : vb + 64 * (size_t)(li - nlk);
      uint32_t saved;
      asm volatile(
          "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
          : "=&s"(saved)
          : "v"(gp), "s"(lds)
          : "memory");
    }
  }
}

// L2 warm-up of the weight rows that XCD g's attention workgroup (j = 0) loads during
// this layer after its attention (gate and up rows 384g .. 384g+11; down_proj rows 0..31,
// columns 384g .. 384g+383) and at the end of it for the next layer (q rows 256g ..
// 256g+15; o_proj rows 0..31, columns 256g .. 256g+255): 960 128-byte lines, one 4-byte
// LDS DMA each, line t on worker t % nworkers (the same workers as kv_warm).
// `wl` is the layer's and `wn` the next layer's weight-pointer row.
__device__ __forceinline__ void att_weight_warm(const uint16_t* const* wl, const uint16_t* const* wn, int g,
                                                uint32_t lds, int wk, int nworkers, int lane) {
  constexpr int NQL = 16 * 16, NOL = 32 * 4, NGL = 12 * 16, NDL = 32 * 6;  // lines per part
  constexpr int NL = NQL + NOL + 2 * NGL + NDL;
  for (int t = 64 * wk + lane; t < NL; t += 64 * nworkers) {
    const uint8_t* a;
    if (t < NQL) {
      a = reinterpret_cast<const uint8_t*>(uniform_ptr(wn[W_Q]) + (size_t)256 * g * H) + 128 * t;
    } else if (t < NQL + NOL) {
      const int u = t - NQL;
      a = reinterpret_cast<const uint8_t*>(uniform_ptr(wn[W_O]) + (size_t)(u >> 2) * QS + 256 * g) + 128 * (u & 3);
    } else if (t < NQL + NOL + 2 * NGL) {
      const int u = t - NQL - NOL;
      const uint16_t* w = uniform_ptr(wl[u < NGL ? W_G : W_U]);
      a = reinterpret_cast<const uint8_t*>(w + (size_t)XUNITS * g * H) + 128 * (u < NGL ? u : u - NGL);
    } else {
      const int u = t - NQL - NOL - 2 * NGL, row = u / 6;
      a = reinterpret_cast<const uint8_t*>(uniform_ptr(wl[W_D]) + (size_t)row * I + XUNITS * g) + 128 * (u - 6 * row);
    }
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(a), "s"(lds)
                 : "memory");
  }
}

// The same for the attention workgroups j < na of a split context: the weight rows that
// they load during this layer after their attention (gate and up rows 384g + 12j .. +11; down_proj rows
// 32j .. 32j+31, columns 384g .. 384g+383) and at the end of it for the next layer (the
// q/k/v rows 16j .. 16j+15 of the group's [q0; q1; k; v]; o_proj rows 32j .. 32j+31,
// columns 256g .. 256g+255): 960 128-byte lines per workgroup, one 4-byte LDS DMA each,
// line t on worker t % nworkers (the same workers as kv_warm).
// `wl` is the layer's and `wn` the next layer's weight-pointer row.
__device__ __forceinline__ void att_weight_warm_n(const uint16_t* const* wl, const uint16_t* const* wn, int g, int na,
                                                uint32_t lds, int wk, int nworkers, int lane) {
  constexpr int NQL = 16 * 16, NOL = 32 * 4, NGL = 12 * 16, NDL = 32 * 6;  // lines per part
  constexpr int NL = NQL + NOL + 2 * NGL + NDL;
  for (int t = 64 * wk + lane; t < na * NL; t += 64 * nworkers) {
    const int ja = t / NL, v = t - NL * ja;
    const uint8_t* a;
    if (v < NQL) {
      const int r = 16 * ja;
      const uint16_t* w = r < 256   ? uniform_ptr(wn[W_Q]) + (size_t)(256 * g + r) * H
                          : r < 384 ? uniform_ptr(wn[W_K]) + (size_t)(128 * g + r - 256) * H
                                    : uniform_ptr(wn[W_V]) + (size_t)(128 * g + r - 384) * H;
      a = reinterpret_cast<const uint8_t*>(w) + 128 * v;
    } else if (v < NQL + NOL) {
      const int u = v - NQL;
      a = reinterpret_cast<const uint8_t*>(uniform_ptr(wn[W_O]) + (size_t)(ROWS * ja + (u >> 2)) * QS + 256 * g) +
          128 * (u & 3);
    } else if (v < NQL + NOL + 2 * NGL) {
      const int u = v - NQL - NOL;
      const uint16_t* w = uniform_ptr(wl[u < NGL ? W_G : W_U]);
      a = reinterpret_cast<const uint8_t*>(w + (size_t)(XUNITS * g + UNITS * ja) * H) + 128 * (u < NGL ? u : u - NGL);
    } else {
      const int u = v - NQL - NOL - 2 * NGL, row = u / 6;
      a = reinterpret_cast<const uint8_t*>(uniform_ptr(wl[W_D]) + (size_t)(ROWS * ja + row) * I + XUNITS * g) +
          128 * (u - 6 * row);
    }
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(a), "s"(lds)
                 : "memory");
  }
}

// K/V rows of a chunk live in LDS as [row][16 chunks of 8 dims], chunk c of row r
// stored in slot c ^ (r & 15) so that 16 rows read at one chunk hit distinct banks.
__device__ __forceinline__ uint32_t kv_off(int row, int chunk) { return row * 256 + 16 * (chunk ^ (row & 15)); }

// Stream wave s copies K and V rows [0, nc) of the chunk starting at position c0
// (except position p, which the layer itself produces) into LDS.
__device__ __forceinline__ void kv_dma(const DecodeParams& P, int layer, int g, int c0, int nc, int p, uint32_t lds,
                                       int s, int lane) {
  const size_t base = ((size_t)(layer * NKV + g) * P.max_seq_len + c0) * HD;
  const uint16_t* kb = P.k_cache + base;
  const uint16_t* vb = P.v_cache + base;
  const int nq = (nc + 3) >> 2;  // one instruction moves 4 rows
  const int rin = lane >> 4, slot = lane & 15;
  for (int q = s; q < nq; q += NSW) {
    const int row = 4 * q + rin;
    if (row < nc && c0 + row != p) {
      const int chunk = slot ^ (row & 15);
      dma16(kb + row * HD + 8 * chunk, lds + q * 1024);
      dma16(vb + row * HD + 8 * chunk, lds + KV_CAP * 256 + q * 1024);
    }
  }
}

// ---- stream-wave stores: inline assembly, so that the compiler's vmcnt
// bookkeeping for the stream waves' register loads ignores them (each makes a
// later wait at most one instruction longer). The exchange waves never store
// inside the layer loop, so their polls never queue behind a store's write
// acknowledgement. `dev` stores (sc1) write through to memory for readers on
// other XCDs; plain stores stay in this XCD's L2.
__device__ __forceinline__ void st1_dev(uint32_t* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st2_dev(uint32_t* p, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st3_dev(uint32_t* p, u32x3 v) {
  asm volatile("global_store_dwordx3 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st4_dev(uint32_t* p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st1_plain(uint32_t* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st2_plain(uint32_t* p, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st4_plain(uint32_t* p, u32x4 v) {
  asm volatile("global_store_dwordx4 %0, %1, off" ::"v"(p), "v"(v) : "memory");
}

// ---- stream waves -> store wave hand-off: each stream wave writes its results to
// LDS and then bumps an LDS counter; the store wave spins on the counter. LDS
// operations of one wave complete in order, and both sides use DS instructions
// only (no fences, no vector-memory waits).
typedef __attribute__((address_space(3))) uint32_t lds_u32;
__device__ __forceinline__ void signal_store(uint32_t* cnt) {
  asm volatile("" ::: "memory");
  __hip_atomic_fetch_add((lds_u32*)(cnt), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void wait_count(uint32_t* cnt, uint32_t target) {
  while (__hip_atomic_load((lds_u32*)(cnt), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target)
    __builtin_amdgcn_s_sleep(0);
  asm volatile("" ::: "memory");
}

// ---- attention of one chunk for the two query heads of a KV group (all 8 waves)
// The K/V rows of the chunk sit in LDS (rows 0..nc-1; rows nc..255 are zero for the
// whole launch: the LDS copy is cleared once and the copies only ever fill rows < nc).
//
// Scores s_sc[h][r] = (q_h . k_r) * scale for r < nc (-inf past nc), from MFMA tiles
// of 16 rows: wave v takes row blocks v and v + 8. Each wave also leaves the maximum
// of its scores per head in s_mx[v].
__device__ __forceinline__ void attn_scores(const uint8_t* s_kv, const uint16_t* s_q, float (*s_sc)[KV_CAP],
                                            float (*s_mx)[2], int nc, float scale, int v, int lane) {
  const int r16 = lane & 15, kg = lane >> 4;
  u32x4 qb[4];
#pragma unroll
  for (int s4 = 0; s4 < 4; s4++) {
    const u32x4 t = *reinterpret_cast<const u32x4*>(s_q + (r16 & 1) * HD + 32 * s4 + 8 * kg);
    qb[s4] = r16 < 2 ? t : u32x4{0u, 0u, 0u, 0u};
  }
  // blocks v and v + 8 together (rows < 256 always lie in the LDS copy; rows at or past nc
  // are masked): both blocks' K operands are read before the two MFMA chains run
  float mx = -INFINITY;
  u32x4 ka[2][4];
#pragma unroll
  for (int bi = 0; bi < 2; bi++)
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++)
      ka[bi][s4] = *reinterpret_cast<const u32x4*>(s_kv + kv_off(16 * (v + 8 * bi) + r16, 4 * s4 + kg));
  f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int s4 = 0; s4 < 4; s4++) {
    acc[0] = mfma_16x16x32(ka[0][s4], qb[s4], acc[0]);
    acc[1] = mfma_16x16x32(ka[1][s4], qb[s4], acc[1]);
  }
  // lane (column r16 = head, rows 4kg + e)
#pragma unroll
  for (int bi = 0; bi < 2; bi++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int r = 16 * (v + 8 * bi) + 4 * kg + e;
      const float val = r < nc ? acc[bi][e] * scale : -INFINITY;
      if (r16 < 2) s_sc[r16][r] = val;
      mx = fmaxf(mx, val);
    }
  // per-head maximum over the lanes of column 0 (head 0) and column 1 (head 1)
  const float m0 = fmaxf(fmaxf(readlane(mx, 0), readlane(mx, 16)), fmaxf(readlane(mx, 32), readlane(mx, 48)));
  const float m1 = fmaxf(fmaxf(readlane(mx, 1), readlane(mx, 17)), fmaxf(readlane(mx, 33), readlane(mx, 49)));
  if (lane == 0) {
    s_mx[v][0] = m0;
    s_mx[v][1] = m1;
  }
}

// Softmax numerators of this wave's 32 rows (blocks v and v + 8) for both heads:
// lane -> head lane / 32, row 16 (v + 8 ((lane >> 4) & 1)) + (lane & 15). Stores
// bf16(exp(s - max)) in s_p (0 past nc; torch's CPU flash kernel feeds bf16 p to P.V)
// and this wave's unrounded sums in s_l[v]; returns the per-head maxima.
__device__ __forceinline__ void attn_softmax(const float (*s_sc)[KV_CAP], uint16_t* s_p, const float (*s_mx)[2],
                                             float (*s_l)[2], int nc, int v, int lane, float& M0, float& M1) {
  M0 = s_mx[0][0];
  M1 = s_mx[0][1];
#pragma unroll
  for (int k = 1; k < 8; k++) {
    M0 = fmaxf(M0, s_mx[k][0]);
    M1 = fmaxf(M1, s_mx[k][1]);
  }
  const int h = lane >> 5, r = 16 * (v + 8 * ((lane >> 4) & 1)) + (lane & 15);
  const float e = r < nc ? expf(s_sc[h][r] - (h ? M1 : M0)) : 0.f;
  s_p[h * KV_CAP + r] = (uint16_t)f2bf(e);
  const float t = row16_sum(e);
  const float l0 = readlane(t, 0) + readlane(t, 16), l1 = readlane(t, 32) + readlane(t, 48);
  if (lane == 0) {
    s_l[v][0] = l0;
    s_l[v][1] = l1;
  }
}

// acc[h][d] = sum_r bf16(p_h[r]) * v_r[d] for this wave's 16 dims d = 16v + (lane & 15)
// over the 32-row blocks that hold rows < nc (rows past nc have p = 0 and finite V).
// The MFMA operand (8 rows of one dim per lane) comes from two LDS transpose reads:
// within each 16-lane group, lane j addresses row base + j / 4, dims 4 (j % 4) .. +3 of
// the wave's 16, and lane i receives that column's 4 rows (ds_read_b64_tr_b16).
// Writes acc / l (fin) or the raw acc (a split-K partial) to s_ao and returns the
// per-head sums l.
__device__ __forceinline__ void attn_pv(const uint8_t* s_kv, const uint16_t* s_p, const float (*s_l)[2],
                                        float (*s_ao)[HD], int nc, int v, int lane, bool fin, float& L0, float& L1) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  const int r16 = lane & 15, kg = lane >> 4;
  const int dim = 16 * v + r16;
  const int dq = 16 * v + 4 * (r16 & 3);                // this lane's 4 dims in the transpose reads
  const uint32_t vb0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(s_kv + KV_CAP * 256);
  // 32-row blocks in pairs with two accumulators (a block past nc has p = 0: rows < 256
  // always lie in the LDS copy and hold finite values)
  const int nb = (nc + 31) >> 5;
  f32x4 acc2[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  for (int t0 = 0; t0 < nb; t0 += 2) {
    u32x4 pa[2], vb[2];
#pragma unroll
    for (int bi = 0; bi < 2; bi++) {
      const int rr = 32 * (t0 + bi) + 8 * kg;
      const u32x4 pt = *reinterpret_cast<const u32x4*>(s_p + (r16 & 1) * KV_CAP + rr);
      pa[bi] = r16 < 2 ? pt : u32x4{0u, 0u, 0u, 0u};
      const int ra = rr + (r16 >> 2), rb = ra + 4;
      const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_v4s*)(uintptr_t)(vb0 + kv_off(ra, dq >> 3) + 2 * (dq & 7)));
      const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_v4s*)(uintptr_t)(vb0 + kv_off(rb, dq >> 3) + 2 * (dq & 7)));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      vb[bi] = u32x4{l2.x, l2.y, h2.x, h2.y};
    }
    acc2[0] = mfma_16x16x32(pa[0], vb[0], acc2[0]);
    acc2[1] = mfma_16x16x32(pa[1], vb[1], acc2[1]);
  }
  const f32x4 acc = acc2[0] + acc2[1];
  L0 = 0.f;
  L1 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    L0 += s_l[k][0];
    L1 += s_l[k][1];
  }
  if (kg == 0) {
    s_ao[0][dim] = fin ? acc[0] * (1.0f / L0) : acc[0];
    s_ao[1][dim] = fin ? acc[1] * (1.0f / L1) : acc[1];
  }
}

// LM-head row r: bf16 logit of x (two 16-byte chunks per lane) against the row's
// chunks w0, w1; tracks this wave's best (first index on ties) and records the logit.
__device__ __forceinline__ void lm_score(int r, int r0, const u32x4& w0, const u32x4& w1, const u32x4& x0,
                                         const u32x4& x1, float* s_lg, int lane, float& bestv, int& besti) {
  const float v = rbf(wave_sum(dot_chunk(w0, x0, dot_chunk(w1, x1, 0.f))));
  if (lane == 0) s_lg[r - r0] = v;
  if (v > bestv) {
    bestv = v;
    besti = r;
  }
}

// Stream-wave weight registers: one stage's slice each.
struct StreamRegs {
  u32x4 a[8];    // q/k/v: 4 rows x 2 chunks
  u32x4 o[4];    // o_proj partials: 4 rows x 1 chunk
  u32x4 gu[12];  // gate rows of 3 units, then their up rows: 6 rows x 2 chunks
  u32x4 d[8];    // down_proj partials: 8 rows x 1 chunk
  u32x2 wln;     // input_layernorm elements 4t .. 4t+3
  u32x2 wpost;   // post_attention_layernorm elements 4t .. 4t+3
  uint32_t qkn;  // q_norm (t < 64) / k_norm (t >= 64) elements 2t, 2t+1 (mod 128)
};

// Exchange waves: one 16-byte chunk (4 tagged words) as fp32 values.
__device__ __forceinline__ void unpack_tagged(const u32x4& v, float* f) {
  f[0] = bflo(v.x);
  f[1] = bflo(v.y);
  f[2] = bflo(v.z);
  f[3] = bflo(v.w);
}

// This poll wave's half of a gathered residual stream (chunks lane + 128c into v0 and
// lane + 128c + 64 into v1) and the stream's sum of squares, added up from the 32 per-workgroup
// sums of squares published with it (the same order in both poll waves, so their norms
// agree bit for bit).
__device__ __forceinline__ float gather_half(const Buf& b, uint32_t* ws, uint32_t base, uint32_t ssbase, uint32_t tag,
                                             uint32_t tag64, int c, int lane, u32x4& v0, u32x4& v1) {
  const uint32_t w0 = base + 4 * (lane + 128 * c), w1 = w0 + 4 * 64;
  const uint32_t wq = ssbase + 4 * (lane & 15);  // the sums of workgroups 2 (lane % 16) and +1
  // poll only the 32 sums of squares (each producer stores its sum after its rows): a
  // third of the polling traffic of polling rows and sums together, which measured 6 us
  // faster per token; then load the rows once and re-poll any that are still stale
  u32x4 q = ldl4(b, wq);
  auto fresh = [&](const u32x4& x) { return (x.y == tag64) & (x.w == tag64); };
  uint32_t spins = 0;
  while (!fresh(q)) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    q = ldl4(b, wq);
  }
  u32x4 a = ldl4(b, w0), e = ldl4(b, w1);
  while (!(tags_ok(a, tag) & tags_ok(e, tag) & fresh(q))) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    if (!tags_ok(a, tag)) a = ldl4(b, w0);
    if (!tags_ok(e, tag)) e = ldl4(b, w1);
    if (!fresh(q)) q = ldl4(b, wq);
  }
  v0 = a;
  v1 = e;
  return wave_sum(lane < 16 ? __uint_as_float(q.x) + __uint_as_float(q.z) : 0.f);
}

// HF Qwen3RMSNorm (modeling_qwen3.py:59-64) of one chunk: y = bf16(w * bf16(x * rstd)),
// written as two bf16 pairs.
__device__ __forceinline__ void norm_chunk(const float* x, float rstd, uint32_t w0, uint32_t w1, uint32_t* dst) {
  dst[0] = pack_bf2(rbf(bflo(w0) * rbf(x[0] * rstd)), rbf(bfhi(w0) * rbf(x[1] * rstd)));
  dst[1] = pack_bf2(rbf(bflo(w1) * rbf(x[2] * rstd)), rbf(bfhi(w1) * rbf(x[3] * rstd)));
}

// ---------------------------------------------------------------- the kernel
// SPLIT = false is the instance for contexts of at most KV_CAP positions (one
// attention workgroup per XCD, one LDS pass): the chunk-merge and two-pass code
// is compiled out of it. SPLIT = true handles every context length.
template <bool SPLIT>
__global__ void __launch_bounds__(NT, 1) mq_decode_kernel(DecodeParams P) {
  __shared__ __align__(16) uint8_t s_kv[2 * KV_CAP * HD * 2];  // K rows, then V rows of the chunk
  __shared__ __align__(16) uint32_t s_x0[H / 2];               // normed h or h1 (bf16 pairs)
  __shared__ __align__(16) uint32_t s_x1[XUNITS / 2];          // attention output or m of the XCD (bf16 pairs)
  __shared__ __align__(16) uint32_t s_wln[H / 2];              // input_layernorm weights
  __shared__ __align__(16) uint32_t s_wpost[H / 2];            // post_attention_layernorm weights
  __shared__ __align__(16) uint32_t s_wfn[H / 2];              // final norm weights
  __shared__ uint32_t s_qkn[HD];                               // q_norm words, then k_norm words
  __shared__ float s_cos[HD], s_sin[HD];
  __shared__ __align__(16) uint16_t s_q[2 * HD];      // normed, rotated q of the two heads
  __shared__ __align__(16) uint16_t s_p[2 * KV_CAP];  // bf16 softmax numerators
  __shared__ float s_sc[2][KV_CAP];                    // attention scores
  __shared__ float s_ao[2][HD];                        // attention output (or unnormalised partial)
  __shared__ float s_ao1[2][HD];                       // second LDS pass's unnormalised partial
  __shared__ float s_mx[8][2], s_l[8][2];              // per-wave score maxima and softmax sums
  __shared__ float s_hrow[ROWS];                       // residual rows 32j .. 32j+31 of h
  __shared__ float s_res[ROWS];                        // stream-wave dot products for the store wave
  __shared__ uint32_t s_cnt;                           // stream-wave results published so far
  __shared__ uint32_t s_attst;                         // attention-output stores issued by the store wave
  __shared__ const uint16_t* s_lw[MAX_LAYERS][11];    // weight pointers, copied once per launch
  __shared__ float s_bestv[8];
  __shared__ int s_besti[8];
  __shared__ uint32_t s_flag;
  float* s_lg = reinterpret_cast<float*>(s_kv);  // this workgroup's logits (K/V rows are dead by then)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // The XCD-local exchanges (plain stores, L2-coherent loads) need each workgroup's group
  // g to be the XCD it runs on, so g is read from the hardware. The dispatcher deals
  // workgroups to the XCDs in turn, starting at an XCD that depends on the launch path
  // (an ordinary launch starts at 0, a HIP graph node need not): the XCD of workgroup w
  // is (w + start) % 8 and j = w / 8 numbers the 32 workgroups of each XCD. Were the
  // deal different, a member slot would stay unfilled and a bounded wait would report
  // the error; no exchange can complete with a wrong member.
  uint32_t xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  const int w = blockIdx.x, g = (int)(xcc & (NXCD - 1)), j = w / NXCD;
  uint32_t* ws = P.ws;
  const Buf wsb(ws);
  // token, position, epoch: kernel arguments, or a device-resident step written by the
  // previous launch's last workgroup (visible at this launch's start)
  int token = P.token, p = P.position, step_count = 0;
  uint32_t epoch = P.epoch;
  if (P.mode & MODE_DEVICE_STEP) {
    const u32x4 sv = *(const gu32x4*)(const void*)P.step;
    token = (int)__builtin_amdgcn_readfirstlane(sv.x);
    p = (int)__builtin_amdgcn_readfirstlane(sv.y);
    epoch = __builtin_amdgcn_readfirstlane(sv.z);
    step_count = (int)__builtin_amdgcn_readfirstlane(sv.w);
    // Every workgroup reads the same step, so all of them leave here together. The first
    // failing step records its error; later launches find the negative token and return.
    if (token < 0 || token >= VOCAB || p < 0 || p >= P.max_seq_len || p >= MAX_CTX || (!SPLIT && p >= KV_CAP) ||
        step_count >= P.out_capacity) {
      if (w == 0 && tid == 0 && token >= 0 && step_count < P.out_capacity) {
        P.out_ids[step_count] = -(int)(1u + ERR_STEP);
        P.step->token = -(int)(1u + ERR_STEP);
        P.step->count = step_count + 1;
      }
      return;
    }
  }
  if (tid == 0 && (xcc & 15u) >= (uint32_t)NXCD) raise_error(ws, ERR_XCD);
  const uint32_t lb = WS_LOCAL + g * LOCAL_WORDS;  // this XCD's exchange region
  const int L = P.num_layers;
  const bool lm = !(P.mode & MODE_NO_LMHEAD);

  // attention chunking: nsplit chunks of <= 2 KV_CAP positions, chunk j on workgroup (g, j),
  // attended in npass LDS passes of <= KV_CAP positions (rows KV_CAP.. in the second)
  const int n_ctx = p + 1;
  const int nsplit = SPLIT ? plan_nsplit(n_ctx) : 1;
  const int CH = SPLIT ? plan_chunk(n_ctx) : n_ctx;
  const bool att = j < nsplit;
  const int c0 = j * CH;
  const int nc = att ? min(n_ctx, c0 + CH) - c0 : 0;
  const int npass = SPLIT ? (nc + KV_CAP - 1) / KV_CAP : 1;
  const int nc0 = min(nc, KV_CAP);
  const bool own_p = att && p >= c0 && p < c0 + nc;  // p is always in the last pass
  const int prow = p - c0 - KV_CAP * (npass - 1);     // its LDS row there
  const uint32_t lds_kv = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)s_kv;

  // LM-head rows of this workgroup: 594 for w < 128, 593 after (151936 in total)
  const int r0 = w < 128 ? w * 594 : 128 * 594 + (w - 128) * 593;
  const int r1 = r0 + (w < 128 ? 594 : 593);

  float bestv = -INFINITY;
  int besti = 0x7fffffff;
  const u32x4* x0v = reinterpret_cast<const u32x4*>(s_x0);
  const u32x4* x1v = reinterpret_cast<const u32x4*>(s_x1);

  // rows past the chunk length must read as zeros in every layer
  for (int i = tid; i < 2 * KV_CAP * HD * 2 / 16; i += NT) reinterpret_cast<u32x4*>(s_kv)[i] = u32x4{0u, 0u, 0u, 0u};

  if (wave < NSW) {
    // ==================================================================== stream waves
    const int s = wave, st = tid;  // st: stream thread 0..255
    for (int i = st; i < L * 11; i += NSW * 64)
      s_lw[i / 11][i % 11] = reinterpret_cast<const uint16_t* const*>(P.layers)[i];
    BAR();  // P00: pointer table visible
    // Weight pointer k of layer l; l >= L (the next-layer loads of the last layer)
    // maps to layer 0.
    auto wp = [&](int l, int k) -> const uint16_t* { return uniform_ptr(s_lw[l < L ? l : 0][k]); };
    // During the last layer the registers are refilled with this wave's first LM-head rows.
    const uint16_t* lmb = P.lm_head + (size_t)(r0 + LM_PRE * s) * H;
    const bool lmnext = lm;
    // o_proj: this lane's 16-byte chunk c of the group's 256 columns, rows 8s + rg + 2i
    const int oc = lane & 31, org = lane >> 5;
    // down_proj: lanes < 48 take chunk `lane` of the XCD's 384 columns (the others re-read chunk 47
    // and are multiplied by zero)
    const int dch = lane < 48 ? lane : 47;

    StreamRegs R;
    auto load_a = [&](int l) {
      const int r = 16 * j + 4 * s;  // this wave's 4 rows of the group's [q0; q1; k; v]
      const uint16_t* pa = (l >= L && lmnext) ? lmb
                           : r < 256          ? wp(l, W_Q) + (size_t)(256 * g + r) * H
                           : r < 384          ? wp(l, W_K) + (size_t)(128 * g + r - 256) * H
                                              : wp(l, W_V) + (size_t)(128 * g + r - 384) * H;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        R.a[2 * k] = ldw(pa + k * H + 8 * lane);
        R.a[2 * k + 1] = ldw(pa + k * H + 512 + 8 * lane);
      }
    };
    auto load_o = [&](int l) {
      const bool lmr = l >= L && lmnext;
      // LM rows 4, 5 of this wave as chunks lane, lane + 64 of two consecutive rows
      const uint16_t* po = lmr ? lmb + 4 * H : wp(l, W_O) + (size_t)(ROWS * j + 8 * s + org) * QS + 256 * g + 8 * oc;
#pragma unroll
      for (int i = 0; i < 4; i++) R.o[i] = ldw(po + (lmr ? 8 * (lane + 64 * i) : (size_t)(2 * i) * QS));
    };
    auto load_gu = [&](int l) {
      R.wln = ldw2(wp(l + 1, W_IN) + 4 * st);  // the next layer's input norm and q/k norms
      R.qkn = ldw1(wp(l + 1, st < 64 ? W_QN : W_KN) + 2 * (st & 63));
      const bool lmr = l >= L && lmnext;
      const uint16_t* pg = lmr ? lmb + 6 * H : wp(l, W_G) + (size_t)(XUNITS * g + UNITS * j + 3 * s) * H;
      const uint16_t* pu = lmr ? lmb + 9 * H : wp(l, W_U) + (size_t)(XUNITS * g + UNITS * j + 3 * s) * H;
#pragma unroll
      for (int k = 0; k < 3; k++) {
        R.gu[2 * k] = ldw(pg + k * H + 8 * lane);
        R.gu[2 * k + 1] = ldw(pg + k * H + 512 + 8 * lane);
      }
#pragma unroll
      for (int k = 0; k < 3; k++) {
        R.gu[6 + 2 * k] = ldw(pu + k * H + 8 * lane);
        R.gu[7 + 2 * k] = ldw(pu + k * H + 512 + 8 * lane);
      }
    };
    auto load_d = [&](int l) {
      R.wpost = ldw2(wp(l + 1, W_POST) + 4 * st);  // the next layer's post-attention norm
      const bool lmr = l >= L && lmnext;
      // LM rows 12 .. 15 of this wave as chunks lane, lane + 64 of four consecutive rows
      const uint16_t* pd = lmr ? lmb + 12 * H : wp(l, W_D) + (size_t)(ROWS * j + 8 * s) * I + XUNITS * g + 8 * dch;
#pragma unroll
      for (int i = 0; i < 8; i++) R.d[i] = ldw(pd + (lmr ? 8 * (lane + 64 * i) : (size_t)i * I));
    };

    auto burst = [&](int l) {
      load_o(l);
      load_gu(l);
      load_d(l);
      load_a(l + 1);
    };

    // ---- prologue: layer-0 norms to LDS, layer-0 K/V copy, layer-0 weights in flight
    {
      const u32x2 ln0 = ldw2(wp(0, W_IN) + 4 * st);
      const uint32_t qk0 = ldw1(wp(0, st < 64 ? W_QN : W_KN) + 2 * (st & 63));
      const u32x2 pn0 = ldw2(wp(0, W_POST) + 4 * st);
      s_wln[2 * st] = ln0.x;
      s_wln[2 * st + 1] = ln0.y;
      s_wpost[2 * st] = pn0.x;
      s_wpost[2 * st + 1] = pn0.y;
      if (st < 128) s_qkn[st] = qk0;
      if (lm) {
        const u32x2 fn = ldw2(P.final_norm + 4 * st);
        s_wfn[2 * st] = fn.x;
        s_wfn[2 * st + 1] = fn.y;
      }
    }
    if (att) kv_dma(P, 0, g, c0, nc0, p, lds_kv, s, lane);
    load_a(0);
    if (att) load_o(0);
    BAR();  // P0

    for (int layer = 0; layer < L; layer++) {
      const int nl = layer + 1;
      // ---------------- q/k/v rows 16j + 4s .. +3 of the group's [q0; q1; k; v]
      BAR();  // A1: normed h in s_x0
      MQ_STAMP(layer * 40 + 0);
      {
        if (layer > 0) {
          s_wpost[2 * st] = R.wpost.x;  // this layer's post-attention norm
          s_wpost[2 * st + 1] = R.wpost.y;
        }
        const u32x4 x0 = x0v[lane], x1 = x0v[64 + lane];
        float r[4];
#pragma unroll
        for (int k = 0; k < 4; k++) r[k] = dot_chunk(R.a[2 * k], x0, dot_chunk(R.a[2 * k + 1], x1, 0.f));
        wave_sum_n(r);
        if (lane == 0) {
#pragma unroll
          for (int k = 0; k < 4; k++) s_res[4 * s + k] = r[k];
          signal_store(&s_cnt);
        }
        AFTER(r[0] + r[1] + r[2] + r[3]);
        MQ_STAMP(layer * 40 + 1);
        // Workgroups without attention load the rest of the layer's weights and the next
        // layer's q/k/v in one burst: it drains while attention runs elsewhere, so the
        // exchanges after attention find this CU's vector-memory pipeline idle (a poll queued
        // behind in-flight HBM loads waits for them). Attention workgroups poll q/k/v right
        // after this stage: they load o_proj at the end of the previous layer and the rest
        // once attention is done.
        if (!att) burst(layer);
      }
      if (att) {
        // this wave's K/V copy of the layer has landed: all of the wave's vector-memory
        // operations are awaited (the copy is inline assembly the compiler does not count;
        // the o_proj loads issued after it are needed right after the attention anyway)
        wait_vmem();
        for (int ps = 0; ps < npass; ps++) {
          if (ps == 1) {
            // second pass: rows KV_CAP .. nc-1 of the chunk replace the first pass's rows
            kv_dma(P, layer, g, c0 + KV_CAP, nc - KV_CAP, p, lds_kv, s, lane);
            wait_vmem();
          }
          const int ncp = ps ? nc - KV_CAP : nc0;
          BAR();  // B1: q, the new k/v row and the K/V rows are in LDS
          MQ_STAMP(layer * 40 + 2);
          attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
          BAR();  // B2
          MQ_STAMP(layer * 40 + 10);
          float M0, M1, L0, L1;
          attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
          BAR();  // B3
          MQ_STAMP(layer * 40 + 11);
          attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1);
          BAR();  // B4: K/V rows consumed
          MQ_STAMP(layer * 40 + 3);
        }
        // the store wave's attention-output store goes first: a CU's vector-memory
        // instructions leave in order, so behind these loads it reached L2 late for
        // the 31 workgroups that wait on it
        wait_count(&s_attst, (uint32_t)layer + 1u);
        load_gu(layer);
      }
      // ---------------- o_proj partials: rows 32j + 8s + 2i + rg over the group's 256 columns
      BAR();  // C1: attention output of the group in s_x1
      MQ_STAMP(layer * 40 + 4);
      {
        const u32x4 xa = x1v[oc];
        float r[4];
#pragma unroll
        for (int i = 0; i < 4; i++) r[i] = dot_chunk(R.o[i], xa, 0.f);
        row16_sum_n(r);
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < 4; i++) {
            s_res[8 * s + 2 * i] = readlane(r[i], 0) + readlane(r[i], 16);
            s_res[8 * s + 2 * i + 1] = readlane(r[i], 32) + readlane(r[i], 48);
          }
          signal_store(&s_cnt);
        }
        AFTER(r[0] + r[1] + r[2] + r[3]);
        MQ_STAMP(layer * 40 + 5);
        if (att) load_d(layer);
      }
      // ---------------- gate/up rows of units 384g + 12j + 3s .. +2
      BAR();  // D1: normed h1 in s_x0
      MQ_STAMP(layer * 40 + 6);
      {
        s_wln[2 * st] = R.wln.x;  // the next layer's input norm and q/k norms
        s_wln[2 * st + 1] = R.wln.y;
        if (st < 128) s_qkn[st] = R.qkn;
        const u32x4 x0 = x0v[lane], x1 = x0v[64 + lane];
        float r[6];
#pragma unroll
        for (int k = 0; k < 6; k++) r[k] = dot_chunk(R.gu[2 * k], x0, dot_chunk(R.gu[2 * k + 1], x1, 0.f));
        wave_sum_n(r);
        if (lane == 0) {
#pragma unroll
          for (int k = 0; k < 6; k++) s_res[6 * s + k] = r[k];
          signal_store(&s_cnt);
        }
        AFTER(r[0] + r[1] + r[2] + r[3] + r[4] + r[5]);
        MQ_STAMP(layer * 40 + 7);
        if (att) load_a(nl);
        // the next layer's K/V rows: the LDS copy is free since B4, and its completion is
        // first needed behind the next layer's q/k/v weights
        if (att && nl < L) kv_dma(P, nl, g, c0, nc0, p, lds_kv, s, lane);
      }
      // ---------------- down_proj partials: rows 32j + 8s + i over the XCD's 384 units
      BAR();  // E1: m of the XCD in s_x1
      MQ_STAMP(layer * 40 + 8);
      {
        const u32x4 xm = lane < 48 ? x1v[lane] : u32x4{0u, 0u, 0u, 0u};
        float r[8];
#pragma unroll
        for (int i = 0; i < 8; i++) r[i] = dot_chunk(R.d[i], xm, 0.f);
        wave_sum_n(r);
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < 8; i++) s_res[8 * s + i] = r[i];
          signal_store(&s_cnt);
        }
        AFTER(r[0] + r[1] + r[2] + r[3] + r[4] + r[5] + r[6] + r[7]);
        MQ_STAMP(layer * 40 + 9);
        if (att && nl < L) load_o(nl);
      }
    }
    BAR();  // F1: final normed h in s_x0
    if (lm) {
      const u32x4 x0 = x0v[lane], x1 = x0v[64 + lane];
      const int rb = r0 + LM_PRE * s;
#pragma unroll
      for (int k = 0; k < 4; k++) lm_score(rb + k, r0, R.a[2 * k], R.a[2 * k + 1], x0, x1, s_lg, lane, bestv, besti);
    }
  } else if (wave < NSW + NPW) {
    // ==================================================================== poll waves
    const int c = wave - NSW, pt = tid - NSW * 64;  // pt: poll thread 0..127
    for (int i = pt; i < 2 * HD; i += NPW * 64) {
      if (i < HD) s_cos[i] = bf2f(ldraw16(P.cos_tab + (size_t)p * HD + i));
      else s_sin[i - HD] = bf2f(ldraw16(P.sin_tab + (size_t)p * HD + i - HD));
    }
    BAR();  // P00
    BAR();  // P0

    // RMSNorm of a gathered residual-stream vector (chunks lane + 64k, k < 4): poll wave c
    // writes the normalised chunks k = 2c, 2c + 1 to s_x0
    auto norm_out = [&](const u32x4& hv0, const u32x4& hv1, float ss, const uint32_t* wn) {
      const float rstd = 1.0f / sqrtf(ss * (1.0f / H) + EPS);
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int k = 2 * c + q;
        float f[4];
        unpack_tagged(q ? hv1 : hv0, f);
        const int ch = lane + 64 * k;
        norm_chunk(f, rstd, wn[2 * ch], wn[2 * ch + 1], s_x0 + 2 * ch);
      }
    };
    // rows 32j .. 32j+31 (chunks 8j .. 8j+7, all in block k = j / 8) for the reduce wave
    auto keep_rows = [&](const u32x4& hv0, const u32x4& hv1, float* dst) {
      const int q = lane - ((8 * j) & 63);
      if (c == (j >> 4) && q >= 0 && q < 8) {  // block j / 8 is in this wave's half
        float f[4];
        unpack_tagged((j >> 3) & 1 ? hv1 : hv0, f);
#pragma unroll
        for (int e = 0; e < 4; e++) dst[4 * q + e] = f[e];
      }
    };

    u32x4 hv0, hv1;  // this wave's half of the residual stream: chunks lane + 128c and lane + 128c + 64
    for (int layer = 0; layer < L; layer++) {
      const uint32_t tag = tag_of(epoch, layer);
      const uint32_t tag64 = epoch * 32u + (uint32_t)layer + 1u;
      MQ_STAMP(layer * 40 + 12);
      // ---------------- gather h (each poll wave its half, with the sum of squares), RMSNorm
      float ss;
      if (layer == 0) {
        const uint16_t* src = (P.mode & MODE_INPUT_HIDDEN) ? P.hidden_in : P.embed + (size_t)token * H;
        ss = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const u32x2 v = ldw2(src + 4 * (lane + 64 * k));
          // widen the raw bf16 values to the tagged layout so every layer reads hv alike
          const u32x4 t = u32x4{v.x & 0xffffu, v.x >> 16, v.y & 0xffffu, v.y >> 16};
          if (k == 2 * c) hv0 = t;
          if (k == 2 * c + 1) hv1 = t;
          float f[4];
          unpack_tagged(t, f);
          ss += (f[0] * f[0] + f[1] * f[1]) + (f[2] * f[2] + f[3] * f[3]);
        }
        ss = wave_sum(ss);
      } else {
        ss = gather_half(wsb, ws, lb + LX_H, lb + LX_HSS, tag_of(epoch, layer - 1), epoch * 32u + (uint32_t)layer, c, lane,
                         hv0, hv1);
      }
      MQ_STAMP(layer * 40 + 13);
      norm_out(hv0, hv1, ss, s_wln);
      MQ_STAMP(layer * 40 + 26);
      keep_rows(hv0, hv1, s_hrow);
      BAR();  // A1
      MQ_STAMP(layer * 40 + 14);
      if (att) {
        // ---------------- QK-norm, RoPE, K/V row p, attention
        // wave 0: q heads 2g and 2g+1; wave 1: k and v; lane holds dims lane, lane + 64
        uint32_t u[4];
        const uint32_t wq = lb + LX_QKV + 2 * HD * c;
#pragma unroll
        for (int q = 0; q < 4; q++) u[q] = ldl1(wsb, wq + 64 * q + lane);
        {
          uint32_t spins = 0;
          while (((u[0] >> 16) != tag) | ((u[1] >> 16) != tag) | ((u[2] >> 16) != tag) | ((u[3] >> 16) != tag)) {
            if (watchdog(wsb, ws, ++spins)) break;
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int q = 0; q < 4; q++)
              if ((u[q] >> 16) != tag) u[q] = ldl1(wsb, wq + 64 * q + lane);
          }
        }
        MQ_STAMP(layer * 40 + 15);
        // HF: q_norm/k_norm over 128 (modeling_qwen3.py:252-253), then apply_rotary_pos_emb (:147-170)
        const int nseg = c == 0 ? 2 : 1;  // segments that get QK-norm and RoPE
        float fr[2][2];
#pragma unroll
        for (int sg = 0; sg < 2; sg++) {
          float fa = bflo(u[2 * sg]), fb = bflo(u[2 * sg + 1]);
          if (sg < nseg) {
            const float ssq = wave_sum(fa * fa + fb * fb);
            const float rstd = 1.0f / sqrtf(ssq * (1.0f / HD) + EPS);
            const int nw0 = c == 1 ? 64 : 0;
            const uint32_t na = s_qkn[nw0 + (lane >> 1)], nb = s_qkn[nw0 + 32 + (lane >> 1)];
            const float wa = (lane & 1) ? bfhi(na) : bflo(na), wb = (lane & 1) ? bfhi(nb) : bflo(nb);
            fa = rbf(wa * rbf(fa * rstd));
            fb = rbf(wb * rbf(fb * rstd));
            const float ra = rbf(rbf(fa * s_cos[lane]) - rbf(fb * s_sin[lane]));
            const float rb = rbf(rbf(fb * s_cos[lane + 64]) + rbf(fa * s_sin[lane + 64]));
            fa = ra;
            fb = rb;
          }
          fr[sg][0] = fa;
          fr[sg][1] = fb;
        }
        if (c == 0) {
#pragma unroll
          for (int sg = 0; sg < 2; sg++) {
            s_q[sg * HD + lane] = (uint16_t)f2bf(fr[sg][0]);
            s_q[sg * HD + 64 + lane] = (uint16_t)f2bf(fr[sg][1]);
          }
        }
        MQ_STAMP(layer * 40 + 25);
        for (int ps = 0; ps < npass; ps++) {
          if (c == 1 && own_p && ps == npass - 1) {
            // the new k and v rows into the LDS copy of the pass that holds position p (the
            // store wave appends them to the cache); a second pass's copy excludes that row
            const int o0 = kv_off(prow, lane >> 3) + 2 * (lane & 7);
            const int o1 = kv_off(prow, 8 + (lane >> 3)) + 2 * (lane & 7);
#pragma unroll
            for (int sg = 0; sg < 2; sg++) {
              uint8_t* base = s_kv + sg * (KV_CAP * 256);
              *reinterpret_cast<uint16_t*>(base + o0) = (uint16_t)f2bf(fr[sg][0]);
              *reinterpret_cast<uint16_t*>(base + o1) = (uint16_t)f2bf(fr[sg][1]);
            }
          }
          const int ncp = ps ? nc - KV_CAP : nc0;
          BAR();  // B1
          MQ_STAMP(layer * 40 + 16);
          attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
          BAR();  // B2
          float M0, M1, L0, L1;
          attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
          BAR();  // B3
          attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1);
          BAR();  // B4
        }
        MQ_STAMP(layer * 40 + 17);
      }
      // ---------------- o_proj input: the group's 256 attention outputs as bf16 pairs in s_x1
      if (nsplit == 1) {
        // poll wave 0: the attention workgroup has them in LDS, the others gather them
        if (c == 0) {
          if (att) {
            const int hh = lane >> 5, dim = 4 * (lane & 31);
            const float* src = &s_ao[hh][dim];
            reinterpret_cast<u32x2*>(s_x1)[lane] =
                u32x2{pack_bf2(rbf(src[0]), rbf(src[1])), pack_bf2(rbf(src[2]), rbf(src[3]))};
          } else {
            u32x4 v = ldl4(wsb, lb + LX_ATT + 4 * lane);
            v = repoll_l4(wsb, ws, lb + LX_ATT + 4 * lane, tag, v);
            reinterpret_cast<u32x2*>(s_x1)[lane] = u32x2{pair_lo(v.x, v.y), pair_lo(v.z, v.w)};
          }
        }
      } else {
        // every workgroup merges the XCD's chunk partials itself, straight into its o_proj
        // input: thread pt takes dims d0, d0 + 1 of head hh (a poll wave per head), CG chunks
        // per round; lane q loads chunk q's (m, l), which the wave then reads by readlane
        const int hh = pt >> 6, d0 = 2 * (pt & 63);
        float Mc = -INFINITY, Lc = 0.f, O0 = 0.f, O1 = 0.f;
        // nine chunks a round: contexts up to 2303 positions merge in one round (2048 and
        // past take nine chunks); measured against 4 and 12 a round, and 6, 8 and 16 spill
        constexpr int CG = 9;
        for (int s0 = 0; s0 < nsplit; s0 += CG) {
          const int nq = min(CG, nsplit - s0);
          const uint32_t b0 = lb + LX_PART + 2 * ((s0 * 2 + hh) * APART);
          const bool mlane = lane < nq;
          const uint32_t bml = b0 + 4 * min(lane, nq - 1) * APART;
          u32x4 ml, ov[CG];  // this lane's chunk (m, tag, l, tag); (acc[d0], tag, acc[d0 + 1], tag) per chunk
          ml = ldl4(wsb, bml);
          auto fresh = [&](const u32x4& v) { return (v.y == tag64) & (v.w == tag64); };
          uint32_t spins = 0;
          // the chunks' (m, l) first (each stored after its chunk's accumulators, and polled
          // by one lane per chunk): far less polling traffic than polling every
          // accumulator pair, 5-14 us per token at split contexts
          while (mlane && !fresh(ml)) {
            if (watchdog(wsb, ws, ++spins)) break;
            __builtin_amdgcn_s_sleep(1);
            ml = ldl4(wsb, bml);
          }
#pragma unroll
          for (int q = 0; q < CG; q++)
            if (q < nq) ov[q] = ldl4(wsb, b0 + 4 * q * APART + 4 + 2 * d0);
          for (;;) {
            bool ok = !mlane || fresh(ml);
#pragma unroll
            for (int q = 0; q < CG; q++) ok &= q >= nq || fresh(ov[q]);
            if (ok || watchdog(wsb, ws, ++spins)) break;
            __builtin_amdgcn_s_sleep(1);
            if (mlane && !fresh(ml)) ml = ldl4(wsb, bml);
#pragma unroll
            for (int q = 0; q < CG; q++)
              if (q < nq && !fresh(ov[q])) ov[q] = ldl4(wsb, b0 + 4 * q * APART + 4 + 2 * d0);
          }
#pragma unroll
          for (int q = 0; q < CG; q++)
            if (q < nq) {
              const float m = __uint_as_float(__builtin_amdgcn_readlane(ml.x, q));
              const float l = __uint_as_float(__builtin_amdgcn_readlane(ml.z, q));
              const float nm = fmaxf(Mc, m);
              const float ea = Mc == -INFINITY ? 0.f : expf(Mc - nm), eb = expf(m - nm);
              Lc = Lc * ea + l * eb;
              O0 = O0 * ea + __uint_as_float(ov[q].x) * eb;
              O1 = O1 * ea + __uint_as_float(ov[q].z) * eb;
              Mc = nm;
            }
        }
        const float rl = 1.0f / Lc;
        s_x1[pt] = pack_bf2(rbf(O0 * rl), rbf(O1 * rl));
      }
      MQ_STAMP(layer * 40 + 19);
      BAR();  // C1
      MQ_STAMP(layer * 40 + 20);
      // ---------------- gather h1; post-attention RMSNorm
      {
        const float ss1 = gather_half(wsb, ws, lb + LX_H1, lb + LX_H1SS, tag, tag64, c, lane, hv0, hv1);
        MQ_STAMP(layer * 40 + 21);
        norm_out(hv0, hv1, ss1, s_wpost);
        MQ_STAMP(layer * 40 + 27);
      }
      BAR();  // D1
      MQ_STAMP(layer * 40 + 22);
      // ---------------- down_proj input: m of the XCD's 384 units (96 chunks)
      {
        const int q = pt;  // chunks pt, pt + 128 (< 96 only for pt < 96)
        if (q < XUNITS / 4) {
          u32x4 v = ldl4(wsb, lb + LX_M + 4 * q);
          v = repoll_l4(wsb, ws, lb + LX_M + 4 * q, tag, v);
          reinterpret_cast<u32x2*>(s_x1)[q] = u32x2{pair_lo(v.x, v.y), pair_lo(v.z, v.w)};
        }
      }
      MQ_STAMP(layer * 40 + 23);
      BAR();  // E1
      MQ_STAMP(layer * 40 + 24);
    }

    // ---------------- final norm
    {
      const float ss = gather_half(wsb, ws, lb + LX_H, lb + LX_HSS, tag_of(epoch, L - 1), epoch * 32u + (uint32_t)L, c, lane,
                                   hv0, hv1);
      MQ_STAMP(32 * 40);
      if (lm) norm_out(hv0, hv1, ss, s_wfn);
      if (w == 0) {
        // hidden_out / normed_out chunks k = 2c, 2c + 1
#pragma unroll
        for (int q = 0; q < 2; q++) {
          const int k = 2 * c + q;
          float f[4];
          unpack_tagged(q ? hv1 : hv0, f);
          const int ch = lane + 64 * k;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            P.hidden_out[4 * ch + e] = (uint16_t)f2bf(f[e]);
            if (lm && P.normed_out) P.normed_out[4 * ch + e] = bf2f((s_x0[2 * ch + (e >> 1)] >> (16 * (e & 1))) & 0xffffu);
          }
        }
      }
    }
    BAR();  // F1
  } else if (wave == NSW + NPW) {
    // ==================================================================== reduce wave
    // Residual rows 32j .. 32j+31 from the 8 XCDs' partial sums (identical on every XCD):
    // lane -> row lane >> 1, XCDs 4 (lane & 1) .. +3.
    BAR();  // P00
    BAR();  // P0
    const int rr = lane >> 1, hx = lane & 1;
    float h1v = 0.f;  // h1 row rr (kept for the down_proj residual)
    // sum of the 8 partials of row rr of `part` in XCD order, identical in both lanes of the pair
    auto reduce_row = [&](uint32_t part, uint32_t tag64) -> float {
      const uint32_t wd = part + 2 * ((j * ROWS + rr) * NXCD + 4 * hx);
      auto ok = [&](const u32x4& v) { return (v.y == tag64) & (v.w == tag64); };
      uint32_t spins = 0;
      u32x4 a = xld4(wsb, wd), b = xld4(wsb, wd + 4);
      // re-poll both stale halves at once (one round trip per iteration)
      while (!(ok(a) & ok(b))) {
        if (watchdog(wsb, ws, ++spins)) break;
        __builtin_amdgcn_s_sleep(1);
        if (!ok(a)) a = xld4(wsb, wd);
        if (!ok(b)) b = xld4(wsb, wd + 4);
      }
      const float s4 = (__uint_as_float(a.x) + __uint_as_float(a.z)) + (__uint_as_float(b.x) + __uint_as_float(b.z));
      return s4 + dpp<0xB1>(s4);  // (XCDs 0..3) + (XCDs 4..7), commutative: same bits in both lanes
    };
    for (int layer = 0; layer < L; layer++) {
      const uint32_t tag = tag_of(epoch, layer);
      const uint32_t tag64 = epoch * 32u + (uint32_t)layer + 1u;
      BAR();  // A1: h rows in s_hrow
      MQ_STAMP(layer * 40 + 28);
      const float hrow = s_hrow[rr];
      if (att) {
        for (int ps = 0; ps < npass; ps++) {
          const int ncp = ps ? nc - KV_CAP : nc0;
          BAR();  // B1
          attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
          BAR();  // B2
          float M0, M1, L0, L1;
          attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
          BAR();  // B3
          attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1);
          BAR();  // B4
        }
      }
      BAR();  // C1
      MQ_STAMP(layer * 40 + 29);
      // h1 = bf16(h + bf16(o)) (modeling_qwen3.py:297-298)
      h1v = rbf(hrow + rbf(reduce_row(X_OPART, tag64)));
      if (hx == 0) st1_plain(ws + lb + LX_H1 + ROWS * j + rr, tagged(tag, h1v));
      {
        const float ssr = wave_sum(hx == 0 ? h1v * h1v : 0.f);
        if (lane == 0) st2_plain(ws + lb + LX_H1SS + 2 * j, u32x2{__float_as_uint(ssr), tag64});
      }
      MQ_STAMP(layer * 40 + 30);
      BAR();  // D1
      BAR();  // E1
      MQ_STAMP(layer * 40 + 31);
      // h' = bf16(h1 + bf16(down)) (modeling_qwen3.py:303-304)
      const float hn = rbf(h1v + rbf(reduce_row(X_DPART, tag64)));
      if (hx == 0) st1_plain(ws + lb + LX_H + ROWS * j + rr, tagged(tag, hn));
      {
        const float ssr = wave_sum(hx == 0 ? hn * hn : 0.f);
        if (lane == 0) st2_plain(ws + lb + LX_HSS + 2 * j, u32x2{__float_as_uint(ssr), tag64});
      }
      MQ_STAMP(layer * 40 + 32);
    }
    BAR();  // F1
  } else {
    // ==================================================================== store wave
    if (lane == 0) {
      s_cnt = 0u;
      s_attst = 0u;
    }
    BAR();  // P00
    BAR();  // P0
    // Every launch writes or clears every exchange word it could ever poll, so that the
    // content a poll can find before the awaited write is at most one launch old, whose
    // tags differ from the polled ones: a split launch clears the attention-output words
    // (read by unsplit launches only), and a workgroup without a chunk partial to store
    // clears its chunk's record (read by split launches with more chunks).
    if (SPLIT && j == 0) st4_plain(ws + lb + LX_ATT + 4 * lane, u32x4{0u, 0u, 0u, 0u});
    if (!SPLIT || !att)
      for (int i = lane; i < 2 * 2 * (int)APART / 4; i += 64)
        st4_plain(ws + lb + LX_PART + 2 * 2 * APART * j + 4 * i, u32x4{0u, 0u, 0u, 0u});
    uint32_t target = 0;
    for (int layer = 0; layer < L; layer++) {
      const uint32_t tag = tag_of(epoch, layer);
      const uint32_t tag64 = epoch * 32u + (uint32_t)layer + 1u;
      BAR();  // A1
      target += NSW;
      wait_count(&s_cnt, target);
      if (lane < 16) st1_plain(ws + lb + LX_QKV + 16 * j + lane, tagged(tag, rbf(s_res[lane])));
      MQ_STAMP(layer * 40 + 34);
      // the next layer's K/V rows into this XCD's L2 ahead of the attention workgroup's
      // LDS copy at its gate/up stage: copying them from HBM there held up its down_proj
      // partials, the last input of the layer's final reduction
      if (!SPLIT && !att && layer + 1 < L) {
        kv_warm(P, layer + 1, g, p, lds_kv, j - 1, WG_PER_XCD - 1, lane);
        // and the attention workgroup's weight rows of its stages after attention
        att_weight_warm(s_lw[layer], s_lw[layer + 1], g, lds_kv, j - 1, WG_PER_XCD - 1, lane);
      }
      // the same for a context split over at most SPLIT_WARM_MAX workgroups (measured: it
      // gains at two and three, and costs from five up, where the copies grow and the
      // workers fall to 27 or fewer)
      if (SPLIT && !att && nsplit <= SPLIT_WARM_MAX && layer + 1 < L) {
        kv_warm(P, layer + 1, g, p, lds_kv, j - nsplit, WG_PER_XCD - nsplit, lane);
        att_weight_warm_n(s_lw[layer], s_lw[layer + 1], g, nsplit, lds_kv, j - nsplit, WG_PER_XCD - nsplit, lane);
      }
      if (att) {
        float M0 = 0.f, M1 = 0.f, L0 = 0.f, L1 = 0.f, Ma0 = 0.f, Ma1 = 0.f, La0 = 0.f, La1 = 0.f;
        for (int ps = 0; ps < npass; ps++) {
          const int ncp = ps ? nc - KV_CAP : nc0;
          BAR();  // B1
          if (own_p && ps == npass - 1) {
            // K/V-cache append at slot p (bf16 [L][8][max_seq][128]): lane -> dims 2 lane, 2 lane + 1
            const size_t slot = ((size_t)(layer * NKV + g) * P.max_seq_len + p) * HD;
            const uint32_t k2 = *reinterpret_cast<const uint32_t*>(s_kv + kv_off(prow, lane >> 2) + 4 * (lane & 3));
            const uint32_t v2 =
                *reinterpret_cast<const uint32_t*>(s_kv + KV_CAP * 256 + kv_off(prow, lane >> 2) + 4 * (lane & 3));
            st1_plain(reinterpret_cast<uint32_t*>(P.k_cache + slot) + lane, k2);
            st1_plain(reinterpret_cast<uint32_t*>(P.v_cache + slot) + lane, v2);
          }
          attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
          BAR();  // B2
          attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
          BAR();  // B3
          attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1);
          BAR();  // B4
          if (ps == 0) {
            Ma0 = M0;
            Ma1 = M1;
            La0 = L0;
            La1 = L1;
          }
        }
        // lane -> outputs 4 lane .. 4 lane + 3 of head hh = lane / 32
        const int hh = lane >> 5, dim = 4 * (lane & 31);
        if (npass == 2) {
          // merge the two passes exactly: rescale both to the larger maximum
#pragma unroll
          for (int h2 = 0; h2 < 2; h2++) {
            const float ma = h2 ? Ma1 : Ma0, mb = h2 ? M1 : M0, mm = fmaxf(ma, mb);
            const float ea = expf(ma - mm), eb = expf(mb - mm);
            if (h2 == hh)
#pragma unroll
              for (int e = 0; e < 4; e++) s_ao[hh][dim + e] = s_ao[hh][dim + e] * ea + s_ao1[hh][dim + e] * eb;
            const float lm2 = (h2 ? La1 : La0) * ea + (h2 ? L1 : L0) * eb;
            if (h2) {
              M1 = mm;
              L1 = lm2;
            } else {
              M0 = mm;
              L0 = lm2;
            }
          }
        }
        if (nsplit == 1) {
          st4_plain(ws + lb + LX_ATT + hh * HD + dim,
                    u32x4{tagged(tag, rbf(s_ao[hh][dim])), tagged(tag, rbf(s_ao[hh][dim + 1])),
                          tagged(tag, rbf(s_ao[hh][dim + 2])), tagged(tag, rbf(s_ao[hh][dim + 3]))});
        } else {
          // chunk partial (m, l, unnormalised acc) as (fp32, tag) pairs; every workgroup of the
          // XCD merges them
          uint32_t* pb = ws + lb + LX_PART + 2 * ((j * 2 + hh) * APART);
          st4_plain(pb + 2 * (2 + dim), u32x4{__float_as_uint(s_ao[hh][dim]), tag64,
                                              __float_as_uint(s_ao[hh][dim + 1]), tag64});
          st4_plain(pb + 2 * (4 + dim), u32x4{__float_as_uint(s_ao[hh][dim + 2]), tag64,
                                              __float_as_uint(s_ao[hh][dim + 3]), tag64});
          if (dim == 0)
            st4_plain(pb, u32x4{__float_as_uint(hh ? M1 : M0), tag64, __float_as_uint(hh ? L1 : L0), tag64});
        }
        // tells the stream waves that this store is ahead of their next weight loads
        if (lane == 0) signal_store(&s_attst);
      }
      MQ_STAMP(layer * 40 + 35);
      // o_proj partials of rows 32j .. 32j+31 over this XCD's two heads
      BAR();  // C1
      target += NSW;
      wait_count(&s_cnt, target);
      if (lane < ROWS)
        st2_dev(ws + X_OPART + 2 * ((j * ROWS + lane) * NXCD + g), u32x2{__float_as_uint(s_res[lane]), tag64});
        MQ_STAMP(layer * 40 + 36);
      // HF Qwen3MLP (modeling_qwen3.py:81-83): m = bf16(bf16(silu(gate)) * up)
      BAR();  // D1
      target += NSW;
      wait_count(&s_cnt, target);
      if (lane < UNITS) {
        const int sw = lane / 3, u = lane - 3 * sw;  // stream wave sw holds gate / up rows 3 sw + u
        const float gt = rbf(s_res[6 * sw + u]), up = rbf(s_res[6 * sw + 3 + u]);
        st1_plain(ws + lb + LX_M + UNITS * j + lane, tagged(tag, rbf(rbf(gt / (1.0f + expf(-gt))) * up)));
      }
      MQ_STAMP(layer * 40 + 37);
      // down_proj partials of rows 32j .. 32j+31 over this XCD's 384 units
      BAR();  // E1
      target += NSW;
      wait_count(&s_cnt, target);
      if (lane < ROWS)
        st2_dev(ws + X_DPART + 2 * ((j * ROWS + lane) * NXCD + g), u32x2{__float_as_uint(s_res[lane]), tag64});
        MQ_STAMP(layer * 40 + 38);
    }
    wait_vmem();  // the warm-up copies have landed before the LM head reuses their LDS
    BAR();  // F1
  }

  // ==================================================================== LM head (all waves)
  MQ_STAMP(32 * 40 + 1);
  if (lm) {
    const u32x4 x0 = x0v[lane], x1 = x0v[64 + lane];
    // rows r0 + NSW * LM_PRE + wave + 8i: four rows per batch, two batches in flight
    auto load_rows = [&](int rb, u32x4 (&Wr)[4][2]) {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = rb + 8 * u;
        if (r < r1) {
          const uint16_t* row = P.lm_head + (size_t)r * H;
          Wr[u][0] = ldw(row + 8 * lane);
          Wr[u][1] = ldw(row + 512 + 8 * lane);
        }
      }
    };
    // bf16 logits of the batch's rows (the four reductions interleaved), best kept with the
    // lowest index on ties (rows are visited in increasing order within a wave)
    auto score_rows = [&](int rb, const u32x4 (&Wr)[4][2]) {
      float d[4];
#pragma unroll
      for (int u = 0; u < 4; u++) d[u] = dot_chunk(Wr[u][0], x0, dot_chunk(Wr[u][1], x1, 0.f));
      wave_sum_n(d);
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = rb + 8 * u;
        if (r < r1) {
          const float v = rbf(d[u]);
          if (lane == 0) s_lg[r - r0] = v;
          if (v > bestv) {
            bestv = v;
            besti = r;
          }
        }
      }
    };
    u32x4 WA[4][2], WB[4][2];
    const int rs = r0 + NSW * LM_PRE + wave;
    load_rows(rs, WA);
    for (int rb = rs; rb < r1; rb += 64) {
      load_rows(rb + 32, WB);
      score_rows(rb, WA);
      load_rows(rb + 64, WA);
      score_rows(rb + 32, WB);
    }
    if (lane == 0) {
      s_bestv[wave] = bestv;
      s_besti[wave] = besti;
    }
  }
  MQ_STAMP(32 * 40 + 2);
  BAR();  // F2
  MQ_STAMP(32 * 40 + 3);
  MQ_STAMP_DUMP();
  if (lm) {
    if (tid == 0) {
      for (int v = 1; v < 8; v++) {
        if (s_bestv[v] > bestv || (s_bestv[v] == bestv && s_besti[v] < besti)) {
          bestv = s_bestv[v];
          besti = s_besti[v];
        }
      }
      wsb.st1(__float_as_uint(bestv), (WS_LMPART + 2 * w) * 4u);
      wsb.st1((uint32_t)besti, (WS_LMPART + 2 * w + 1) * 4u);
    }
    if (P.mode & MODE_LOGITS)
      for (int i = tid; i < r1 - r0; i += NT) P.logits_out[r0 + i] = s_lg[i];
  }

  // ---- completion ticket: the last workgroup reduces and resets the workspace
  wait_vmem();
  BAR();
  if (tid == 0) {
    const uint32_t old =
        __hip_atomic_fetch_add(ws + WS_FINAL_TICKET, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_flag = (old == (uint32_t)(NWG - 1)) ? 1u : 0u;
  }
  BAR();
  if (!s_flag) return;
  int tok = 0;
  if (lm) {
    float v = -INFINITY;
    int i = 0x7fffffff;
    if (tid < NWG) {
      v = __uint_as_float(wsb.ld1((WS_LMPART + 2 * tid) * 4u));
      i = (int)wsb.ld1((WS_LMPART + 2 * tid + 1) * 4u);
    }
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
    BAR();
    float bv = s_bestv[0];
    int bi = s_besti[0];
    for (int q = 1; q < 8; q++) {
      if (s_bestv[q] > bv || (s_bestv[q] == bv && s_besti[q] < bi)) {
        bv = s_bestv[q];
        bi = s_besti[q];
      }
    }
    tok = bi;
  }
  if (tid == 0) {
    const uint32_t err = wsb.ld1(WS_ERR * 4u);
    const int res = err ? -(int)(1u + err) : tok;
    *P.out_token = res;
    if (P.mode & MODE_DEVICE_STEP) {
      // the next launch's input: this token at the next position, with the next epoch (a
      // failed step keeps its position, and its negative token stops the launches after it)
      P.out_ids[step_count] = res;
      *reinterpret_cast<u32x4*>(P.step) =
          u32x4{(uint32_t)res, (uint32_t)(res >= 0 ? p + 1 : p), epoch + 1u, (uint32_t)(step_count + 1)};
    }
    wsb.st1(0u, WS_ERR * 4u);
    wsb.st1(0u, WS_FINAL_TICKET * 4u);
  }
}

// ---------------------------------------------------------------- host side
struct DeviceState {
  bool init = false;
  int status = MQ_OK;
  uint32_t* ws = nullptr;
  // Launches on the device so far. The epoch comes from the host rather than from the
  // workspace: an ordinary launch may start its first workgroups on CUs that the previous
  // launch has already released while that launch's last workgroup is still finishing.
  std::atomic<uint32_t> launches{0};
};
static std::mutex g_mu;
static DeviceState g_dev[64];

// The device can hold all NWG workgroups of both kernel instances at once (no allocation).
static int check_device(int dev) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return MQ_ERR_HIP;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0 || !prop.cooperativeLaunch) return MQ_ERR_DEVICE;
  for (const void* k : {reinterpret_cast<const void*>(mq_decode_kernel<false>),
                        reinterpret_cast<const void*>(mq_decode_kernel<true>)}) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, NT, 0) != hipSuccess) return MQ_ERR_HIP;
    if (per_cu * prop.multiProcessorCount < NWG) return MQ_ERR_DEVICE;
  }
  return MQ_OK;
}

static int ensure_device(int dev) {
  if (dev < 0 || dev >= 64) return MQ_ERR_DEVICE;
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState& d = g_dev[dev];
  if (d.init) return d.status;
  d.init = true;
  if ((d.status = check_device(dev)) != MQ_OK) return d.status;
  void* p = nullptr;
  if (hipMalloc(&p, WS_BYTES) != hipSuccess) return d.status = MQ_ERR_ALLOC;
  if (hipMemset(p, 0, WS_BYTES) != hipSuccess) return d.status = MQ_ERR_HIP;
  if (hipDeviceSynchronize() != hipSuccess) return d.status = MQ_ERR_HIP;
  d.ws = static_cast<uint32_t*>(p);
  return d.status = MQ_OK;
}

static std::atomic<int> g_cooperative{0};

// Workspace of launch_ldg_decode_noalloc: the same layout as the allocated workspace,
// one copy per GPU (in the code object's global memory, zero when the code object is
// loaded), kept until the process ends. Host code never passes `scratch` itself: its
// device address comes from hipGetSymbolAddress, per device.
static __device__ __align__(256) uint32_t scratch[WS_WORDS];

struct NoAllocState {
  bool init = false;
  int status = MQ_OK;
  uint32_t* ptr = nullptr;  // this device's address of `scratch`
};
static NoAllocState g_noalloc[64];

// Set-up of the no-allocation path on device `dev` (current): the device checks and the
// device address of `scratch`, once per device. Allocates nothing.
static int noalloc_workspace(int dev, uint32_t** ws) {
  if (dev < 0 || dev >= 64) return MQ_ERR_DEVICE;
  std::lock_guard<std::mutex> lk(g_mu);
  NoAllocState& d = g_noalloc[dev];
  if (!d.init) {
    d.init = true;
    if ((d.status = check_device(dev)) == MQ_OK) {
      void* p = nullptr;
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
        d.status = MQ_ERR_HIP;
      else
        d.ptr = static_cast<uint32_t*>(p);
    }
  }
  *ws = d.ptr;
  return d.status;
}

// split_instance < 0: chosen from P.position. noalloc: the `scratch` workspace instead of
// the allocated one.
static int launch(DecodeParams& P, hipStream_t stream, int split_instance = -1, bool noalloc = false) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MQ_ERR_HIP;
  if (noalloc) {
    const int st = noalloc_workspace(dev, &P.ws);
    if (st != MQ_OK) return st;
    if (!P.out_token) return MQ_ERR_ARG;
  } else {
    const int st = ensure_device(dev);
    if (st != MQ_OK) return st;
    P.ws = g_dev[dev].ws;
    if (!P.out_token) P.out_token = reinterpret_cast<int*>(g_dev[dev].ws + WS_WORDS);
  }
  if (!(P.mode & MODE_DEVICE_STEP)) P.epoch = g_dev[dev].launches.fetch_add(1u, std::memory_order_relaxed) + 1u;
  // All NWG workgroups must be resident at once. Each one needs a whole CU
  // (its LDS use exceeds half a CU's), ensure_device() checked that the GPU has
  // NWG such slots, and every inter-workgroup wait in the kernel ends in an
  // error after a bounded spin, so an ordinary launch is the default. The
  // cooperative launch (the reference's) is kept as an option, for comparison.
  void* args[] = {&P};
  const bool split = split_instance < 0 ? P.position >= KV_CAP : split_instance != 0;
  const void* kern = split ? reinterpret_cast<const void*>(mq_decode_kernel<true>)
                           : reinterpret_cast<const void*>(mq_decode_kernel<false>);
  const hipError_t e = g_cooperative.load(std::memory_order_relaxed)
                           ? hipLaunchCooperativeKernel(kern, dim3(NWG), dim3(NT), args, 0, stream)
                           : hipLaunchKernel(kern, dim3(NWG), dim3(NT), args, 0, stream);
  return e == hipSuccess ? MQ_OK : MQ_ERR_HIP;
}

// The calling thread's current device's workspace, allocated on first use
// (shared with the prefill kernels, which use word WS_PREFILL_ERR).
int current_workspace(uint32_t** ws) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MQ_ERR_HIP;
  const int st = ensure_device(dev);
  if (st != MQ_OK) return st;
  *ws = g_dev[dev].ws;
  return MQ_OK;
}

static bool bad_scale(float s) { return !(s > 0.f) || !isfinite(s); }

}  // namespace mq

using namespace mq;

// Body of the full-model decode entry points (the reference's unused scratch pointers
// are not passed on).
static int decode_entry(int input_token_id, int* output_token_id, float* logits_output, const void* embed_weight,
                        const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                        const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                        void* v_cache, void* hidden_buffer, void* g_normalized, int num_layers, int position,
                        int cache_len, int max_seq_len, float attn_scale, hipStream_t stream, bool noalloc) {
  if (!output_token_id || !embed_weight || !layer_weights || !final_norm_weight || !lm_head_weight || !cos_table ||
      !sin_table || !k_cache || !v_cache || !hidden_buffer)
    return MQ_ERR_ARG;
  if (num_layers < 1 || num_layers > MAX_LAYERS || max_seq_len < 1 || position < 0 || position >= max_seq_len ||
      position >= MAX_CTX || cache_len != position + 1 || input_token_id < 0 || input_token_id >= VOCAB || bad_scale(attn_scale))
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
  return launch(P, stream, -1, noalloc);
}

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
  return decode_entry(input_token_id, output_token_id, logits_output, embed_weight, layer_weights, final_norm_weight,
                      lm_head_weight, cos_table, sin_table, k_cache, v_cache, hidden_buffer, g_normalized, num_layers,
                      position, cache_len, max_seq_len, attn_scale, stream, false);
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

extern "C" int launch_ldg_decode_noalloc(int input_token_id, int* output_token_id, const void* embed_weight,
                                         const LDGLayerWeights* layer_weights, const void* final_norm_weight,
                                         const void* lm_head_weight, const void* cos_table, const void* sin_table,
                                         void* k_cache, void* v_cache, void* hidden_buffer, void* g_normalized,
                                         int num_layers, int position, int cache_len, int max_seq_len,
                                         float attn_scale, hipStream_t stream) {
  return decode_entry(input_token_id, output_token_id, nullptr, embed_weight, layer_weights, final_norm_weight,
                      lm_head_weight, cos_table, sin_table, k_cache, v_cache, hidden_buffer, g_normalized, num_layers,
                      position, cache_len, max_seq_len, attn_scale, stream, true);
}

extern "C" int mq_decode_layer(const void* hidden_in, void* hidden_out, const LDGLayerWeights* layer_weights,
                               const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
                               int position, int max_seq_len, float attn_scale, hipStream_t stream) {
  if (!hidden_in || !hidden_out || !layer_weights || !cos_table || !sin_table || !k_cache || !v_cache)
    return MQ_ERR_ARG;
  if (max_seq_len < 1 || position < 0 || position >= max_seq_len || position >= MAX_CTX || bad_scale(attn_scale))
    return MQ_ERR_ARG;
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

extern "C" int mq_decode_step_init(MqDecodeStep* step, int token, int position, int capacity, hipStream_t stream) {
  if (!step || token < 0 || token >= VOCAB || position < 0 || position >= MAX_CTX || capacity < 1) return MQ_ERR_ARG;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MQ_ERR_HIP;
  const int st = ensure_device(dev);
  if (st != MQ_OK) return st;
  // the epochs first .. first + capacity - 1 belong to these steps alone
  const uint32_t first = g_dev[dev].launches.fetch_add((uint32_t)capacity, std::memory_order_relaxed) + 1u;
  const MqDecodeStep h{token, position, first, 0};
  return hipMemcpyAsync(step, &h, sizeof(h), hipMemcpyHostToDevice, stream) == hipSuccess &&
                 hipStreamSynchronize(stream) == hipSuccess
             ? MQ_OK
             : MQ_ERR_HIP;
}

extern "C" int mq_decode_step_device(MqDecodeStep* step, int* out_ids, int out_capacity, int split_instance,
                                     const void* embed_weight, const LDGLayerWeights* layer_weights,
                                     const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                                     const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
                                     void* g_normalized, int num_layers, int max_seq_len, float attn_scale,
                                     hipStream_t stream) {
  if (!step || !out_ids || out_capacity < 1 || !embed_weight || !layer_weights || !final_norm_weight ||
      !lm_head_weight || !cos_table || !sin_table || !k_cache || !v_cache || !hidden_buffer)
    return MQ_ERR_ARG;
  if (num_layers < 1 || num_layers > MAX_LAYERS || max_seq_len < 1 || bad_scale(attn_scale) ||
      (split_instance != 0 && split_instance != 1))
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
  P.out_token = nullptr;
  P.num_layers = num_layers;
  P.max_seq_len = max_seq_len;
  P.attn_scale = attn_scale;
  P.mode = MODE_DEVICE_STEP;
  P.step = step;
  P.out_ids = out_ids;
  P.out_capacity = out_capacity;
  return launch(P, stream, split_instance);
}

extern "C" int mq_decode_plan(int position, int* instance, int* nsplit, int* chunk, int* npass) {
  if (position < 0 || position >= MAX_CTX) return MQ_ERR_ARG;
  const int n = position + 1;
  const int ns = plan_nsplit(n), ch = plan_chunk(n);
  if (instance) *instance = position >= KV_CAP ? 1 : 0;
  if (nsplit) *nsplit = ns;
  if (chunk) *chunk = ch;
  if (npass) *npass = (ch + KV_CAP - 1) / KV_CAP;
  return MQ_OK;
}

extern "C" int mq_set_launch_mode(int cooperative) {
  return g_cooperative.exchange(cooperative ? 1 : 0, std::memory_order_relaxed);
}

extern "C" int mq_debug_set_error(int device, unsigned flags) {
  const int st = ensure_device(device);
  if (st != MQ_OK) return st;
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return MQ_ERR_HIP;
  if (hipSetDevice(device) != hipSuccess) return MQ_ERR_HIP;
  hipError_t e = hipMemcpy(g_dev[device].ws + WS_ERR, &flags, sizeof(flags), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (hipSetDevice(cur) != hipSuccess) return MQ_ERR_HIP;
  return e == hipSuccess ? MQ_OK : MQ_ERR_HIP;
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
