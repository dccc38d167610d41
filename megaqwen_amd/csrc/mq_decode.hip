// Persistent decode kernel for Qwen3-0.6B on MI355X (gfx950).
//
// One launch = one greedy decode step of the whole model (embedding, 28
// decoder layers, final norm, tied LM head, argmax), the role of the
// reference's ldg_decode_kernel + ldg_lm_head_phase1/2
// (csrc/megakernel/fused_decode_ldg.cu:617-887).
//
// Chip layout: 256 workgroups of 512 threads, one per CU; workgroup w serves the
// XCD g it runs on (read from the hardware XCC id) as that XCD's member j = w / 8.
// XCD g owns KV group g: the 512 q/k/v rows of query heads 2g, 2g+1 and KV head g,
// the attention of those heads, the o_proj columns of those heads (a K-split of
// o_proj across XCDs) and MLP units 384g .. 384g+383 (a K-split of down_proj).
//
// The 32 workgroups of an XCD form two groups of 16 that take turns on the critical
// path of a layer:
//   group A (members 0..15): input RMSNorm, q/k/v rows 32a .. 32a+31 of the group's
//     [q0; q1; k; v], the attention (contexts of at most 256 positions: every member
//     attends over the whole context, so the output needs no hand-out; longer ones:
//     members a < nsplit each attend over one chunk), o_proj partial sums of rows
//     64a .. 64a+63 over the group's 256
//     columns, and the cross-XCD reduction of those rows into h1;
//   group B (members 16..31, b = j - 16): post-attention RMSNorm, gate and up rows of
//     units 384g + 24b .. +23, down_proj partial sums of rows 64b .. 64b+63 over the
//     XCD's 384 units, and the cross-XCD reduction of those rows into h.
// While one group works, the other streams its next layer's weights into registers
// (and the attention workgroups their next K/V rows into LDS): a CU's loads and its
// exchange polls complete in order, so a group only ever polls with no weight load
// in flight. Each group issues its burst as soon as its reduce wave has stored its
// rows, so that the burst has landed before the other group's cross-XCD reduction.
//
// Every workgroup runs four roles, one per wave kind:
//   * stream waves 0-3 hold the group's weight slice in registers, compute the dot
//     products and store them (a wave's rows regrouped through its own LDS slots);
//   * poll waves 4-5 gather the XCD-local exchanges (h, q/k/v, attention output,
//     h1, m), normalise, apply QK-norm and RoPE, and merge attention chunks;
//   * reduce wave 6 sums the eight XCDs' partials of the workgroup's 64 residual
//     rows and applies the residual add;
//   * store wave 7 appends the new K/V row, stores the attention output and the
//     stage cues, and clears the words a launch does not write.
// A layer has five XCD-local all-gathers and two cross-XCD reductions and no grid
// barrier. The kernel has three instances: SPLIT = false for contexts of at most 256
// positions (one attention workgroup per XCD, no chunk merge compiled in), SPLIT = true
// for the rest (up to 16 chunks of up to four 256-position LDS passes), and its PIPE
// variant, which overlaps the later passes' K/V copies with the previous pass (used
// where a chunk takes more than one pass: past 4096 positions).
//
// Exchanges use "tagged words": a bf16 value in the low half of a 32-bit word
// and a 16-bit tag (launch epoch x 32 + layer) in the high half, or an fp32
// value with a 32-bit tag in a 64-bit word. A consumer issues all its loads at
// once, keeps two such poll rounds in flight (half a round trip apart) and keeps
// each word from the first round that returns it with the expected tag, so an
// exchange costs about one memory round trip after the producer's store. Across
// XCDs both sides use device-scope (sc1) accesses; inside an XCD
// producers use plain stores and consumers non-temporal loads, served by the
// XCD's shared L2. A watchdog bounds every poll and turns a lost producer into an
// error code instead of a hang.
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
// (slot = layer * 40 + event; stream events 0..11, poll 12..27, reduce 28..32,
// store 34..38; slots 32 * 40 .. +3 the final norm and LM head, + 4 the kernel's entry;
// a workgroup keeps its
// own slots, so group A's attention reuses 21..23, which only group B writes otherwise),
// MQ_STAMP_DUMP()
// runs once at the end of the kernel. Both compile to nothing unless a tracing build
// (csrc/trace/mq_decode_trace.cpp) defines them before including this file.
#ifdef MQ_STAMP
#define MQ_TRACE_BUILD 1
#else
#define MQ_STAMP(i) ((void)0)
#endif
#ifndef MQ_STAMP_DUMP
#define MQ_STAMP_DUMP() ((void)0)
#endif
// MQ_STAMP_AFTER(slot, v) stamps once the value v is available (a load has returned).
#ifndef MQ_STAMP_AFTER
#define MQ_STAMP_AFTER(i, v) ((void)0)
#endif
// MQ_LANDED(slot) stamps once the wave's outstanding loads have landed (a tracing build only)
#ifndef MQ_LANDED
#define MQ_LANDED(i) ((void)0)
#endif
// MQ_VALUE(slot, v) records the value v in a slot instead of a time (a tracing build only)
#ifndef MQ_VALUE
#define MQ_VALUE(i, v) ((void)0)
#endif

namespace mq {

constexpr int NWG = 256;
constexpr int NT = 512;
constexpr int NSW = 4;  // stream waves 0..3
constexpr int NPW = 2;  // poll waves 4..5; wave 6 reduces the cross-XCD partial sums, wave 7 stores
constexpr int NXCD = 8;
constexpr int WG_PER_XCD = NWG / NXCD;  // 32
constexpr int NGA = 16;                  // group-A workgroups per XCD
constexpr int NGB = WG_PER_XCD - NGA;    // group-B workgroups per XCD
constexpr int ROWS = H / NGA;            // residual rows a workgroup reduces: 64 (A: h1, B: h)
static_assert(H / NGB == ROWS, "both groups reduce the same number of rows");
constexpr int QROWS = 4 * HD / NGA;      // q/k/v rows per A workgroup: 32
constexpr int XUNITS = I / NXCD;         // MLP units per XCD: 384
constexpr int UNITS = XUNITS / NGB;      // MLP units per B workgroup: 24
constexpr int KV_CAP = 256;              // positions per LDS pass of an attention workgroup
constexpr int MAX_PASS = 4;              // LDS passes per attention workgroup
constexpr int MAX_CTX = NGA * MAX_PASS * KV_CAP;  // 16384

// Attention split of a context of n positions (the query at n - 1): nsplit chunks of at
// most `chunk` positions, chunk a on A workgroup (g, a) of every XCD g, each attended in
// passes of at most KV_CAP positions (the LDS copy holds KV_CAP rows).
__host__ __device__ constexpr int plan_nsplit(int n) {
  return (n + KV_CAP - 1) / KV_CAP < NGA ? (n + KV_CAP - 1) / KV_CAP : NGA;
}
__host__ __device__ constexpr int plan_chunk(int n) { return (n + plan_nsplit(n) - 1) / plan_nsplit(n); }
// Every context length the kernel accepts (1 .. MAX_CTX) gives chunks of at most MAX_PASS
// LDS passes, none of them empty, covering all n positions.
constexpr bool plan_is_sound() {
  for (int n = 1; n <= MAX_CTX; n++) {
    const int ns = plan_nsplit(n), ch = plan_chunk(n);
    if (ns < 1 || ns > NGA || ch > MAX_PASS * KV_CAP || ch * ns < n || (ns - 1) * ch >= n) return false;
  }
  return true;
}
static_assert(plan_is_sound(), "attention chunks must fit MAX_PASS LDS passes and cover the context");
// Kernel instance for the query at `position`: 0 (one attention workgroup per XCD, one
// pass) below KV_CAP, 2 (passes pipelined) where a chunk takes more than one LDS pass,
// else 1.
__host__ __device__ constexpr int plan_instance(int position) {
  return position < KV_CAP ? 0 : plan_chunk(position + 1) > KV_CAP ? 2 : 1;
}

// Workspace layout, in 32-bit words.
constexpr uint32_t WS_RESERVED = 0;  // (words 0..31 unused)
constexpr uint32_t WS_ERR = 32;
constexpr uint32_t WS_FINAL_TICKET = 64;
// word WS_PREFILL_ERR (96) belongs to the prefill kernels
// The epoch of the workspace's last completed launch: a launch tags its exchanges with this
// value + 1 and its last workgroup stores that back, so consecutive launches on one workspace
// differ by exactly one epoch whichever entry point makes them (host-driven and
// device-resident launches share the allocated workspace and its count; the no-allocation
// entry point's workspace keeps its own).
constexpr uint32_t WS_EPOCH = 128;
// per-XCD regions of tagged words, written and read only by that XCD's workgroups
constexpr uint32_t WS_LOCAL = 1024;
constexpr uint32_t LOCAL_WORDS = 32768;
constexpr uint32_t LX_H = 0;        // [1024] residual stream after the layer (from B)
constexpr uint32_t LX_H1 = 1024;    // [1024] residual stream after attention (from A)
constexpr uint32_t LX_QKV = 2048;   // [512]  raw q0, q1, k, v rows of the XCD's KV group
constexpr uint32_t LX_ATT = 2560;   // [256]  attention output of the two query heads (split, one chunk)
constexpr uint32_t LX_M = 2816;     // [384]  SiLU(gate) * up of the XCD's MLP units
// cue words (a 16-bit tag each): group A member 0 writes LX_CUE_A after its o_proj
// partials, group B member 0 writes LX_CUE_B after its down_proj partials. The other group
// watches the cue (one word) before it polls the residual stream (2 KB a wave), which
// keeps the long waits off the XCD's L2; the gathered data carry their own tags.
constexpr uint32_t LX_CUE_A = 3200;
constexpr uint32_t LX_CUE_B = 3232;
constexpr uint32_t APART = 130;     // attention partial of one head: m, l, acc[128]
constexpr uint32_t LX_PART = 4096;  // [16 chunks][2 heads][APART] (fp32, tag) pairs
// cross-XCD partial sums: [member][xcd][row] (fp32, tag) pairs
constexpr uint32_t X_OPART = WS_LOCAL + NXCD * LOCAL_WORDS;
constexpr uint32_t X_DPART = X_OPART + 2 * NGA * ROWS * NXCD;
constexpr uint32_t WS_LMPART = X_DPART + 2 * NGB * ROWS * NXCD;  // [NWG][2]: best logit, index
constexpr uint32_t WS_WORDS = WS_LMPART + NWG * 2;
constexpr size_t WS_BYTES = ((WS_WORDS * 4 + 4 + 65535) / 65536) * 65536;
static_assert(LX_PART + 2 * NGA * 2 * APART <= LOCAL_WORDS, "per-XCD region overflow");

constexpr uint32_t POLL_LIMIT = 1u << 21;  // ~1 s of polling before the watchdog fires
// Exchange polls keep two rounds of loads in flight, the second issued this many s_sleep
// units (64 clocks each) after the first; a poll round then returns about every half round
// trip instead of every round trip, which shortens the time from a producer's store to the
// consumer seeing it.
constexpr int POLL_STAGGER = 4;
// From this many context positions on (in the unsplit instance) group B's reduce waves
// also sum the o_proj partials into h1, so that group A streams its next weights and K/V
// rows right after its o_proj partials: its burst, which grows with the K/V rows, then lands
// before the layer ends instead of holding up its own gather of h (CU loads complete in
// order). Shorter contexts keep the reduction in group A, whose short burst would otherwise
// overlap that cross-XCD reduction. Measured crossover: 128 positions, where the attention
// takes a second 16-row score block per wave and a second P.V trip (same box, group A summing
// against group B: p120 288.7 against 294.8 us, p128 295.0 against 293.4, p144 298.5 against
// 293.8).
constexpr int B_H1_MIN_CTX = 129;
constexpr uint32_t ERR_POLL = 1u;
constexpr uint32_t ERR_XCD = 2u;  // a workgroup ran on an XCD numbered 8 or above
constexpr uint32_t ERR_STEP = 4u;  // a device-resident step found an invalid token, position or count

constexpr int NT_LD = 2;  // non-temporal cache policy: bypasses the CU's L1, served by the XCD's L2

// The first LM_KV_ROWS LM-head rows of a workgroup are copied into its K/V LDS array before the LM
// head (group A after its last layer's o_proj partials, group B a few a layer in its quiet
// windows, in the instance where its array is otherwise unused), behind the first LM_OFF bytes,
// which hold the workgroup's logits; the LM-head loop reads them from LDS.
constexpr int LM_KV_ROWS = 62;
constexpr uint32_t LM_OFF = 4096;
// and, in the split instance without the pipelined passes (where only group A copies rows), the
// next LM_X_ROWS rows into an LDS array of their own, in what the kernel's other arrays leave of
// the CU's 160 KB (less in the tracing build, whose stamps sit in LDS). Measured (same box):
// p1024 330.6 -> 329.3 us, p3000 374.1 -> 371.4 in this instance; p200 288.3 -> 289.1 and
// p8192 551.6 -> 551.9 in the other two, which keep LM_KV_ROWS
#ifdef MQ_TRACE_BUILD
constexpr int LM_X_ROWS = 4;
#else
constexpr int LM_X_ROWS = 7;
#endif
constexpr int LM_ROWS = LM_KV_ROWS + LM_X_ROWS;


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
  // MODE_DEVICE_STEP: token and position come from *step (advanced by the launch's last
  // workgroup), and each launch's token is appended to out_ids[step->count]
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

// ---- XCD-local exchange: plain stores, non-temporal loads (served by the XCD's L2)
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
// One 16-byte chunk of tagged words with two poll rounds in flight (as in reduce_row8).
__device__ __forceinline__ u32x4 poll2_l4(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag) {
  u32x4 r[2], v = u32x4{0u, 0u, 0u, 0u};
  bool have = false;
  r[0] = ldl4(b, word);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_sleep(POLL_STAGGER);
  r[1] = ldl4(b, word);
  asm volatile("" ::: "memory");
  auto merge = [&](const u32x4& x) {
    if (!have && tags_ok(x, tag)) {
      v = x;
      have = true;
    }
    return __all(have);
  };
#define MQ_MSTEP(k)                   \
  if (merge(r[(k) % 2])) return v;    \
  r[(k) % 2] = ldl4(b, word);         \
  asm volatile("" ::: "memory");
  MQ_MSTEP(0) MQ_MSTEP(1) MQ_MSTEP(2) MQ_MSTEP(3) MQ_MSTEP(4) MQ_MSTEP(5)
  MQ_MSTEP(6) MQ_MSTEP(7) MQ_MSTEP(8) MQ_MSTEP(9) MQ_MSTEP(10) MQ_MSTEP(11)
#undef MQ_MSTEP
  merge(r[0]);
  merge(r[1]);
  uint32_t spins = 0;
  while (!have) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    const u32x4 x = ldl4(b, word);
    if (tags_ok(x, tag)) {
      v = x;
      have = true;
    }
  }
  return v;
}

// K/V rows of a chunk live in LDS as [row][16 chunks of 8 dims], chunk c of row r
// stored in slot c ^ (r & 15) so that 16 rows read at one chunk hit distinct banks.
__device__ __forceinline__ uint32_t kv_off(int row, int chunk) { return row * 256 + 16 * (chunk ^ (row & 15)); }
// V rows use their own swizzle, chunk c of row r in slot c ^ vsw(r): P.V's transpose reads
// take 16 rows (8 kg + i of a 32-row block, i < 4) by one 32-byte chunk pair each, and vsw
// (bits 1..3 = r % 4 and bit 3 of r) spreads those 16 rows evenly over the 8 pair slots.
__device__ __forceinline__ int vsw(int row) { return 2 * ((row & 3) | (((row >> 3) & 1) << 2)); }
__device__ __forceinline__ uint32_t vkv_off(int row, int chunk) { return row * 256 + 16 * (chunk ^ vsw(row)); }

// Stream wave s copies K and V rows [0, nc) of the chunk starting at position c0
// (except position p, which the layer itself produces) into LDS (WHAT: 1 the K rows,
// 2 the V rows, 3 both); nt picks the non-temporal cache policy.
template <int WHAT = 3>
__device__ __forceinline__ void kv_dma(bool nt, const DecodeParams& P, int layer, int g, int c0, int nc, int p, uint32_t lds,
                                       int s, int lane) {
  const size_t base = ((size_t)(layer * NKV + g) * P.max_seq_len + c0) * HD;
  const uint16_t* kb = P.k_cache + base;
  const uint16_t* vb = P.v_cache + base;
  const int nq = (nc + 3) >> 2;  // one instruction moves 4 rows
  const int rin = lane >> 4, slot = lane & 15;
  for (int q = s; q < nq; q += NSW) {
    const int row = 4 * q + rin;
    if (row < nc && c0 + row != p) {
      if (nt) {
        if constexpr ((WHAT & 1) != 0) dma16_nt(kb + row * HD + 8 * (slot ^ (row & 15)), lds + q * 1024);
        if constexpr ((WHAT & 2) != 0) dma16_nt(vb + row * HD + 8 * (slot ^ vsw(row)), lds + KV_CAP * 256 + q * 1024);
      } else {
        if constexpr ((WHAT & 1) != 0) dma16(kb + row * HD + 8 * (slot ^ (row & 15)), lds + q * 1024);
        if constexpr ((WHAT & 2) != 0) dma16(vb + row * HD + 8 * (slot ^ vsw(row)), lds + KV_CAP * 256 + q * 1024);
      }
    }
  }
}

// ---- exchange stores: inline assembly, so that the compiler's vmcnt bookkeeping for
// the stream waves' register loads ignores them (each makes a later wait at most one
// instruction longer). The stream waves store their dot products (q/k/v rows, o_proj and
// down_proj partials, m) as soon as they have them, before their next weight burst; the
// reduce waves store after their last poll of the stage, so no poll queues behind a
// store's write acknowledgement. `dev` stores (sc1) write through to memory for readers
// on other XCDs; plain stores stay in this XCD's L2.
__device__ __forceinline__ void st2_dev(uint32_t* p, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st2_plain(uint32_t* p, u32x2 v) {
  asm volatile("global_store_dwordx2 %0, %1, off" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void st1_plain(uint32_t* p, uint32_t v) {
  asm volatile("global_store_dword %0, %1, off" ::"v"(p), "v"(v) : "memory");
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
// of 16 rows: wave v takes row blocks v and v + 8, NB of them (the blocks that hold a row
// below nc; the others are neither read nor written: no later phase reads s_sc past nc).
// Returns the wave's maximum of its scores per head (lanes 0 and 1: heads 0 and 1).
template <int NB>
__device__ __forceinline__ float attn_score_blocks(const uint8_t* s_kv, const uint16_t* s_q, float (*s_sc)[KV_CAP],
                                                   int nc, float scale, int v, int lane) {
  const int r16 = lane & 15, kg = lane >> 4;
  u32x4 qb[4];
#pragma unroll
  for (int s4 = 0; s4 < 4; s4++) {
    const u32x4 t = *reinterpret_cast<const u32x4*>(s_q + (r16 & 1) * HD + 32 * s4 + 8 * kg);
    qb[s4] = r16 < 2 ? t : u32x4{0u, 0u, 0u, 0u};
  }
  // the blocks' K operands are all read before the MFMA chains run
  float mx = -INFINITY;
  u32x4 ka[NB][4];
#pragma unroll
  for (int bi = 0; bi < NB; bi++)
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++)
      ka[bi][s4] = *reinterpret_cast<const u32x4*>(s_kv + kv_off(16 * (v + 8 * bi) + r16, 4 * s4 + kg));
  f32x4 acc[NB];
#pragma unroll
  for (int bi = 0; bi < NB; bi++) acc[bi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
    for (int bi = 0; bi < NB; bi++) acc[bi] = mfma_16x16x32(ka[bi][s4], qb[s4], acc[bi]);
  // lane (column r16 = head, rows 4kg + e): one 16-byte write of its four scores per block
#pragma unroll
  for (int bi = 0; bi < NB; bi++) {
    const int r = 16 * (v + 8 * bi) + 4 * kg;
    f32x4 val;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      val[e] = r + e < nc ? acc[bi][e] * scale : -INFINITY;
      mx = fmaxf(mx, val[e]);
    }
    if (r16 < 2) *reinterpret_cast<f32x4*>(&s_sc[r16][r]) = val;
  }
  return mx;
}
// Scores of wave v's blocks (see attn_score_blocks); leaves the wave's per-head maxima in s_mx[v].
__device__ __forceinline__ void attn_scores(const uint8_t* s_kv, const uint16_t* s_q, float (*s_sc)[KV_CAP],
                                            float (*s_mx)[2], int nc, float scale, int v, int lane) {
  const int nb16 = (nc + 15) >> 4;  // 16-row blocks that hold a row below nc
  float mx = v + 8 < nb16 ? attn_score_blocks<2>(s_kv, s_q, s_sc, nc, scale, v, lane)
             : v < nb16   ? attn_score_blocks<1>(s_kv, s_q, s_sc, nc, scale, v, lane)
                          : -INFINITY;
  // per-head maximum over the lanes of column 0 (head 0) and column 1 (head 1): lane groups
  // kg meet through permlane swaps; lanes 0 and 1 hold the two heads' maxima
  {
    const auto a2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = fmaxf(__uint_as_float(a2[0]), __uint_as_float(a2[1]));
    const auto b2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = fmaxf(__uint_as_float(b2[0]), __uint_as_float(b2[1]));
  }
  if (lane < 2) s_mx[v][lane] = mx;
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
  // rows 0 + 1 (head 0) and 2 + 3 (head 1) of the 16-lane sums, as readlane pairs would add
  // them; lanes 0 and 32 hold the two heads' sums
  float t = row16_sum(e);
  {
    const auto b2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(t), __float_as_uint(t), false, false);
    t = __uint_as_float(b2[0]) + __uint_as_float(b2[1]);
  }
  if ((lane & 31) == 0) s_l[v][lane >> 5] = t;
}

// acc[h][d] = sum_r bf16(p_h[r]) * v_r[d] for this wave's 16 dims d = 16v + (lane & 15)
// over the 32-row blocks that hold rows < nc (rows past nc have p = 0 and finite V).
// The MFMA operand (8 rows of one dim per lane) comes from two LDS transpose reads:
// within each 16-lane group, lane j addresses row base + j / 4, dims 4 (j % 4) .. +3 of
// the wave's 16, and lane i receives that column's 4 rows (ds_read_b64_tr_b16).
// Writes acc / l (fin) or the raw acc (a split-K partial) to s_ao, or with out16 the
// bf16-rounded acc / l to out16[h * 128 + d] (the o_proj input), and returns the per-head
// sums l (the waves' sums s_l[k][h], k = 0..7, added in order).
__device__ __forceinline__ void attn_pv(const uint8_t* s_kv, const uint16_t* s_p, const float (*s_l)[2],
                                        float (*s_ao)[HD], int nc, int v, int lane, bool fin, float& L0, float& L1,
                                        uint16_t* out16 = nullptr) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  const int r16 = lane & 15, kg = lane >> 4;
  const int dim = 16 * v + r16;
  const int dq = 16 * v + 4 * (r16 & 3);                // this lane's 4 dims in the transpose reads
  const uint32_t vb0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)(s_kv + KV_CAP * 256);
  // the softmax sums as four 16-byte reads (s_l[2i], s_l[2i + 1] in each), ahead of the products
  const f32x4* sl = reinterpret_cast<const f32x4*>(&s_l[0][0]);
  const f32x4 l01 = sl[0], l23 = sl[1], l45 = sl[2], l67 = sl[3];
  L0 = 0.f + l01[0] + l01[2] + l23[0] + l23[2] + l45[0] + l45[2] + l67[0] + l67[2];
  L1 = 0.f + l01[1] + l01[3] + l23[1] + l23[3] + l45[1] + l45[3] + l67[1] + l67[3];
  // 32-row blocks in pairs with two accumulators (a block past nc has p = 0: rows < 256
  // always lie in the LDS copy and hold finite values)
  const int nb = (nc + 31) >> 5;
  f32x4 acc2[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  // four blocks a trip (all their LDS reads issued together), block t0 + bi into
  // accumulator bi % 2 as in a two-block loop; blocks past nb have p = 0
  for (int t0 = 0; t0 < nb; t0 += 4) {
    u32x4 pa[4], vb[4];
#pragma unroll
    for (int bi = 0; bi < 4; bi++) {
      const int rr = 32 * (t0 + bi) + 8 * kg;
      const u32x4 pt = *reinterpret_cast<const u32x4*>(s_p + (r16 & 1) * KV_CAP + rr);
      pa[bi] = r16 < 2 ? pt : u32x4{0u, 0u, 0u, 0u};
      const int ra = rr + (r16 >> 2), rb = ra + 4;
      const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_v4s*)(uintptr_t)(vb0 + vkv_off(ra, dq >> 3) + 2 * (dq & 7)));
      const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_v4s*)(uintptr_t)(vb0 + vkv_off(rb, dq >> 3) + 2 * (dq & 7)));
      const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
      vb[bi] = u32x4{l2.x, l2.y, h2.x, h2.y};
    }
    acc2[0] = mfma_16x16x32(pa[0], vb[0], acc2[0]);
    acc2[1] = mfma_16x16x32(pa[1], vb[1], acc2[1]);
    acc2[0] = mfma_16x16x32(pa[2], vb[2], acc2[0]);
    acc2[1] = mfma_16x16x32(pa[3], vb[3], acc2[1]);
  }
  const f32x4 acc = acc2[0] + acc2[1];
  if (kg == 0) {
    if (out16) {
      out16[dim] = (uint16_t)f2bf(acc[0] * (1.0f / L0));
      out16[HD + dim] = (uint16_t)f2bf(acc[1] * (1.0f / L1));
    } else {
      s_ao[0][dim] = fin ? acc[0] * (1.0f / L0) : acc[0];
      s_ao[1][dim] = fin ? acc[1] * (1.0f / L1) : acc[1];
    }
  }
}

// Stream-wave weight registers: group A holds a layer's q/k/v rows and o_proj partial rows,
// group B its gate/up rows and down_proj partial rows.
struct ARegs {
  u32x4 a[16];   // q/k/v: 8 rows x 2 chunks
  u32x4 o[8];    // o_proj partials: 16 rows as 8 pairs of rows, one chunk per lane
  u32x2 wln;     // input_layernorm elements 4t .. 4t+3
  uint32_t qkn;  // q_norm (t < 64) / k_norm (t >= 64) elements 2t, 2t+1 (mod 128)
};
struct BRegs {
  u32x4 gu[24];  // gate rows of 6 units, then their up rows: 12 rows x 2 chunks
  u32x4 d[16];   // down_proj partials: 16 rows, one chunk per lane (lanes < 48)
  u32x2 wpost;   // post_attention_layernorm elements 4t .. 4t+3
};

// Exchange waves: one 16-byte chunk (4 tagged words) as fp32 values.
__device__ __forceinline__ void unpack_tagged(const u32x4& v, float* f) {
  f[0] = bflo(v.x);
  f[1] = bflo(v.y);
  f[2] = bflo(v.z);
  f[3] = bflo(v.w);
}

// Wait until the cue word carries `tag` (all lanes load the same word: one request).
__device__ __forceinline__ void wait_cue(const Buf& b, uint32_t* ws, uint32_t word, uint32_t tag) {
  uint32_t v = ldl1(b, word), spins = 0;
  while (v != tag) {
    if (watchdog(b, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(2);
    v = ldl1(b, word);
  }
}

// This poll wave's half of a gathered residual stream (chunks lane + 128c into v0 and
// lane + 128c + 64 into v1) and the stream's sum of squares: each poll wave adds up the
// squares of its half, and the two halves' sums meet in LDS and are added in a fixed
// order (half 0 first), so both waves' norms agree bit for bit. `target` is the number
// of half sums the LDS counter holds once this exchange is complete.
__device__ __forceinline__ float gather_half(const Buf& b, uint32_t* ws, uint32_t base, uint32_t tag, int c, int lane,
                                             u32x4& v0, u32x4& v1, float* s_ssx, uint32_t* s_ssn, uint32_t target,
                                             int sk = 0) {
  const uint32_t w0 = base + 4 * (lane + 128 * c), w1 = w0 + 4 * 64;
  // two poll rounds in flight (as in reduce_row8): round k % 2 is checked while the other
  // is outstanding, then re-issued; a chunk is kept once a round returns it with the tag
  u32x4 a = u32x4{0u, 0u, 0u, 0u}, e = a;
  bool ha = false, he = false;
  u32x4 ra[2], re[2];
  ra[0] = ldl4(b, w0);
  re[0] = ldl4(b, w1);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_sleep(POLL_STAGGER);
  ra[1] = ldl4(b, w0);
  re[1] = ldl4(b, w1);
  asm volatile("" ::: "memory");
  MQ_STAMP_AFTER(sk, ra[0].x + re[0].x);
  auto merge = [&](const u32x4& x0, const u32x4& x1) {
    if (!ha && tags_ok(x0, tag)) {
      a = x0;
      ha = true;
    }
    if (!he && tags_ok(x1, tag)) {
      e = x1;
      he = true;
    }
    return __all(ha & he);
  };
#define MQ_GSTEP(k)                                  \
  if (merge(ra[(k) % 2], re[(k) % 2])) goto gathered; \
  ra[(k) % 2] = ldl4(b, w0);                         \
  re[(k) % 2] = ldl4(b, w1);                         \
  asm volatile("" ::: "memory");
  MQ_GSTEP(0) MQ_GSTEP(1) MQ_GSTEP(2) MQ_GSTEP(3) MQ_GSTEP(4) MQ_GSTEP(5)
  MQ_GSTEP(6) MQ_GSTEP(7) MQ_GSTEP(8) MQ_GSTEP(9) MQ_GSTEP(10) MQ_GSTEP(11)
#undef MQ_GSTEP
  merge(ra[0], re[0]);
  merge(ra[1], re[1]);
  {
    uint32_t spins = 0;
    while (!(ha & he)) {
      if (watchdog(b, ws, ++spins)) break;
      __builtin_amdgcn_s_sleep(1);
      if (!ha) {
        const u32x4 v = ldl4(b, w0);
        if (tags_ok(v, tag)) {
          a = v;
          ha = true;
        }
      }
      if (!he) {
        const u32x4 v = ldl4(b, w1);
        if (tags_ok(v, tag)) {
          e = v;
          he = true;
        }
      }
    }
  }
gathered:
  v0 = a;
  v1 = e;
  float fa[4], fe[4];
  unpack_tagged(a, fa);
  unpack_tagged(e, fe);
  const float part = wave_sum(((fa[0] * fa[0] + fa[1] * fa[1]) + (fa[2] * fa[2] + fa[3] * fa[3])) +
                              ((fe[0] * fe[0] + fe[1] * fe[1]) + (fe[2] * fe[2] + fe[3] * fe[3])));
  if (lane == 0) {
    s_ssx[c] = part;
    signal_store(s_ssn);
  }
  wait_count(s_ssn, target);
  return s_ssx[0] + s_ssx[1];
}

// HF Qwen3RMSNorm (modeling_qwen3.py:59-64) of one chunk: y = bf16(w * bf16(x * rstd)),
// written as two bf16 pairs.
__device__ __forceinline__ void norm_chunk(const float* x, float rstd, uint32_t w0, uint32_t w1, uint32_t* dst) {
  float a = x[0] * rstd, b = x[1] * rstd, c = x[2] * rstd, d = x[3] * rstd;
  rbf2(a, b);
  rbf2(c, d);
  dst[0] = pack_bf2(bflo(w0) * a, bfhi(w0) * b);
  dst[1] = pack_bf2(bflo(w1) * c, bfhi(w1) * d);
}

// Waits until this XCD's own partial of the workgroup's first row carries tag64 (all lanes on
// one word: one request a poll), before the eight-XCD poll of reduce_row8 starts, where the
// partial comes from another workgroup (group B summing group A's o_proj partials). The other
// XCDs' partials are stored at about the same time, so the reduction ends as it would, while
// the reduce waves' device-scope polls, 4 KB a round per wave otherwise, no longer load the
// memory system through the long wait before the partials exist. (Where the workgroup's own
// stream waves produce the partials, the reduce wave waits for their LDS signals instead.)
__device__ __forceinline__ void wait_own_part(const Buf& wsb, uint32_t* ws, uint32_t word, uint32_t tag64) {
  uint32_t v = wsb.ld1(word * 4u), spins = 0;
  while (v != tag64) {
    if (watchdog(wsb, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
    v = wsb.ld1(word * 4u);
  }
}

// Sum of the eight XCDs' (fp32, tag) partials of one row, in XCD order, from the
// cross-XCD array at `part` (pairs [member][xcd][row], so that each producer writes, and
// each of the consumer's loads reads, one contiguous 512-byte run): lane = row.
__device__ __forceinline__ float reduce_row8(const Buf& wsb, uint32_t* ws, uint32_t wd, uint32_t tag64) {
  auto ok = [&](const u32x2& v) { return v.y == tag64; };
  uint32_t spins = 0;
  u32x2 q[NXCD];
  // Two poll rounds in flight: the older round is checked while the other is still
  // outstanding, then re-issued; a pair is kept once a round returns it with the expected
  // tag. The rounds are unrolled (no loop-carried loads, so the compiler's waits stay exact),
  // the compiler barriers keep each round's loads where they are issued, and the exit tests
  // are wave-uniform; past the unrolled rounds the single-round loop takes over.
  constexpr int NR = 2;
  u32x2 r[NR][NXCD];
  bool have[NXCD];
#pragma unroll
  for (int x = 0; x < NXCD; x++) {
    have[x] = false;
    q[x] = u32x2{0u, 0u};
  }
#pragma unroll
  for (int k = 0; k < NR; k++) {
    if (k) __builtin_amdgcn_s_sleep(POLL_STAGGER);
#pragma unroll
    for (int x = 0; x < NXCD; x++) r[k][x] = wsb.ld2((wd + 2 * ROWS * x) * 4u);
    asm volatile("" ::: "memory");
  }
  auto merge = [&](const u32x2 (&v)[NXCD]) {
    bool all = true;
#pragma unroll
    for (int x = 0; x < NXCD; x++) {
      if (!have[x] && ok(v[x])) {
        q[x] = v[x];
        have[x] = true;
      }
      all &= have[x];
    }
    return __all(all);
  };
  auto reissue = [&](u32x2 (&v)[NXCD]) {
#pragma unroll
    for (int x = 0; x < NXCD; x++) v[x] = wsb.ld2((wd + 2 * ROWS * x) * 4u);
    asm volatile("" ::: "memory");
  };
  // the oldest round is r[k % NR] at step k
#define MQ_RSTEP(k)                          \
  if (merge(r[(k) % NR])) goto reduced;      \
  reissue(r[(k) % NR]);
  MQ_RSTEP(0) MQ_RSTEP(1) MQ_RSTEP(2) MQ_RSTEP(3) MQ_RSTEP(4) MQ_RSTEP(5)
  MQ_RSTEP(6) MQ_RSTEP(7) MQ_RSTEP(8) MQ_RSTEP(9) MQ_RSTEP(10) MQ_RSTEP(11)
#undef MQ_RSTEP
  {
    // the pairs not yet kept, one round at a time
#pragma unroll
    for (int k = 0; k < NR; k++) merge(r[k]);
    for (;;) {
      bool all = true;
#pragma unroll
      for (int x = 0; x < NXCD; x++) all &= have[x];
      if (all || watchdog(wsb, ws, ++spins)) break;
      __builtin_amdgcn_s_sleep(1);
#pragma unroll
      for (int x = 0; x < NXCD; x++)
        if (!have[x]) {
          const u32x2 v = wsb.ld2((wd + 2 * ROWS * x) * 4u);
          if (ok(v)) {
            q[x] = v;
            have[x] = true;
          }
        }
    }
  }
reduced:
  auto f = [&](int x) { return __uint_as_float(q[x].x); };
  return ((f(0) + f(1)) + (f(2) + f(3))) + ((f(4) + f(5)) + (f(6) + f(7)));
}

// Polls N tagged words (word w[i] + lane) of the XCD's exchange region until all carry `tag`.
template <bool PIPE, int N>
__device__ __forceinline__ void poll_words(const Buf& wsb, uint32_t* ws, const uint32_t (&w)[N], uint32_t tag,
                                           uint32_t (&u)[N]) {
  if (PIPE) {
  // two poll rounds in flight (as in reduce_row8)
  uint32_t r[2][N];
  bool have[N];
#pragma unroll
  for (int i = 0; i < N; i++) {
    have[i] = false;
    u[i] = 0u;
    r[0][i] = ldl1(wsb, w[i]);
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_sleep(POLL_STAGGER);
#pragma unroll
  for (int i = 0; i < N; i++) r[1][i] = ldl1(wsb, w[i]);
  asm volatile("" ::: "memory");
  auto merge = [&](const uint32_t (&v)[N]) {
    bool all = true;
#pragma unroll
    for (int i = 0; i < N; i++) {
      if (!have[i] && (v[i] >> 16) == tag) {
        u[i] = v[i];
        have[i] = true;
      }
      all &= have[i];
    }
    return __all(all);
  };
#define MQ_WSTEP(k)                              \
  if (merge(r[(k) % 2])) return;                 \
  _Pragma("unroll") for (int i = 0; i < N; i++) r[(k) % 2][i] = ldl1(wsb, w[i]); \
  asm volatile("" ::: "memory");
  MQ_WSTEP(0) MQ_WSTEP(1) MQ_WSTEP(2) MQ_WSTEP(3) MQ_WSTEP(4) MQ_WSTEP(5)
  MQ_WSTEP(6) MQ_WSTEP(7) MQ_WSTEP(8) MQ_WSTEP(9) MQ_WSTEP(10) MQ_WSTEP(11)
#undef MQ_WSTEP
  merge(r[0]);
  merge(r[1]);
  uint32_t spins = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; i++) ok &= have[i];
    if (ok || watchdog(wsb, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; i++)
      if (!have[i]) {
        const uint32_t v = ldl1(wsb, w[i]);
        if ((v >> 16) == tag) {
          u[i] = v;
          have[i] = true;
        }
      }
  }
  return;
  }
  {
#pragma unroll
  for (int i = 0; i < N; i++) u[i] = ldl1(wsb, w[i]);
  uint32_t spins = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; i++) ok &= (u[i] >> 16) == tag;
    if (ok || watchdog(wsb, ws, ++spins)) break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int i = 0; i < N; i++)
      if ((u[i] >> 16) != tag) u[i] = ldl1(wsb, w[i]);
  }
  }
}

// v[q] for q = 0..3 as two levels of selects on the bits of q (no branches)
__device__ __forceinline__ float pick4(int q, float v0, float v1, float v2, float v3) {
  const float lo = (q & 1) ? v1 : v0, hi = (q & 1) ? v3 : v2;
  return (q & 2) ? hi : lo;
}
// For lanes 0..15: x of lanes j + 16, j + 32 and j + 48 (j = lane), the "other" results of
// v_permlane16_swap / v_permlane32_swap of x with itself (a lane's pair of results holds its
// own value and its partner's, in either order; equal bits either way when they are equal).
__device__ __forceinline__ float swap_other(float own, u32x2 sw) {
  return __uint_as_float(sw[0] == __float_as_uint(own) ? sw[1] : sw[0]);
}
__device__ __forceinline__ void lane_rows(float x, float& a1, float& a2, float& a3) {
  const uint32_t u = __float_as_uint(x);
  const auto s16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  a1 = swap_other(x, u32x2{s16[0], s16[1]});  // lanes 0..15: lane + 16; lanes 32..47: lane + 16
  const auto s32 = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  a2 = swap_other(x, u32x2{s32[0], s32[1]});  // lanes 0..31: lane + 32
  const uint32_t u1 = __float_as_uint(a1);
  const auto s32b = __builtin_amdgcn_permlane32_swap(u1, u1, false, false);
  a3 = swap_other(a1, u32x2{s32b[0], s32b[1]});  // lanes 0..15: a1 of lane + 32, i.e. x of lane + 48
}

// HF Qwen3's q_norm / k_norm over one head (modeling_qwen3.py:252-253), then RoPE
// (apply_rotary_pos_emb, :147-170), each op rounded to bf16: lane holds dims lane and
// lane + 64 (tagged words u0, u1); nw0 selects the q_norm (0) or k_norm (64) weight words.
__device__ __forceinline__ void qk_norm_rope(uint32_t u0, uint32_t u1, const uint32_t* s_qkn, int nw0,
                                             const float* s_cos, const float* s_sin, int lane, float& ra,
                                             float& rb) {
  const uint32_t na = s_qkn[nw0 + (lane >> 1)], nb = s_qkn[nw0 + 32 + (lane >> 1)];
  const float wa = (lane & 1) ? bfhi(na) : bflo(na), wb = (lane & 1) ? bfhi(nb) : bflo(nb);
  const float x0 = bflo(u0), x1 = bflo(u1);
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float rstd = 1.0f / sqrtf(ss * (1.0f / HD) + EPS);
  float fa = x0 * rstd, fb = x1 * rstd;
  rbf2(fa, fb);
  fa *= wa;
  fb *= wb;
  rbf2(fa, fb);
  float p0 = fa * s_cos[lane], p1 = fb * s_sin[lane], p2 = fb * s_cos[lane + 64], p3 = fa * s_sin[lane + 64];
  rbf2(p0, p1);
  rbf2(p2, p3);
  ra = p0 - p1;
  rb = p2 + p3;
  rbf2(ra, rb);
}

// ---------------------------------------------------------------- the kernel
// SPLIT = false is the instance for contexts of at most KV_CAP positions (one
// attention workgroup per XCD, one LDS pass): the chunk-merge and multi-pass code
// is compiled out of it. SPLIT = true handles every context length; PIPE (with SPLIT)
// overlaps a chunk's later LDS passes' K/V copies with the previous pass's work, the
// instance for chunks of more than one pass (compiled apart, so that the one-pass
// instance keeps its own register allocation).
template <bool SPLIT, bool PIPE = false>
__global__ void __launch_bounds__(NT, 1) mq_decode_kernel(DecodeParams P) {
  static_assert(SPLIT || !PIPE, "the pipelined passes belong to the split instance");
  __shared__ __align__(16) uint8_t s_kv[2 * KV_CAP * HD * 2];  // K rows, then V rows of the chunk
  __shared__ __align__(16) uint32_t s_x0[H / 2];               // normed h (A) or h1 (B) (bf16 pairs)
  __shared__ __align__(16) uint32_t s_x1[XUNITS / 2];          // attention output (A) or m (B) of the XCD
  __shared__ __align__(16) uint32_t s_wn[H / 2];               // A: input_layernorm, B: post_attention_layernorm
  __shared__ __align__(16) uint32_t s_wfn[H / 2];              // final norm weights
  __shared__ uint32_t s_qkn[HD];                               // q_norm words, then k_norm words
  __shared__ float s_cos[HD], s_sin[HD];
  __shared__ __align__(16) uint16_t s_q[2 * HD];      // normed, rotated q of the two heads
  __shared__ __align__(16) uint16_t s_p[2 * KV_CAP];  // bf16 softmax numerators
  __shared__ __align__(16) float s_sc[2][KV_CAP];      // attention scores
  __shared__ float s_ao[2][HD];                        // attention output (or unnormalised partial)
  __shared__ float s_ao1[2][HD];                       // a later LDS pass's unnormalised partial
  __shared__ float s_mx[8][2];                          // per-wave score maxima
  __shared__ __align__(16) float s_l[8][2];             // per-wave softmax sums
  __shared__ float s_hrow[ROWS];                       // the residual rows this workgroup reduces
  __shared__ uint32_t s_cnt;                           // stream-wave results published so far
  __shared__ uint32_t s_red;                           // reductions stored by the reduce wave
  __shared__ uint32_t s_nrm;                           // norm-weight sets written by the stream waves
  __shared__ float s_ssx[2];                           // the poll waves' half sums of squares
  __shared__ uint32_t s_ssn;                           // half sums written so far
  __shared__ const uint16_t* s_lw[MAX_LAYERS][11];    // weight pointers, copied once per launch
  __shared__ float s_bestv[8];
  __shared__ int s_besti[8];
  __shared__ uint32_t s_flag;
  __shared__ uint32_t s_epoch;                         // this launch's epoch
  float* s_lg = reinterpret_cast<float*>(s_kv);  // this workgroup's logits (K/V rows are dead by then)
  __shared__ __align__(16) uint8_t s_lmx[LM_X_ROWS * H * 2];   // LM-head rows LM_KV_ROWS .. LM_ROWS - 1
  static_assert(LM_OFF + LM_KV_ROWS * H * 2 <= sizeof(s_kv) && LM_OFF >= 594 * 4, "LM rows fit behind the logits");
  // The unsplit instance: every group-A workgroup attends over the whole context in one pass,
  // and P.V writes the bf16 attention output straight into the o_proj input (s_x1), so the
  // o_proj dot products follow the attention's last barrier (B4) with no hand-out.
  uint16_t* const pv16 = SPLIT ? nullptr : reinterpret_cast<uint16_t*>(s_x1);

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
  const bool ga = j < NGA;                 // group A (else B)
  const int m = ga ? j : j - NGA;          // member index within the group
  uint32_t* ws = P.ws;
  const Buf wsb(ws);
  // token and position: kernel arguments, or a device-resident step written by the previous
  // launch's last workgroup. Launches on one stream do not overlap (a launch's first
  // workgroup starts after the previous launch's last one has finished), so the step, like
  // the workspace's epoch word, holds the previous launch's values; both are written and
  // read with device-scope (sc1) accesses.
  MQ_STAMP(32 * 40 + 4);
  int token = P.token, p = P.position, step_count = 0;
  uint32_t epoch = 0;  // this launch's exchange epoch: set from the workspace at P00
  if (P.mode & MODE_DEVICE_STEP) {
    const u32x4 sv = Buf(P.step).ld4(0);
    token = (int)__builtin_amdgcn_readfirstlane(sv.x);
    p = (int)__builtin_amdgcn_readfirstlane(sv.y);
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

  // attention chunking: nsplit chunks, chunk a on A workgroup (g, a), attended in npass LDS
  // passes of <= KV_CAP positions
  const int n_ctx = p + 1;
  const int nsplit = SPLIT ? plan_nsplit(n_ctx) : 1;
  const int CH = SPLIT ? plan_chunk(n_ctx) : n_ctx;
  // contexts of at most KV_CAP positions: every group-A workgroup attends over the whole
  // context (the same result in each), so none needs the attention output handed out;
  // longer contexts: chunk m on member m < nsplit
  const bool att = ga && (SPLIT ? m < nsplit : true);
  const int c0 = SPLIT ? m * CH : 0;  // the unsplit instance: every A workgroup from position 0
  const int nc = att ? min(n_ctx, c0 + CH) - c0 : 0;
  const int npass = SPLIT ? (nc + KV_CAP - 1) / KV_CAP : 1;
  const int nc0 = min(nc, KV_CAP);
  // K/V rows by non-temporal copies where that measured faster: the unsplit instance and
  // chunks of several passes (one-pass chunks of 257..4096-position contexts lose 1-9 us)
  const bool kv_nt = !SPLIT || npass > 1;
  const bool own_p = att && p >= c0 && p < c0 + nc;  // p is always in the last pass
  // which group's reduce waves sum the o_proj partials (uniform across the grid)
  const bool b_h1 = !SPLIT && n_ctx >= B_H1_MIN_CTX;
  const int prow = p - c0 - KV_CAP * (npass - 1);     // its LDS row there
  const uint32_t lds_kv = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)s_kv;
  auto pass_rows = [&](int ps) { return ps == npass - 1 ? nc - KV_CAP * ps : KV_CAP; };

  // LM-head rows of this workgroup: 594 for w < 128, 593 after (151936 in total)
  const int r0 = w < 128 ? w * 594 : 128 * 594 + (w - 128) * 593;
  const int r1 = r0 + (w < 128 ? 594 : 593);
  // the workgroups whose first LM-head rows sit in LDS for the LM head, and how many: group A
  // copies LM_N after its last layer, group B NSW in the quiet window of each layer but the
  // last
  const bool lm_lds = lm && (ga || !SPLIT);
  constexpr int LM_X = SPLIT && !PIPE ? LM_X_ROWS : 0;  // rows in s_lmx in this instance
  constexpr int LM_N = LM_KV_ROWS + LM_X;
  const int lm_n = !lm_lds ? 0 : ga ? LM_N : min(LM_N, NSW * (L - 1));
  // LM-head row r0 + i into the K/V LDS array (two 1 KB halves, non-temporal)
  auto lm_row_dma = [&](int i) {
    const uint16_t* src = P.lm_head + (size_t)(r0 + i) * H + 8 * (tid & 63);
    const uint32_t dst = __builtin_amdgcn_readfirstlane(
        LM_X == 0 || i < LM_KV_ROWS ? lds_kv + LM_OFF + 2048u * (uint32_t)i
                       : (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)s_lmx +
                             2048u * (uint32_t)(i - LM_KV_ROWS));
    dma16_nt(src, dst);
    dma16_nt(src + 512, dst + 1024u);
  };

  float bestv = -INFINITY;
  int besti = 0x7fffffff;
  const u32x4* x0v = reinterpret_cast<const u32x4*>(s_x0);
  const u32x4* x1v = reinterpret_cast<const u32x4*>(s_x1);

  // rows past the chunk length must read as zeros in every layer
  for (int i = tid; i < 2 * KV_CAP * HD * 2 / 16; i += NT) reinterpret_cast<u32x4*>(s_kv)[i] = u32x4{0u, 0u, 0u, 0u};

  if (wave < NSW) {
    // ==================================================================== stream waves
    const int s = wave, st = tid;  // st: stream thread 0..255
    // the workspace's epoch word, loaded ahead of the pointer table (a wave's loads complete
    // in order, so it has landed when the table has)
    uint32_t ew = 0;
    if (st == 0) ew = wsb.ld1(WS_EPOCH * 4u);
    for (int i = st; i < L * 11; i += NSW * 64)
      s_lw[i / 11][i % 11] = reinterpret_cast<const uint16_t* const*>(P.layers)[i];
    if (st == 0) s_epoch = ew + 1u;
    BAR();  // P00: pointer table and epoch visible
    epoch = __builtin_amdgcn_readfirstlane(s_epoch);
    auto wp = [&](int l, int k) -> const uint16_t* { return uniform_ptr(s_lw[l][k]); };
    if (lm) {
      const u32x2 fn = ldw2(P.final_norm + 4 * st);
      s_wfn[2 * st] = fn.x;
      s_wfn[2 * st + 1] = fn.y;
    }
    // the norm weights of layer l into LDS for the poll waves, then counted (the poll waves
    // read them only after the count shows the set complete)
    auto publish_norms = [&]() {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) signal_store(&s_nrm);
    };
    if (ga) {
      // ================================================================ group A
      ARegs R;
      const int oc = lane & 31, org = lane >> 5;  // o_proj: chunk oc of the group's 256 columns, row pair half
      auto load_a = [&](int l) {
        const int r = QROWS * m + 8 * s;  // this wave's 8 rows of the group's [q0; q1; k; v]
        const uint16_t* pa = r < 256   ? wp(l, W_Q) + (size_t)(256 * g + r) * H
                             : r < 384 ? wp(l, W_K) + (size_t)(128 * g + r - 256) * H
                                       : wp(l, W_V) + (size_t)(128 * g + r - 384) * H;
#pragma unroll
        for (int k = 0; k < 8; k++) {
          R.a[2 * k] = ldw(pa + k * H + 8 * lane);
          R.a[2 * k + 1] = ldw(pa + k * H + 512 + 8 * lane);
        }
      };
      auto load_o = [&](int l) {  // rows 64m + 16s + 2i + org
        const uint16_t* po = wp(l, W_O) + (size_t)(ROWS * m + 16 * s + org) * QS + 256 * g + 8 * oc;
#pragma unroll
        for (int i = 0; i < 8; i++) R.o[i] = ldw(po + (size_t)(2 * i) * QS);
      };
      auto load_norms = [&](int l) {
        R.wln = ldw2(wp(l, W_IN) + 4 * st);
        R.qkn = ldw1(wp(l, st < 64 ? W_QN : W_KN) + 2 * (st & 63));
      };
      auto put_norms = [&]() {
        s_wn[2 * st] = R.wln.x;
        s_wn[2 * st + 1] = R.wln.y;
        if (st < 128) s_qkn[st] = R.qkn;
        publish_norms();
      };
      // ---- prologue: layer-0 norms, weights and K/V rows
      load_norms(0);
      load_a(0);
      put_norms();
      BAR();  // P0
      if (att) kv_dma(kv_nt, P, 0, g, c0, nc0, p, lds_kv, s, lane);
      load_o(0);  // (needed after the attention)
      for (int layer = 0; layer < L; layer++) {
        // ---------------- q/k/v rows 32m + 8s .. +7 of the group's [q0; q1; k; v]
        BAR();  // A1: normed h in s_x0
        MQ_STAMP(layer * 40 + 0);
        {
          const u32x4 x0 = x0v[lane], x1 = x0v[64 + lane];
          float r[8];
#pragma unroll
          for (int k = 0; k < 8; k++) r[k] = dot_chunk(R.a[2 * k], x0, dot_chunk(R.a[2 * k + 1], x1, 0.f));
          wave_sum_t(r);  // lane 16q holds rows 2q, 2q + 1
          // the wave publishes its own 8 rows (tagged, bf16), no hand-off to the store wave
          if ((lane & 15) == 0)
            st2_plain(ws + lb + LX_QKV + QROWS * m + 8 * s + 2 * (lane >> 4),
                      u32x2{tagged(tag_of(epoch, layer), rbf(r[0])), tagged(tag_of(epoch, layer), rbf(r[1]))});
          if (lane == 0) signal_store(&s_cnt);
          AFTER(r[0] + r[1]);
          MQ_STAMP(layer * 40 + 1);
        }
        if (att) {
          // this wave's K/V copy of the layer has landed (issued in the previous layer's
          // quiet window; all of the wave's vector-memory operations are awaited)
          wait_vmem();
          // Later passes of a chunk (contexts past 256 positions a chunk). PIPE: a pass's K
          // rows are copied while the previous pass runs its P.V (the previous K rows are
          // consumed at B2), its V rows while it runs its own scores and softmax (the previous
          // V rows are consumed at B4); each copy is issued after the wave's last wait, so
          // every wait is for all of the wave's copies in flight. Otherwise a pass's K and V
          // rows are copied, and awaited, after the previous pass.
          if constexpr (PIPE) {
            const bool piped = npass > 1;
            for (int ps = 0; ps < npass; ps++) {
              if (ps > 0) {
                wait_vmem();  // the pass's K rows
                kv_dma<2>(kv_nt, P, layer, g, c0 + KV_CAP * ps, pass_rows(ps), p, lds_kv, s, lane);
              }
              // the new v row (the raw bf16 values), polled when no copy of this wave is in
              // flight: before B1, or before B3 when the passes are pipelined
              auto v_row = [&]() {
                const uint32_t w[2] = {lb + LX_QKV + 3 * HD + lane, lb + LX_QKV + 3 * HD + 64 + lane};
                uint32_t u[2];
                poll_words<!SPLIT>(wsb, ws, w, tag_of(epoch, layer), u);
                uint8_t* vbase = s_kv + KV_CAP * 256;
                *reinterpret_cast<uint16_t*>(vbase + vkv_off(prow, lane >> 3) + 2 * (lane & 7)) = (uint16_t)(u[0] & 0xffffu);
                *reinterpret_cast<uint16_t*>(vbase + vkv_off(prow, 8 + (lane >> 3)) + 2 * (lane & 7)) =
                    (uint16_t)(u[1] & 0xffffu);
              };
              const bool vrow = s == 0 && own_p && ps == npass - 1;
              if (vrow && !piped) v_row();
              const int ncp = pass_rows(ps);
              BAR();  // B1: q, the new k row (unless pipelined: and v row) and the pass's K rows are in LDS
              MQ_STAMP(layer * 40 + 2);
              attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
              BAR();  // B2: the pass's K rows consumed
              float M0, M1, L0, L1;
              attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
              if (piped) {
                wait_vmem();  // the pass's V rows
                if (vrow) v_row();
                if (ps + 1 < npass)
                  kv_dma<1>(kv_nt, P, layer, g, c0 + KV_CAP * (ps + 1), pass_rows(ps + 1), p, lds_kv, s, lane);
              }
              BAR();  // B3: the pass's V rows and the new v row are in LDS
              attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1, pv16);
              BAR();  // B4: the pass's V rows consumed
              MQ_STAMP(layer * 40 + 3);
            }
          } else {
            for (int ps = 0; ps < npass; ps++) {
              if (ps > 0) {
                // rows KV_CAP * ps .. of the chunk replace the previous pass's rows
                kv_dma(kv_nt, P, layer, g, c0 + KV_CAP * ps, pass_rows(ps), p, lds_kv, s, lane);
                wait_vmem();
              }
              if (s == 0 && own_p && ps == npass - 1) {
                // the new v row (the raw bf16 values; no loads of this wave are in flight)
                const uint32_t w[2] = {lb + LX_QKV + 3 * HD + lane, lb + LX_QKV + 3 * HD + 64 + lane};
                uint32_t u[2];
                poll_words<!SPLIT>(wsb, ws, w, tag_of(epoch, layer), u);
                uint8_t* vbase = s_kv + KV_CAP * 256;
                *reinterpret_cast<uint16_t*>(vbase + vkv_off(prow, lane >> 3) + 2 * (lane & 7)) = (uint16_t)(u[0] & 0xffffu);
                *reinterpret_cast<uint16_t*>(vbase + vkv_off(prow, 8 + (lane >> 3)) + 2 * (lane & 7)) =
                    (uint16_t)(u[1] & 0xffffu);
              }
              const int ncp = pass_rows(ps);
              BAR();  // B1: q, the new k/v row and the K/V rows are in LDS
              MQ_STAMP(layer * 40 + 2);
              attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
              BAR();  // B2
              float M0, M1, L0, L1;
              attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
              BAR();  // B3
              attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1, pv16);
              BAR();  // B4: K/V rows consumed
              MQ_STAMP(layer * 40 + 3);
            }
          }
        }
        // ---------------- o_proj partials: rows 64m + 16s + 2i + org over the group's 256 columns
        if constexpr (SPLIT) BAR();  // C1: attention output of the group in s_x1 (unsplit: at B4)
        MQ_STAMP(layer * 40 + 4);
        {
          const u32x4 xa = x1v[oc];
          float r[8];
#pragma unroll
          for (int i = 0; i < 8; i++) r[i] = dot_chunk(R.o[i], xa, 0.f);
          half_sum_t(r);  // every lane of lane row q holds pairs i + 4 (q & 1), i < 4, of row half q >> 1
          // lanes 16q + i (i < 4) store pair i + 4 (q & 1) of row half q >> 1, i.e. row
          // 2 (i + 4 (q & 1)) + (q >> 1), straight from registers: the 16 lanes write the wave's
          // 16 (value, tag) pairs, one 128-byte run (a regrouping into lanes 0..15, through LDS
          // or by permlane swaps, measured slower)
          {
            const int i4 = lane & 3, q = lane >> 4;
            const float rv = pick4(i4, r[0], r[1], r[2], r[3]);
            if ((lane & 12) == 0)
              st2_dev(ws + X_OPART + 2 * ((m * NXCD + g) * ROWS + 16 * s + 2 * (i4 + 4 * (q & 1)) + (q >> 1)),
                      u32x2{__float_as_uint(rv), epoch * 32u + (uint32_t)layer + 1u});
          }
          if (lane == 0) signal_store(&s_cnt);
          AFTER(r[0] + r[1] + r[2] + r[3]);
          MQ_STAMP(layer * 40 + 5);
        }
        // group A's quiet window: once this workgroup's reduce wave has stored its h1 rows,
        // group B carries the layer, and this workgroup streams its next layer's weights
        if (!b_h1) wait_count(&s_red, (uint32_t)layer + 1u);
        if (layer + 1 < L) {
          load_norms(layer + 1);
          load_a(layer + 1);
          load_o(layer + 1);
          put_norms();
          if (att) kv_dma(kv_nt, P, layer + 1, g, c0, nc0, p, lds_kv, s, lane);
          MQ_LANDED(layer * 40 + 10);
        } else if (lm_lds) {
          // the K/V rows are dead (the last attention is done): this wave's share of the
          // workgroup's first LM-head rows into LDS
          for (int i = s; i < LM_N; i += NSW) lm_row_dma(i);
        }
      }
    } else {
      // ================================================================ group B
      BRegs R;
      // down_proj: lanes < 48 take chunk `lane` of the XCD's 384 columns (the others re-read
      // chunk 47 and are multiplied by zero)
      const int dch = lane < 48 ? lane : 47;
      auto load_gu = [&](int l) {  // gate and up rows of units 384g + 24m + 6s .. +5
        const uint16_t* pg = wp(l, W_G) + (size_t)(XUNITS * g + UNITS * m + 6 * s) * H;
        const uint16_t* pu = wp(l, W_U) + (size_t)(XUNITS * g + UNITS * m + 6 * s) * H;
#pragma unroll
        for (int k = 0; k < 6; k++) {
          R.gu[2 * k] = ldw(pg + k * H + 8 * lane);
          R.gu[2 * k + 1] = ldw(pg + k * H + 512 + 8 * lane);
        }
#pragma unroll
        for (int k = 0; k < 6; k++) {
          R.gu[12 + 2 * k] = ldw(pu + k * H + 8 * lane);
          R.gu[13 + 2 * k] = ldw(pu + k * H + 512 + 8 * lane);
        }
      };
      auto load_d = [&](int l) {  // rows 64m + 16s .. +15, the XCD's 384 columns
        const uint16_t* pd = wp(l, W_D) + (size_t)(ROWS * m + 16 * s) * I + XUNITS * g + 8 * dch;
#pragma unroll
        for (int i = 0; i < 16; i++) R.d[i] = ldw(pd + (size_t)i * I);
      };
      auto put_norms = [&]() {
        s_wn[2 * st] = R.wpost.x;
        s_wn[2 * st + 1] = R.wpost.y;
        publish_norms();
      };
      // ---- prologue: layer-0 post-attention norm and weights (streamed during group A's
      // first layer)
      // the norm weights alone first: the layer-0 MLP weights (needed only once group A's
      // attention is done) go out after the prologue barrier, so that the first q/k/v rows
      // and norm weights of every workgroup meet less traffic
      R.wpost = ldw2(wp(0, W_POST) + 4 * st);
      put_norms();
      BAR();  // P0
      load_gu(0);
      load_d(0);
      // split contexts of more than one chunk: this workgroup reads the first pass's K/V rows
      // of chunk m two layers ahead into its (otherwise unused) K/V LDS array, so that they
      // sit in the XCD's L2 when the chunk's attention workgroup copies them (its copy is
      // issued a layer before their use, behind its own weight burst)
      auto warm_kv = [&](int l) {
        if constexpr (SPLIT) {
          if (l < L && m < nsplit && nsplit > 1) {
            const int wc0 = m * CH;
            kv_dma(false, P, l, g, wc0, min(min(n_ctx, wc0 + CH) - wc0, KV_CAP), p, lds_kv, s, lane);
          }
        }
      };
      warm_kv(1);
      for (int layer = 0; layer < L; layer++) {
        // ---------------- gate/up rows of units 384g + 24m + 6s .. +5
        BAR();  // D1: normed h1 in s_x0
        MQ_STAMP(layer * 40 + 6);
        {
          const u32x4 x0 = x0v[lane], x1 = x0v[64 + lane];
          float r[12];
#pragma unroll
          for (int k = 0; k < 12; k++) r[k] = dot_chunk(R.gu[2 * k], x0, dot_chunk(R.gu[2 * k + 1], x1, 0.f));
          wave_sum_t(r);  // every lane of lane row q holds rows 3q .. 3q + 2
          // HF Qwen3MLP (modeling_qwen3.py:81-83): m = bf16(bf16(silu(gate)) * up) of the
          // wave's 6 units, stored by the wave. Lane j < 6 takes unit j: its gate row j is r[j % 3]
          // of lane row j / 3, its up row 6 + j is r[j % 3] of lane row 2 + j / 3; the values reach
          // lanes 0..5 by permlane swaps (no regrouping through LDS)
          {
            const int j = lane & 15, k = j % 3;
            float a1, a2, a3;
            const float x = pick4(k, r[0], r[1], r[2], r[2]);
            lane_rows(x, a1, a2, a3);
            if (lane < 6) {
              const float gt = rbf(lane < 3 ? x : a1), up = rbf(lane < 3 ? a2 : a3);
              st1_plain(ws + lb + LX_M + UNITS * m + 6 * s + lane,
                        tagged(tag_of(epoch, layer), rbf(rbf(gt / (1.0f + expf(-gt))) * up)));
            }
          }
          if (lane == 0) signal_store(&s_cnt);
          AFTER(r[0] + r[1] + r[2]);
          MQ_STAMP(layer * 40 + 7);
        }
        // ---------------- down_proj partials: rows 64m + 16s .. +15 over the XCD's 384 units
        BAR();  // E1: m of the XCD in s_x1
        MQ_STAMP(layer * 40 + 8);
        {
          const u32x4 xm = lane < 48 ? x1v[lane] : u32x4{0u, 0u, 0u, 0u};
          float r[16];
#pragma unroll
          for (int i = 0; i < 16; i++) r[i] = dot_chunk(R.d[i], xm, 0.f);
          wave_sum_t(r);  // every lane of lane row q holds rows 4q .. 4q + 3
          // lanes 16q + k (k < 4) store row 4q + k straight from registers: the wave's 16
          // partials as one 128-byte run of (value, tag) pairs (a regrouping into lanes 0..15
          // measured slower)
          {
            const int k4 = lane & 3;
            const float rv = pick4(k4, r[0], r[1], r[2], r[3]);
            if ((lane & 12) == 0)
              st2_dev(ws + X_DPART + 2 * ((m * NXCD + g) * ROWS + 16 * s + 4 * (lane >> 4) + k4),
                      u32x2{__float_as_uint(rv), epoch * 32u + (uint32_t)layer + 1u});
          }
          if (lane == 0) signal_store(&s_cnt);
          AFTER(r[0] + r[1] + r[2] + r[3]);
          MQ_STAMP(layer * 40 + 9);
        }
        // group B's quiet window: once this workgroup's reduce wave has stored its h rows,
        // group A carries the next layer, and this workgroup streams its next MLP weights
        wait_count(&s_red, (uint32_t)layer + 1u);
        if (layer + 1 < L) {
          // hold the burst until group A has published the next layer's q/k/v rows (its
          // member 0's first word), so that it runs during A's attention
          // (before the weight loads, so that waiting for them covers these copies too)
          if (NSW * layer + s < lm_n) lm_row_dma(NSW * layer + s);
          R.wpost = ldw2(wp(layer + 1, W_POST) + 4 * st);
          load_gu(layer + 1);
          load_d(layer + 1);
          put_norms();
          MQ_LANDED(layer * 40 + 11);
          if constexpr (SPLIT) {
            // once chunk m's attention of the next layer is done (its partial record carries
            // that layer's tag; there are records only with more than one chunk), the XCD's
            // L2 has room: warm the chunk's first pass of the layer after it, which its
            // attention workgroup copies after its o_proj partials
            if (layer + 2 < L && m < nsplit && nsplit > 1) {
              const uint32_t rec = lb + LX_PART + 2 * (m * 2 * APART) + 1, want = epoch * 32u + (uint32_t)layer + 2u;
              uint32_t spins = 0;
              while (ldl1(wsb, rec) != want) {
                if (watchdog(wsb, ws, ++spins)) break;
                __builtin_amdgcn_s_sleep(8);
              }
              warm_kv(layer + 2);
            }
          }
        }
      }
    }
    if (lm_lds) wait_vmem();  // the LM-head rows' copies have landed
    BAR();  // F1: final normed h in s_x0
  } else if (wave < NSW + NPW) {
    // ==================================================================== poll waves
    const int c = wave - NSW, pt = tid - NSW * 64;  // pt: poll thread 0..127
    // group A's layer-0 residual stream (the embedding row, or the hidden input), loaded
    // before the prologue so that its latency overlaps the pointer table's and the norms'
    u32x2 emb[4];
    if (ga) {
      const uint16_t* src = (P.mode & MODE_INPUT_HIDDEN) ? P.hidden_in : P.embed + (size_t)token * H;
#pragma unroll
      for (int k = 0; k < 4; k++) emb[k] = ldw2(src + 4 * (lane + 64 * k));
    }
    for (int i = pt; i < 2 * HD; i += NPW * 64) {
      if (i < HD) s_cos[i] = bf2f(ldraw16(P.cos_tab + (size_t)p * HD + i));
      else s_sin[i - HD] = bf2f(ldraw16(P.sin_tab + (size_t)p * HD + i - HD));
    }
    BAR();  // P00
    epoch = __builtin_amdgcn_readfirstlane(s_epoch);
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
    // rows 64m .. 64m+63 (chunks 16m .. 16m+15, all in block k = m / 4) for the reduce wave
    auto keep_rows = [&](const u32x4& hv0, const u32x4& hv1) {
      const int q = lane - ((16 * m) & 63);
      if (c == (m >> 3) && q >= 0 && q < 16) {  // block m / 4 is in this wave's half
        float f[4];
        unpack_tagged((m >> 2) & 1 ? hv1 : hv0, f);
#pragma unroll
        for (int e = 0; e < 4; e++) s_hrow[4 * q + e] = f[e];
      }
    };
    // norm weights of layer l published by the stream waves (NSW per layer, from layer 0)
    auto wait_norms = [&](int l) { wait_count(&s_nrm, (uint32_t)(NSW * (l + 1))); };

    u32x4 hv0, hv1;  // this wave's half of the residual stream: chunks lane + 128c and lane + 128c + 64
    uint32_t ngat = 0;  // residual-stream gathers so far
    if (ga) {
      // ================================================================ group A
      for (int layer = 0; layer < L; layer++) {
        const uint32_t tag = tag_of(epoch, layer);
        const uint32_t tag64 = epoch * 32u + (uint32_t)layer + 1u;
        MQ_STAMP(layer * 40 + 12);
        // ---------------- gather h (each poll wave its half, with the sum of squares), RMSNorm
        float ss;
        if (layer == 0) {
          ss = 0.f;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            const u32x2 v = emb[k];
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
          ngat++;
          wait_cue(wsb, ws, lb + LX_CUE_B, tag_of(epoch, layer - 1));
          MQ_STAMP(layer * 40 + 39);
          ss = gather_half(wsb, ws, lb + LX_H, tag_of(epoch, layer - 1), c, lane, hv0, hv1, s_ssx, &s_ssn, 2u * ngat,
                           layer * 40 + 18);
        }
        MQ_STAMP(layer * 40 + 13);
        wait_norms(layer);
        norm_out(hv0, hv1, ss, s_wn);
        keep_rows(hv0, hv1);
        BAR();  // A1
        MQ_STAMP(layer * 40 + 14);
        if (att) {
          // ---------------- QK-norm, RoPE, K/V row p, attention
          // poll wave 0: q head 2g; poll wave 1: k; the reduce wave: q head 2g + 1; stream
          // wave 0: v
          // (lane holds dims lane, lane + 64)
          float fr[1][2];
          if (c == 0) {
            const uint32_t w[2] = {lb + LX_QKV + lane, lb + LX_QKV + 64 + lane};
            uint32_t u[2];
            poll_words<!SPLIT>(wsb, ws, w, tag, u);
            MQ_STAMP(layer * 40 + 15);
            float ra, rb;
            qk_norm_rope(u[0], u[1], s_qkn, 0, s_cos, s_sin, lane, ra, rb);
            s_q[lane] = (uint16_t)f2bf(ra);
            s_q[64 + lane] = (uint16_t)f2bf(rb);
          } else {
            const uint32_t w[2] = {lb + LX_QKV + 2 * HD + lane, lb + LX_QKV + 2 * HD + 64 + lane};
            uint32_t u[2];
            poll_words<!SPLIT>(wsb, ws, w, tag, u);
            qk_norm_rope(u[0], u[1], s_qkn, 64, s_cos, s_sin, lane, fr[0][0], fr[0][1]);
          }
          MQ_STAMP(layer * 40 + 25);
          for (int ps = 0; ps < npass; ps++) {
            if (c == 1 && own_p && ps == npass - 1) {
              // the new k row into the LDS copy of the pass that holds position p (stream wave
              // 0 writes the v row; the store wave appends both to the cache); the passes'
              // copies exclude that row
              const int o0 = kv_off(prow, lane >> 3) + 2 * (lane & 7);
              const int o1 = kv_off(prow, 8 + (lane >> 3)) + 2 * (lane & 7);
              *reinterpret_cast<uint16_t*>(s_kv + o0) = (uint16_t)f2bf(fr[0][0]);
              *reinterpret_cast<uint16_t*>(s_kv + o1) = (uint16_t)f2bf(fr[0][1]);
            }
            const int ncp = pass_rows(ps);
            BAR();  // B1
            MQ_STAMP(layer * 40 + 16);
            attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
            MQ_STAMP(layer * 40 + 21);  // (slots 21..23: group B's elsewhere)
            BAR();  // B2
            MQ_STAMP(layer * 40 + 26);
            float M0, M1, L0, L1;
            attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
            MQ_STAMP(layer * 40 + 22);
            BAR();  // B3
            MQ_STAMP(layer * 40 + 27);
            attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1, pv16);
            MQ_STAMP(layer * 40 + 23);
            BAR();  // B4
          }
          MQ_STAMP(layer * 40 + 17);
        }
        // ---------------- o_proj input: the group's 256 attention outputs as bf16 pairs in s_x1
        // (the unsplit instance's P.V has written them)
        if (SPLIT && nsplit == 1) {
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
        } else if (SPLIT) {
          // every A workgroup merges the XCD's chunk partials itself, straight into its o_proj
          // input: thread pt takes dims d0, d0 + 1 of head hh (a poll wave per head), CG chunks
          // per round; lane q loads chunk q's (m, l), which the wave then reads by readlane
          const int hh = pt >> 6, d0 = 2 * (pt & 63);
          float Mc = -INFINITY, Lc = 0.f, O0 = 0.f, O1 = 0.f;
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
            // by one lane per chunk), then the accumulator pairs
            while (mlane && !fresh(ml)) {
              if (watchdog(wsb, ws, ++spins)) break;
              __builtin_amdgcn_s_sleep(1);
              ml = ldl4(wsb, bml);
            }
            MQ_STAMP(layer * 40 + 6);  // (slots 6..9: group B's stream waves elsewhere)
#pragma unroll
            for (int q = 0; q < CG; q++) ov[q] = q < nq ? ldl4(wsb, b0 + 4 * q * APART + 4 + 2 * d0) : u32x4{0u, 0u, 0u, 0u};
            MQ_STAMP_AFTER(layer * 40 + 9, ov[CG - 1].x);
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
            MQ_STAMP(layer * 40 + 7);
            MQ_VALUE(layer * 40 + 11, spins);
            // Chunk q's rescale factors in lane q: the running maximum before and after chunk q
            // (a chain of readlanes and maxima), then one exponential for all chunks at once:
            // the maximum after a chunk is the previous maximum or the chunk's own, whose
            // factor is exp(0) = 1 exactly, so exp(min - max) gives the other factor. The sums
            // then run chunk by chunk in order, as fma(l, eb, L * ea), with the factors read
            // back by readlane.
            float pm = Mc, mb = 0.f, ma = 0.f;  // this lane's chunk: running maximum before / after it
#pragma unroll
            for (int q = 0; q < CG; q++) {
              const bool in = q < nq;
              const float nm = fmaxf(pm, __uint_as_float(__builtin_amdgcn_readlane(ml.x, q)));
              mb = lane == q ? pm : mb;
              ma = lane == q ? nm : ma;
              pm = in ? nm : pm;
            }
            const float mq = __uint_as_float(ml.x);
            const bool up = mq > mb;
            const float e = expf(fminf(mb, mq) - ma);
            const float fa = mb == -INFINITY ? 0.f : (up ? e : 1.f), fb = up ? 1.f : e;
#pragma unroll
            for (int q = 0; q < CG; q++) {
              const bool in = q < nq;
              const float ea = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(fa), q));
              const float eb = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(fb), q));
              const float lq = __uint_as_float(__builtin_amdgcn_readlane(ml.z, q));
              const float nL = __builtin_fmaf(lq, eb, Lc * ea);
              const float n0 = __builtin_fmaf(__uint_as_float(ov[q].x), eb, O0 * ea);
              const float n1 = __builtin_fmaf(__uint_as_float(ov[q].z), eb, O1 * ea);
              Lc = in ? nL : Lc;
              O0 = in ? n0 : O0;
              O1 = in ? n1 : O1;
            }
            Mc = pm;
            MQ_STAMP_AFTER(layer * 40 + 8, O0 + O1 + Lc);
          }
          const float rl = 1.0f / Lc;
          s_x1[pt] = pack_bf2(rbf(O0 * rl), rbf(O1 * rl));
        }
        MQ_STAMP(layer * 40 + 19);
        if constexpr (SPLIT) BAR();  // C1
        MQ_STAMP(layer * 40 + 20);
      }
    } else {
      // ================================================================ group B
      for (int layer = 0; layer < L; layer++) {
        const uint32_t tag = tag_of(epoch, layer);
        const uint32_t tag64 = epoch * 32u + (uint32_t)layer + 1u;
        MQ_STAMP(layer * 40 + 12);
        // ---------------- gather h1; post-attention RMSNorm
        ngat++;
        wait_cue(wsb, ws, lb + LX_CUE_A, tag);
        MQ_STAMP(layer * 40 + 39);
        const float ss1 = gather_half(wsb, ws, lb + LX_H1, tag, c, lane, hv0, hv1, s_ssx, &s_ssn, 2u * ngat,
                                      layer * 40 + 18);
        MQ_STAMP(layer * 40 + 21);
        wait_norms(layer);
        norm_out(hv0, hv1, ss1, s_wn);
        keep_rows(hv0, hv1);
        BAR();  // D1
        MQ_STAMP(layer * 40 + 22);
        // ---------------- down_proj input: m of the XCD's 384 units (96 chunks)
        {
          const int q = pt;
          if (q < XUNITS / 4) {
            const u32x4 v = poll2_l4(wsb, ws, lb + LX_M + 4 * q, tag);
            reinterpret_cast<u32x2*>(s_x1)[q] = u32x2{pair_lo(v.x, v.y), pair_lo(v.z, v.w)};
          }
        }
        MQ_STAMP(layer * 40 + 23);
        BAR();  // E1
        MQ_STAMP(layer * 40 + 24);
      }
    }

    // ---------------- final norm (both groups)
    {
      ngat++;
      wait_cue(wsb, ws, lb + LX_CUE_B, tag_of(epoch, L - 1));
      const float ss = gather_half(wsb, ws, lb + LX_H, tag_of(epoch, L - 1), c, lane, hv0, hv1, s_ssx, &s_ssn, 2u * ngat);
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
    // The workgroup's 64 residual rows (lane = row) from the 8 XCDs' partial sums
    // (identical on every XCD): group A reduces o_proj into h1, group B down_proj into h.
    BAR();  // P00
    epoch = __builtin_amdgcn_readfirstlane(s_epoch);
    BAR();  // P0
    const int row = ROWS * m + lane;
    // group B with b_h1: this workgroup's 64 rows of the residual stream h (the embedding or
    // hidden-input rows, then each layer's own down_proj reduction)
    float hcur = 0.f;
    if (!ga && b_h1) {
      const uint16_t* src = (P.mode & MODE_INPUT_HIDDEN) ? P.hidden_in : P.embed + (size_t)token * H;
      hcur = bf2f(ldraw16(src + row));
    }
    for (int layer = 0; layer < L; layer++) {
      const uint32_t tag = tag_of(epoch, layer);
      const uint32_t tag64 = epoch * 32u + (uint32_t)layer + 1u;
      if (ga) {
        BAR();  // A1: h rows in s_hrow
        MQ_STAMP(layer * 40 + 28);
        const float hrow = s_hrow[lane];
        if (att) {
          {
            // q head 2g + 1: QK-norm and RoPE (the poll waves take q head 2g, k and v)
            const uint32_t w[2] = {lb + LX_QKV + HD + lane, lb + LX_QKV + HD + 64 + lane};
            uint32_t u[2];
            poll_words<!SPLIT>(wsb, ws, w, tag, u);
            float ra, rb;
            qk_norm_rope(u[0], u[1], s_qkn, 0, s_cos, s_sin, lane, ra, rb);
            s_q[HD + lane] = (uint16_t)f2bf(ra);
            s_q[HD + 64 + lane] = (uint16_t)f2bf(rb);
          }
          for (int ps = 0; ps < npass; ps++) {
            const int ncp = pass_rows(ps);
            BAR();  // B1
            attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
            BAR();  // B2
            float M0, M1, L0, L1;
            attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
            BAR();  // B3
            attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1, pv16);
            BAR();  // B4
          }
        }
        if constexpr (SPLIT) BAR();  // C1
        MQ_STAMP(layer * 40 + 29);
        if (!b_h1) {
          // h1 = bf16(h + bf16(o)) (modeling_qwen3.py:297-298)
          // the eight-XCD poll starts once this workgroup's stream waves have issued their
          // o_proj partials (four signals a stage), not through the whole attention phase
          wait_count(&s_cnt, 8u * (uint32_t)layer + 8u);
          const float h1v = rbf(hrow + rbf(reduce_row8(wsb, ws, X_OPART + 2 * (m * NXCD * ROWS + lane), tag64)));
          st1_plain(ws + lb + LX_H1 + row, tagged(tag, h1v));
          // the stream waves' next weight loads go behind this store
          if (lane == 0) signal_store(&s_red);
          MQ_STAMP(layer * 40 + 30);
        }
      } else {
        float h1row;
        if (b_h1) {
          // h1 = bf16(h + bf16(o)) of the same 64 rows, from the o_proj partials
          wait_own_part(wsb, ws, X_OPART + 2 * ((m * NXCD + g) * ROWS) + 1, tag64);
          h1row = rbf(hcur + rbf(reduce_row8(wsb, ws, X_OPART + 2 * (m * NXCD * ROWS + lane), tag64)));
          st1_plain(ws + lb + LX_H1 + row, tagged(tag, h1row));
          MQ_STAMP(layer * 40 + 33);
          BAR();  // D1
        } else {
          BAR();  // D1: h1 rows in s_hrow
          h1row = s_hrow[lane];
        }
        BAR();  // E1
        MQ_STAMP(layer * 40 + 31);
        // h' = bf16(h1 + bf16(down)) (modeling_qwen3.py:303-304)
        // the eight-XCD poll starts once this workgroup's stream waves have issued their
        // down_proj partials (a memory poll of its own partial instead measured slower)
        wait_count(&s_cnt, 8u * (uint32_t)layer + 8u);
        const float hn = rbf(h1row + rbf(reduce_row8(wsb, ws, X_DPART + 2 * (m * NXCD * ROWS + lane), tag64)));
        st1_plain(ws + lb + LX_H + row, tagged(tag, hn));
        hcur = hn;
        if (lane == 0) signal_store(&s_red);
        MQ_STAMP(layer * 40 + 32);
      }
    }
    BAR();  // F1
  } else {
    // ==================================================================== store wave
    if (lane == 0) {
      s_cnt = 0u;
      s_red = 0u;
      s_nrm = 0u;
      s_ssn = 0u;
    }
    BAR();  // P00
    epoch = __builtin_amdgcn_readfirstlane(s_epoch);
    BAR();  // P0
    // Every launch writes or clears every exchange word it could ever poll, so that the
    // content a poll can find before the awaited write is at most one launch old, whose
    // tags differ from the polled ones: a launch that does not write the attention-output
    // words clears them (only split launches with one chunk write and read them), and an A
    // workgroup without a chunk partial to store clears its chunk's record (read by split
    // launches with more chunks).
    if (ga && m == 0 && !(SPLIT && nsplit == 1)) st4_plain(ws + lb + LX_ATT + 4 * lane, u32x4{0u, 0u, 0u, 0u});
    if (ga && (!SPLIT || !att))
      for (int i = lane; i < 2 * 2 * (int)APART / 4; i += 64)
        st4_plain(ws + lb + LX_PART + 2 * 2 * APART * m + 4 * i, u32x4{0u, 0u, 0u, 0u});
    uint32_t target = 0;
    for (int layer = 0; layer < L; layer++) {
      const uint32_t tag = tag_of(epoch, layer);
      const uint32_t tag64 = epoch * 32u + (uint32_t)layer + 1u;
      if (ga) {
        BAR();  // A1
        target += NSW;
        wait_count(&s_cnt, target);  // (the stream waves store the q/k/v rows themselves)
        MQ_STAMP(layer * 40 + 34);
        if (att) {
          float Mr0 = 0.f, Mr1 = 0.f, Lr0 = 0.f, Lr1 = 0.f;  // running max / sum over the passes
          for (int ps = 0; ps < npass; ps++) {
            const int ncp = pass_rows(ps);
            BAR();  // B1
            if (own_p && (SPLIT || m == 0) && ps == npass - 1 && !(PIPE && npass > 1)) {
              // K/V-cache append (one workgroup per XCD) at slot p (bf16 [L][8][max_seq][128]):
              // lane -> dims 2 lane, 2 lane + 1; at B1 the new k and v rows are in LDS (at B3
              // when the passes are pipelined)
              const size_t slot = ((size_t)(layer * NKV + g) * P.max_seq_len + p) * HD;
              const uint32_t k2 = *reinterpret_cast<const uint32_t*>(s_kv + kv_off(prow, lane >> 2) + 4 * (lane & 3));
              const uint32_t v2 =
                  *reinterpret_cast<const uint32_t*>(s_kv + KV_CAP * 256 + vkv_off(prow, lane >> 2) + 4 * (lane & 3));
              st1_plain(reinterpret_cast<uint32_t*>(P.k_cache + slot) + lane, k2);
              st1_plain(reinterpret_cast<uint32_t*>(P.v_cache + slot) + lane, v2);
            }
            attn_scores(s_kv, s_q, s_sc, s_mx, ncp, P.attn_scale, wave, lane);
            BAR();  // B2
            float M0, M1, L0, L1;
            attn_softmax(s_sc, s_p, s_mx, s_l, ncp, wave, lane, M0, M1);
            BAR();  // B3
            if constexpr (PIPE) {
              if (own_p && ps == npass - 1 && npass > 1) {
                const size_t slot = ((size_t)(layer * NKV + g) * P.max_seq_len + p) * HD;
                const uint32_t k2 = *reinterpret_cast<const uint32_t*>(s_kv + kv_off(prow, lane >> 2) + 4 * (lane & 3));
                const uint32_t v2 =
                    *reinterpret_cast<const uint32_t*>(s_kv + KV_CAP * 256 + vkv_off(prow, lane >> 2) + 4 * (lane & 3));
                st1_plain(reinterpret_cast<uint32_t*>(P.k_cache + slot) + lane, k2);
                st1_plain(reinterpret_cast<uint32_t*>(P.v_cache + slot) + lane, v2);
              }
            }
            attn_pv(s_kv, s_p, s_l, ps ? s_ao1 : s_ao, ncp, wave, lane, nsplit == 1, L0, L1, pv16);
            BAR();  // B4
            if (ps == 0) {
              Mr0 = M0;
              Mr1 = M1;
              Lr0 = L0;
              Lr1 = L1;
            } else {
              // merge this pass into the running partial exactly: rescale both to the larger
              // maximum (lane -> outputs 4 lane .. 4 lane + 3 of head lane / 32); done before
              // the next pass's P.V rewrites s_ao1, which waits for this wave at B1
              const int hh = lane >> 5, dim = 4 * (lane & 31);
#pragma unroll
              for (int h2 = 0; h2 < 2; h2++) {
                const float ma = h2 ? Mr1 : Mr0, mb = h2 ? M1 : M0, mm = fmaxf(ma, mb);
                // exp(ma - mm) and exp(mb - mm): mm is one of the two, whose factor is
                // exp(0) = 1 exactly, so one exponential (of the same argument) gives both
                const bool up = mb > ma;
                const float e = expf(fminf(ma, mb) - mm);
                const float ea = up ? e : 1.f, eb = up ? 1.f : e;
                if (h2 == hh)
#pragma unroll
                  for (int e = 0; e < 4; e++) s_ao[hh][dim + e] = s_ao[hh][dim + e] * ea + s_ao1[hh][dim + e] * eb;
                const float lm2 = (h2 ? Lr1 : Lr0) * ea + (h2 ? L1 : L0) * eb;
                if (h2) {
                  Mr1 = mm;
                  Lr1 = lm2;
                } else {
                  Mr0 = mm;
                  Lr0 = lm2;
                }
              }
            }
          }
          const int hh = lane >> 5, dim = 4 * (lane & 31);
          if (nsplit == 1) {
            // split instance, one chunk: the other group-A workgroups gather it (in the
            // unsplit instance every group-A workgroup has attended itself)
            if (SPLIT)
              st4_plain(ws + lb + LX_ATT + hh * HD + dim,
                        u32x4{tagged(tag, rbf(s_ao[hh][dim])), tagged(tag, rbf(s_ao[hh][dim + 1])),
                              tagged(tag, rbf(s_ao[hh][dim + 2])), tagged(tag, rbf(s_ao[hh][dim + 3]))});
          } else {
            // chunk partial (m, l, unnormalised acc) as (fp32, tag) pairs; every A workgroup of
            // the XCD merges them
            uint32_t* pb = ws + lb + LX_PART + 2 * ((m * 2 + hh) * APART);
            st4_plain(pb + 2 * (2 + dim), u32x4{__float_as_uint(s_ao[hh][dim]), tag64,
                                                __float_as_uint(s_ao[hh][dim + 1]), tag64});
            st4_plain(pb + 2 * (4 + dim), u32x4{__float_as_uint(s_ao[hh][dim + 2]), tag64,
                                                __float_as_uint(s_ao[hh][dim + 3]), tag64});
            if (dim == 0)
              st4_plain(pb, u32x4{__float_as_uint(hh ? Mr1 : Mr0), tag64, __float_as_uint(hh ? Lr1 : Lr0), tag64});
          }
        }
        MQ_STAMP(layer * 40 + 35);
        // o_proj partials of rows 64m .. 64m+63 over this XCD's two heads
        if constexpr (SPLIT) BAR();  // C1
        target += NSW;
        wait_count(&s_cnt, target);  // (the stream waves store the partials themselves)
        if (m == 0 && lane == 0) st1_plain(ws + lb + LX_CUE_A, tag);
        MQ_STAMP(layer * 40 + 36);
      } else {
        // HF Qwen3MLP (modeling_qwen3.py:81-83): m = bf16(bf16(silu(gate)) * up)
        BAR();  // D1
        target += NSW;
        wait_count(&s_cnt, target);  // (the stream waves store m themselves)
        MQ_STAMP(layer * 40 + 37);
        // down_proj partials of rows 64m .. 64m+63 over this XCD's 384 units
        BAR();  // E1
        target += NSW;
        wait_count(&s_cnt, target);  // (the stream waves store the partials themselves)
        if (m == 0 && lane == 0) st1_plain(ws + lb + LX_CUE_B, tag);
        MQ_STAMP(layer * 40 + 38);
      }
    }
    wait_vmem();
    BAR();  // F1
  }

  // ==================================================================== LM head (all waves)
  MQ_STAMP(32 * 40 + 1);
  if (lm) {
    const u32x4 x0 = x0v[lane], x1 = x0v[64 + lane];
    // rows r0 + wave + 8i: four rows per batch, two batches in flight
    auto load_rows = [&](int rb, u32x4 (&Wr)[4][2]) {
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int r = rb + 8 * u;
        if (r < r1) {
          if (r - r0 < lm_n) {
            const uint8_t* lp = (LM_X == 0 || r - r0 < LM_KV_ROWS ? s_kv + LM_OFF + 2048 * (r - r0)
                                                     : s_lmx + 2048 * (r - r0 - LM_KV_ROWS)) +
                                16 * lane;
            Wr[u][0] = *reinterpret_cast<const u32x4*>(lp);
            Wr[u][1] = *reinterpret_cast<const u32x4*>(lp + 1024);
          } else {
            const uint16_t* rowp = P.lm_head + (size_t)r * H;
            Wr[u][0] = ldw(rowp + 8 * lane);
            Wr[u][1] = ldw(rowp + 512 + 8 * lane);
          }
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
    const int rs = r0 + wave;
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
      // the next launch's input: this token at the next position (a failed step keeps its
      // position, and its negative token stops the launches after it); the epoch field
      // records the epoch this step used
      P.out_ids[step_count] = res;
      Buf(P.step).st4(u32x4{(uint32_t)res, (uint32_t)(res >= 0 ? p + 1 : p), epoch, (uint32_t)(step_count + 1)}, 0);
    }
    wsb.st1(0u, WS_ERR * 4u);
    wsb.st1(0u, WS_FINAL_TICKET * 4u);
    wsb.st1(epoch, WS_EPOCH * 4u);
  }
}

// ---------------------------------------------------------------- host side
// The library's workspace of a device. A launch takes its exchange epoch from the
// workspace itself (WS_EPOCH, advanced by each launch's last workgroup), not from the host:
// launches on one stream run one after another (the next launch's first workgroup starts
// about 1 us after the previous launch's last workgroup has finished, measured with
// s_memrealtime stamps for ordinary launches and for HIP graph replays alike), so every
// workgroup of a launch reads the epoch the previous launch on this workspace stored.
struct DeviceState {
  bool init = false;
  int status = MQ_OK;
  uint32_t* ws = nullptr;
};
static std::mutex g_mu;
static DeviceState g_dev[64];

// The device can hold all NWG workgroups of both kernel instances at once (no allocation).
static int check_device(int dev) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return MQ_ERR_HIP;
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0 || !prop.cooperativeLaunch) return MQ_ERR_DEVICE;
  for (const void* k : {reinterpret_cast<const void*>(mq_decode_kernel<false>),
                        reinterpret_cast<const void*>(mq_decode_kernel<true>),
                        reinterpret_cast<const void*>(mq_decode_kernel<true, true>)}) {
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
  // All NWG workgroups must be resident at once. Each one needs a whole CU
  // (its LDS use exceeds half a CU's), ensure_device() checked that the GPU has
  // NWG such slots, and every inter-workgroup wait in the kernel ends in an
  // error after a bounded spin, so an ordinary launch is the default. The
  // cooperative launch (the reference's) is kept as an option, for comparison.
  void* args[] = {&P};
  const int inst = split_instance < 0 ? plan_instance(P.position) : split_instance;
  const void* kern = inst == 2   ? reinterpret_cast<const void*>(mq_decode_kernel<true, true>)
                     : inst == 1 ? reinterpret_cast<const void*>(mq_decode_kernel<true>)
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
                        int cache_len, int max_seq_len, float attn_scale, hipStream_t stream, bool noalloc,
                        int split_instance = -1) {
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
  return launch(P, stream, split_instance, noalloc);
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

extern "C" int mq_decode_variant(int variant, int input_token_id, int* output_token_id, float* logits_output,
                                 const void* embed_weight, const LDGLayerWeights* layer_weights,
                                 const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                                 const void* sin_table, void* k_cache, void* v_cache, void* hidden_buffer,
                                 void* g_normalized, int num_layers, int position, int cache_len, int max_seq_len,
                                 float attn_scale, hipStream_t stream) {
  // variant -> kernel instance: baseline picks per step, unsplit is instance 0 (contexts of
  // at most KV_CAP positions only), split is instance 1, or 2 where a chunk takes more than
  // one LDS pass
  int inst = -1;
  if (variant == MQ_VARIANT_UNSPLIT) {
    if (position < 0 || position >= KV_CAP) return MQ_ERR_ARG;
    inst = 0;
  } else if (variant == MQ_VARIANT_SPLIT) {
    if (position < 0 || position >= MAX_CTX) return MQ_ERR_ARG;
    inst = plan_instance(position) == 0 ? 1 : plan_instance(position);
  } else if (variant != MQ_VARIANT_BASELINE) {
    return MQ_ERR_ARG;
  }
  return decode_entry(input_token_id, output_token_id, logits_output, embed_weight, layer_weights, final_norm_weight,
                      lm_head_weight, cos_table, sin_table, k_cache, v_cache, hidden_buffer, g_normalized, num_layers,
                      position, cache_len, max_seq_len, attn_scale, stream, false, inst);
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
  const MqDecodeStep h{token, position, 0u, 0};
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
      split_instance < 0 || split_instance > 2)
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
  if (instance) *instance = plan_instance(position);
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
  // the no-allocation entry point's workspace (`scratch`, through its device address) as well,
  // once that entry point has set it up on this device (a synchronous memset allocates nothing)
  uint32_t* na = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_noalloc[device].init && g_noalloc[device].status == MQ_OK) na = g_noalloc[device].ptr;
  }
  if (e == hipSuccess && na) e = hipMemset(na, 0, sizeof(uint32_t) * WS_WORDS);
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
