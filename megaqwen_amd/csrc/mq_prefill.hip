// Prefill of S prompt tokens for Qwen3-0.6B on MI355X (gfx950).
//
// Replaces launch_prefill_float (csrc/megakernel/fused_prefill.cu:601-867): the
// prompt's hidden states go through every layer as [S, *] bf16 matrices, K/V
// slots 0..S-1 of every layer are written, and the greedy next token is taken
// from the last row. After embed_rows and the first layer's rmsnorm_rows, per layer:
//   gemm_nt (q, k, v in one launch; its epilogue applies QK-norm and RoPE and appends K/V)
//   -> attn_prefill or, past 1024 tokens, attn_prefill_fa3, past 5120 attn_prefill_fa2 (causal, MFMA)
//   -> gemm_nt (o_proj, k split four ways)
//   -> resid_norm_rows (partials + residual, post-attention RMSNorm)
//   -> gemm_nt (gate and up, SiLU(gate) * up epilogue) -> gemm_nt (down_proj, k split)
//   -> resid_norm_rows (partials + residual, the next layer's input RMSNorm)
// then lm_partial (final norm of the last row, tied LM head, per-block argmax) and
// argmax_final. The GEMMs run on v_mfma_f32_16x16x32_bf16 with fp32 accumulation.
//
// The intermediates, the fp32 partial sums included, live in the caller's scratch
// buffers (the reference's own argument list), so a launch allocates nothing.
//
// Numerics are HF Qwen3's bf16 rounding points, as in the decode kernel. The
// attention reproduces torch's CPU flash kernel (the sdpa path HF runs on the
// CPU): scores in fp32, keys in blocks of 512 with a running maximum, exp in
// fp32 summed unrounded, probabilities rounded to bf16 before P.V, output
// bf16(acc * (1 / sum)).

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "megaqwen_amd.h"
#include "mq_common.h"

// Instrumentation hook of a tracing build: MQ_PF_STAMP(slot) marks a point of a kernel's
// timeline; it compiles to nothing unless a tracing harness defines it first.
#ifndef MQ_PF_STAMP
#define MQ_PF_STAMP(i) ((void)0)
#endif

namespace mq {

int current_workspace(uint32_t** ws);  // mq_decode.hip: this device's library workspace

namespace pf {

// ------------------------------------------------------------------ GEMM
// C[m, n] = sum_k A[m, k] * W[n, k] (both operands k-contiguous, HF nn.Linear
// layout), one TM x TN output tile per workgroup, k in steps of 64.
//
// Operand tiles move from global memory straight into LDS (global_load_lds_dwordx4,
// no register staging) through NST LDS stages, so NST - 1 stages are in flight
// while one is multiplied. A stage holds KS consecutive 64-wide k-steps, each as the
// A tile (TM rows) and then the B tile (TN rows), each row as eight 16-byte chunks
// XOR-swizzled with the row, so that the 8 rows a quarter-wave reads in one fragment
// load fall in distinct banks. A DMA instruction writes 64 consecutive chunk slots
// (lane l -> slot base + l), so the swizzle is applied on the source side: the lane
// that owns slot s fetches the chunk that belongs there.
//
// The WM x WN waves tile the output: wave (wm, wn) owns TM / WM rows and TN / WN
// columns, as 16 x 16 MFMA blocks. A launch streams M N K 2 (1 / TM + 1 / TN) operand
// bytes from L2 into the CUs, so tiles are large (128 rows), and the N = 1024 products
// split k over blockIdx.z (EPI_PART: fp32 partial sums, added up by the row kernel
// that follows) so that their grid still fills the 256 CUs.
constexpr int TK = 64;

enum : int { EPI_STORE = 0, EPI_SILU = 1, EPI_PART = 2, EPI_QKN = 3, EPI_RESADD = 4 };
// EPI_RESADD: the product's k range is summed as four consecutive quarters, each its own
// MFMA chain from zero, added in quarter order (((q0 + q1) + q2) + q3) -- the same sums as a
// four-way k split whose fp32 partials resid_norm_rows adds in split order -- and the
// epilogue applies the residual add out = bf16(out + bf16(sum)) in place
constexpr int RES_QUARTERS = 4;

struct GemmSeg {
  const uint16_t* w;   // weight rows [n, k]; EPI_SILU: gate_proj rows
  const uint16_t* w2;  // EPI_SILU: up_proj rows
  uint16_t* out;       // [m, ldo] bf16
  int ntiles;          // column tiles of this segment (EPI_SILU: TN / 2 units each)
  int ldo;
};
// EPI_PART output: the fp32 partial sums of one k split over a [m, 1024] output, as two
// 512-column halves, each with its own base and row pitch (in floats), so that a set
// can live in one [m, 1024] fp32 buffer (hi = lo + 512, ld = 1024) or in two buffers of
// 2 KB rows (ld = 512)
constexpr int MAX_SPLIT = 4, PART_HALF = 512;
struct PartSet {
  float* lo[MAX_SPLIT];
  float* hi[MAX_SPLIT];
  int ld[MAX_SPLIT];
  int n;
};
// EPI_QKN: the q, k, v segments' tiles are whole heads; the epilogue applies QK-norm and
// RoPE to q and k and writes q to `q_out` and k, v to the caches at slot = row
struct QknArgs {
  const uint16_t *qn, *kn, *cos_t, *sin_t;
  uint16_t *q_out, *kc, *vc;
  int max_seq;
};
// Tile order across XCDs. The hardware deals workgroup L (linear id within the grid) to
// XCD L % 8, and each XCD has its own L2, so the tiles that share an operand should run on
// one XCD. With `xg` > 0 the grid's tiles (per k split) are dealt as 8 rectangles, 8 / xg
// row bands by xg column bands, one per XCD class L % 8; inside its rectangle an XCD takes
// panels of `xp` row tiles, column by column inside a panel (row tile fastest), so the
// workgroups that run together (one panel) share xp A row tiles and a run of W tiles, and
// each A row tile comes from HBM once per XCD instead of once per XCD for every column
// band. xg = 0: blockIdx order (column tile = blockIdx.x). Either order computes every
// tile the same way.
struct XcdMap {
  int xg, xp;
};
// Cache warm-up by workgroups that no tile uses. A launch that leaves CUs idle (gate/up at
// S = 512 has 192 workgroups for 256 CUs) appends one row of workgroups (blockIdx.y ==
// `row`) that read the weights of the launches after it, each column tile of a consumer on
// the XCD that will read it: in blockIdx order with a multiple of 8 column tiles, a
// consumer's column tile t runs on XCD t % 8 whatever its row tile and k split. Nothing is
// stored: the reads leave the rows in that XCD's L2 and in the memory-side cache, and the
// product's own tiles run on other CUs, so their loads do not queue behind these. The set is
// the second argument of its own kernel (gemm_nt_warm), not a field of GemmArgs: with it in
// every launch's argument block the launches without a warm-up row ran slower (whole
// prefill, same box: S = 300 1.779 -> 1.807 ms, 512 1.962 -> 1.992).
constexpr int MAX_WARM = 5, NUM_CUS = 256;  // (MI355X: 8 XCDs of 32 CUs)
// Prompts up to this length warm in gate/up (whole prefill, same box, without -> with the
// warm-up: S = 64 1.465 -> 1.408 ms, 128 1.511 -> 1.474, 256 1.675 -> 1.639, 288 1.755 ->
// 1.730, 352 1.804 -> 1.760, 384 1.839 -> 1.782; from 385 tokens gate/up has 192 tile
// workgroups, and with the warm-up row S = 400 measured 1.794 -> 1.801, 512 1.930 -> 1.927)
constexpr int WARM_MAX_S = 384;
struct WarmSet {
  const uint16_t* w[MAX_WARM];  // weight matrices [n, k] bf16, in the order they are read
  int tile_bytes[MAX_WARM];     // bytes of one consumer column tile (a multiple of 1 KB)
  int ntiles[MAX_WARM];         // the consumer's column tiles in this matrix
  int xcd0[MAX_WARM];           // XCD of the matrix's first tile (its first tile index mod 8)
  int n;                        // ranges; 0: no warm-up row
  int row;                      // blockIdx.y of the warm-up row (set by the launcher)
};
struct GemmArgs {
  const uint16_t* a;  // [m, lda] bf16
  int lda, m, k;
  GemmSeg seg[3];  // q/k/v: q, k, v; the others: one
  PartSet part;  // EPI_PART: set z takes the partial sums of k split z (blockIdx.z)
  QknArgs qkn;   // EPI_QKN
  XcdMap xm;
};
// One launch's argument block: only the fields its epilogue reads (q/k/v: three segments
// and the QK-norm/RoPE block, 200 bytes; the k-split products: one segment and the
// partial-sum set, 160; the others: one segment, 72). The whole GemmArgs (280 bytes) in
// every launch ran slower (whole prefill, same box: S = 128 1.422 -> 1.401 ms, 512
// 1.958 -> 1.946, 2048 5.333 -> 5.329; same bits). The grid's size comes in the block
// too: a kernel that reads gridDim gets the 256 bytes of hidden arguments appended to its
// block (S = 128 1.402 -> 1.395 ms, 512 1.954 -> 1.937 without them, the attention
// kernels' likewise).
template <int EPI> struct EpiBlock {};
template <> struct EpiBlock<EPI_PART> { PartSet part; };
template <> struct EpiBlock<EPI_QKN> { QknArgs qkn; };
template <int EPI>
struct KernArgs : EpiBlock<EPI> {
  static constexpr int NSEG = EPI == EPI_QKN ? 3 : 1;
  const uint16_t* a;
  int lda, m, k;
  XcdMap xm;
  int nx, ny, kp;  // the grid's column tiles and row tiles (no warm-up row), k per split
  GemmSeg seg[NSEG];
};
static_assert(sizeof(KernArgs<EPI_SILU>) == 72 && sizeof(KernArgs<EPI_PART>) == 160 &&
              sizeof(KernArgs<EPI_QKN>) == 200, "the argument block sizes stated above");

// The warm-up row's work. Its gridDim.x / 8 workgroups on XCD c (linear id L, L % 8 == c;
// the launcher keeps gridDim.x a multiple of 8 and one k split) split every tile t with
// (xcd0 + t) % 8 == c into equal runs of 1 KB units; a wave reads one unit per DMA (64
// lanes x 16 bytes) into its own 1 KB of the workgroup's LDS, which nothing reads.
template <int NW>
__device__ void warm_tiles(const WarmSet& W, int nx, uint32_t lds, int wv, int lane) {
  const int L = blockIdx.x + nx * blockIdx.y, c = L & 7;
  const int nwg = nx >> 3, j = (L >> 3) - (nx >> 3) * W.row;
  const uint32_t dst = __builtin_amdgcn_readfirstlane(lds + 1024u * (uint32_t)wv);
#pragma unroll
  for (int r = 0; r < MAX_WARM; r++) {
    if (r >= W.n) break;
    const int units = W.tile_bytes[r] >> 10, u0 = units * j / nwg, u1 = units * (j + 1) / nwg;
    for (int t = (c - W.xcd0[r]) & 7; t < W.ntiles[r]; t += 8) {
      const char* base = reinterpret_cast<const char*>(W.w[r]) + (size_t)t * W.tile_bytes[r] + 16 * lane;
      for (int u = u0 + wv; u < u1; u += NW) dma16(base + ((size_t)u << 10), dst);
    }
  }
  wait_vmem();  // no DMA may still target this workgroup's LDS when it exits
}

// LDS slot (in 16-byte chunks) of chunk kc (0..7) of tile row r.
__device__ __forceinline__ int tslot(int r, int kc) { return r * 8 + (kc ^ (r & 7)); }

template <int EPI, int TM, int TN, int NST, int KS, int WM, int WN, bool WARM>
__device__ __forceinline__ void gemm_tiles(const KernArgs<EPI>& G, const WarmSet* W) {
  constexpr int NW = WM * WN, NT = 64 * NW;
  constexpr int RB = TM / (16 * WM);      // 16-row blocks per wave
  constexpr int CB = TN / (16 * WN);      // 16-column blocks per wave
  constexpr int HB = TN / 32;             // EPI_SILU: gate (and up) blocks per tile
  constexpr int ACH = TM * 8, BCH = TN * 8;  // chunk slots of the A and B tiles
  constexpr int SCH = ACH + BCH;          // slots per k-step
  constexpr int NI = KS * SCH / NT;       // DMA instructions per thread and stage
  static_assert(RB * 16 * WM == TM && CB * 16 * WN == TN, "waves tile the output");
  static_assert(EPI != EPI_SILU || CB % 2 == 0, "a wave pairs each gate block with its up block");
  static_assert(ACH % 64 == 0 && BCH % 64 == 0 && (KS * SCH) % NT == 0,
                "a DMA instruction covers 64 slots of one operand of one k-step");
  __shared__ u32x4 sbuf[NST][KS][SCH];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, wm = wv / WN, wn = wv % WN;
  if (WARM && (int)blockIdx.y == W->row) {
    static_assert(NW * 1024 <= NST * KS * SCH * 16, "a wave's DMA unit fits the ring");
    warm_tiles<NW>(*W, G.nx, (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&sbuf[0][0][0], wv, lane);
    return;
  }
  int nt = blockIdx.x, mt = blockIdx.y;  // column tile, row tile
  const int z = blockIdx.z;               // k split
  if (G.xm.xg > 0) {
    // (the host sets xg only when 8 divides the tile count, xg the column tiles, 8 / xg the
    // row tiles and xp the row tiles of a band)
    const int nx = G.nx, L = blockIdx.x + nx * blockIdx.y, c = L & 7, s = L >> 3;
    const int cw = nx / G.xm.xg, rh = G.ny / (8 / G.xm.xg), pn = G.xm.xp * cw;
    const int r = s / pn * G.xm.xp + s % pn % G.xm.xp, cc = s % pn / G.xm.xp;
    mt = c / G.xm.xg * rh + r;
    nt = c % G.xm.xg * cw + cc;
  }
  int si = 0;
  if constexpr (KernArgs<EPI>::NSEG > 1)
    while (si + 1 < KernArgs<EPI>::NSEG && nt >= G.seg[si].ntiles) nt -= G.seg[si++].ntiles;
  const GemmSeg S = G.seg[si];
  const int m0 = mt * TM;
  const int kp = G.kp, kz = kp * z;  // this split's k range
  const int KT = kp / (TK * KS);

  // the wave's column blocks; EPI_SILU: blocks j < CB / 2 are gate blocks, each paired with
  // the up block j + CB / 2 (gate rows are the tile's first TN / 2 rows, up rows the rest)
  int jb[CB];
#pragma unroll
  for (int j = 0; j < CB; j++)
    jb[j] = EPI == EPI_SILU ? (j < CB / 2 ? (CB / 2) * wn + j : HB + (CB / 2) * wn + j - CB / 2) : CB * wn + j;

  // DMA instruction i of this wave fills the 64 slots 64 b .. 64 b + 63 of a stage,
  // b = NW i + wv, counted over the stage's KS k-steps
  const uint16_t* src[NI];
  uint32_t dst[NI];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&sbuf[0][0][0];
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int b0 = 64 * (NW * i + wv), q = b0 / SCH, s0 = b0 % SCH, sl = s0 + lane;
    dst[i] = __builtin_amdgcn_readfirstlane(lds0 + 16u * (uint32_t)b0);  // wave-uniform (M0)
    const uint16_t* p;
    if (s0 < ACH) {
      const int r = sl >> 3, kc = (sl & 7) ^ (r & 7);
      const int row = min(m0 + r, G.m - 1);  // rows past the prompt repeat its last row (never stored)
      p = G.a + (size_t)row * G.lda + 8 * kc;
    } else {
      const int t = sl - ACH, r = t >> 3, kc = (t & 7) ^ (r & 7);
      if (EPI == EPI_SILU)
        p = (r < TN / 2 ? S.w + (size_t)(TN / 2 * nt + r) * G.k : S.w2 + (size_t)(TN / 2 * nt + r - TN / 2) * G.k) +
            8 * kc;
      else
        p = S.w + (size_t)(TN * nt + r) * G.k + 8 * kc;
    }
    src[i] = p + kz + TK * q;
  }
  // stage kt % NST <- k-steps KS kt .. KS kt + KS - 1 of the split; steps past the end
  // re-load the last ones (kept uniform so that every wave issues the same number of DMAs
  // and the vmcnt waits below are exact)
  auto issue = [&](int kt) {
    const int kk = min(kt, KT - 1) * TK * KS;
    const uint32_t so = 16u * (uint32_t)(KS * SCH * (kt % NST));
#pragma unroll
    for (int i = 0; i < NI; i++) dma16(src[i] + kk, dst[i] + so);
  };

  f32x4 acc[RB][CB];
#pragma unroll
  for (int i = 0; i < RB; i++)
#pragma unroll
    for (int j = 0; j < CB; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // EPI_RESADD: the sum of the quarters done so far
  f32x4 tot[EPI == EPI_RESADD ? RB : 1][EPI == EPI_RESADD ? CB : 1];
  const int kq = KT / RES_QUARTERS;  // k-steps (of TK * KS) per quarter
#pragma unroll
  for (int kt = 0; kt < NST - 1; kt++) issue(kt);
  for (int kt = 0; kt < KT; kt++) {
    // this wave's DMAs of stage kt have landed (the NST - 2 later stages may still fly);
    // the barrier publishes every wave's, and tells that stage kt - 1 is free
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NST - 2) * NI) : "memory");
    __syncthreads();
    issue(kt + NST - 1);
#pragma unroll
    for (int q = 0; q < KS; q++) {
      const u32x4* sa = sbuf[kt % NST][q];
      const u32x4* sb = sa + ACH;
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const int kc = 4 * ks + (lane >> 4), r = lane & 15;
        u32x4 bf[CB];
#pragma unroll
        for (int j = 0; j < CB; j++) bf[j] = sb[tslot(16 * jb[j] + r, kc)];
#pragma unroll
        for (int i = 0; i < RB; i++) {
          const u32x4 af = sa[tslot(16 * (RB * wm + i) + r, kc)];
#pragma unroll
          for (int j = 0; j < CB; j++) acc[i][j] = mfma_16x16x32(af, bf[j], acc[i][j]);
        }
      }
    }
    if constexpr (EPI == EPI_RESADD) {
      if ((kt + 1) % kq == 0) {
        // a quarter ends: fold it into the running sum (the first one is the sum) and
        // start the next quarter's chain from zero
        const bool first = kt + 1 == kq;
#pragma unroll
        for (int i = 0; i < RB; i++)
#pragma unroll
          for (int j = 0; j < CB; j++) {
            tot[i][j] = first ? acc[i][j] : tot[i][j] + acc[i][j];
            acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
      }
    }
  }
  wait_vmem();  // no DMA may still target this workgroup's LDS when it exits

  // lane holds rows 4 * (lane / 16) + e of column lane % 16 of each block
  const int col = lane & 15, rq = 4 * (lane >> 4);
  if constexpr (EPI == EPI_QKN && TN == 2 * HD) {
    // Two heads a tile (long prompts: 256 x 256 tiles on sixteen waves): both heads'
    // bf16-rounded outputs go through LDS as bf16 (exact, the values being bf16), [2][TM][HD]
    // with each row's 16-byte chunks in slots chunk ^ (row % 16), so that the whole tile fits
    // the ring and every accumulator is dead before the rows are processed; then each row of
    // both heads is processed as in the one-head epilogue below, term for term (the norm
    // weights and the row's cos/sin loaded once for both heads).
    constexpr int RPI = 8 * NW, NPASS = TM / RPI;
    static_assert(2 * TM * HD * 2 <= NST * KS * SCH * 16 && TM % RPI == 0, "both heads' rows fit the ring");
    uint16_t* tile = reinterpret_cast<uint16_t*>(&sbuf[0][0][0]);
    auto slot = [](int hh, int r, int d) { return (hh * TM + r) * HD + 8 * ((d >> 3) ^ (r & 15)) + (d & 7); };
    __syncthreads();  // every wave is past its last read of the ring
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int j = 0; j < CB; j++) {
          const int c = 16 * jb[j] + col;
          tile[slot(c >> 7, 16 * (RB * wm + i) + rq + e, c & (HD - 1))] = (uint16_t)f2bf(acc[i][j][e]);
        }
    __syncthreads();
    const QknArgs& Q = G.qkn;
    const int pd = 8 * (lane & 7), rr = lane >> 3;
    auto bf8 = [](const u32x4 v, float (&f)[8]) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        f[2 * e] = bf2f(v[e] & 0xffffu);
        f[2 * e + 1] = bf2f(v[e] >> 16);
      }
    };
    if (si == 2) {
      // v rows: a copy
#pragma unroll
      for (int it = 0; it < NPASS; it++) {
        const int r = RPI * it + 8 * wv + rr, t = m0 + r;
        if (t >= G.m) continue;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
          uint16_t* dst = Q.vc + ((size_t)(2 * nt + hh) * Q.max_seq + t) * HD;
          *reinterpret_cast<u32x4*>(dst + pd) = *reinterpret_cast<const u32x4*>(tile + slot(hh, r, pd));
          *reinterpret_cast<u32x4*>(dst + 64 + pd) = *reinterpret_cast<const u32x4*>(tile + slot(hh, r, 64 + pd));
        }
      }
      return;
    }
    const uint16_t* nwp = si == 0 ? Q.qn : Q.kn;
    float w1[8], w2[8];
    bf8(ldw(nwp + pd), w1);
    bf8(ldw(nwp + 64 + pd), w2);
    u32x4 cs[NPASS][4];
#pragma unroll
    for (int it = 0; it < NPASS; it++) {
      const size_t t = (size_t)min(m0 + RPI * it + 8 * wv + rr, G.m - 1) * HD;  // rows past the prompt: never stored
      cs[it][0] = ldw(Q.cos_t + t + pd);
      cs[it][1] = ldw(Q.cos_t + t + 64 + pd);
      cs[it][2] = ldw(Q.sin_t + t + pd);
      cs[it][3] = ldw(Q.sin_t + t + 64 + pd);
    }
#pragma unroll
    for (int it = 0; it < NPASS; it++) {
      const int r = RPI * it + 8 * wv + rr, t = m0 + r;
      float c1[8], c2[8], s1[8], s2[8];
      bf8(cs[it][0], c1);
      bf8(cs[it][1], c2);
      bf8(cs[it][2], s1);
      bf8(cs[it][3], s2);
#pragma unroll
      for (int hh = 0; hh < 2; hh++) {
        float x1[8], x2[8];
        bf8(*reinterpret_cast<const u32x4*>(tile + slot(hh, r, pd)), x1);
        bf8(*reinterpret_cast<const u32x4*>(tile + slot(hh, r, 64 + pd)), x2);
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = x1[e] * x1[e] + x2[e] * x2[e];
        float ss = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        ss += dpp<0xB1>(ss);
        ss += dpp<0x4E>(ss);
        ss += dpp<0x141>(ss);
        const float rstd = 1.0f / sqrtf(ss * (1.0f / HD) + EPS);
        uint32_t o1[4], o2[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float r1[2], r2[2];
#pragma unroll
          for (int u = 0; u < 2; u++) {
            const float n1 = rbf(w1[e + u] * rbf(x1[e + u] * rstd)), n2 = rbf(w2[e + u] * rbf(x2[e + u] * rstd));
            r1[u] = rbf(rbf(n1 * c1[e + u]) - rbf(n2 * s1[e + u]));
            r2[u] = rbf(rbf(n2 * c2[e + u]) + rbf(n1 * s2[e + u]));
          }
          o1[e / 2] = pack_bf2(r1[0], r1[1]);
          o2[e / 2] = pack_bf2(r2[0], r2[1]);
        }
        if (t >= G.m) continue;
        const int h = 2 * nt + hh;
        uint16_t* dst = si == 0 ? Q.q_out + (size_t)t * QS + HD * h : Q.kc + ((size_t)h * Q.max_seq + t) * HD;
        *reinterpret_cast<u32x4*>(dst + pd) = u32x4{o1[0], o1[1], o1[2], o1[3]};
        *reinterpret_cast<u32x4*>(dst + 64 + pd) = u32x4{o2[0], o2[1], o2[2], o2[3]};
      }
    }
    return;
  }
  if constexpr (EPI == EPI_QKN && TN == HD) {
    // QK-norm (per head over 128, weights q_norm/k_norm) and RoPE (modeling_qwen3.py:247-257,
    // rotate_half form, three bf16 ops) of the tile's rows, which are tokens m0.. of head
    // nt of segment si (q, k or v); per token the reference's ldg_qk_norm_rope_cache
    // (fused_decode_ldg.cu:166-276) for a whole prompt. The bf16-rounded outputs go through
    // LDS ([TM][QP] fp32: the pitch puts the 64 lanes of a fragment store in 64 banks and keeps
    // rows 16-byte aligned); then eight lanes take a row, lane p of them dims 8 p .. 8 p + 7
    // and their rotation partners 64 + 8 p .. + 7, with 16-byte loads and stores.
    constexpr int QP = HD + 4, RPI = 8 * NW;  // tile pitch (floats); rows per pass of the workgroup
    static_assert(TN == HD && TM * QP * 4 <= NST * KS * SCH * 16 && TM % RPI == 0, "a tile is one head and fits the ring");
    float* tile = reinterpret_cast<float*>(&sbuf[0][0][0]);
    __syncthreads();  // every wave is past its last read of the ring
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int j = 0; j < CB; j++) tile[(16 * (RB * wm + i) + rq + e) * QP + 16 * jb[j] + col] = rbf(acc[i][j][e]);
    __syncthreads();
    const QknArgs& Q = G.qkn;
    const int h = nt, pd = 8 * (lane & 7), rr = lane >> 3;
    constexpr int NPASS = TM / RPI;
    auto bf8 = [](const u32x4 v, float (&f)[8]) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        f[2 * e] = bf2f(v[e] & 0xffffu);
        f[2 * e + 1] = bf2f(v[e] >> 16);
      }
    };
    if (si == 2) {
      // v rows: a copy (exact: the tile holds bf16 values)
#pragma unroll
      for (int it = 0; it < NPASS; it++) {
        const int r = RPI * it + 8 * wv + rr, t = m0 + r;
        if (t >= G.m) continue;
        const float* x = tile + r * QP;
        uint16_t* dst = Q.vc + ((size_t)h * Q.max_seq + t) * HD;
#pragma unroll
        for (int half = 0; half < 2; half++) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(x + 64 * half + pd);
          const f32x4 b = *reinterpret_cast<const f32x4*>(x + 64 * half + pd + 4);
          *reinterpret_cast<u32x4*>(dst + 64 * half + pd) =
              u32x4{pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3]), pack_bf2(b[0], b[1]), pack_bf2(b[2], b[3])};
        }
      }
      return;
    }
    // every pass's cos/sin and the norm weights first: one memory round trip
    const uint16_t* nwp = si == 0 ? Q.qn : Q.kn;
    float w1[8], w2[8];
    bf8(ldw(nwp + pd), w1);
    bf8(ldw(nwp + 64 + pd), w2);
    u32x4 cs[NPASS][4];
#pragma unroll
    for (int it = 0; it < NPASS; it++) {
      const size_t t = (size_t)min(m0 + RPI * it + 8 * wv + rr, G.m - 1) * HD;  // rows past the prompt: never stored
      cs[it][0] = ldw(Q.cos_t + t + pd);
      cs[it][1] = ldw(Q.cos_t + t + 64 + pd);
      cs[it][2] = ldw(Q.sin_t + t + pd);
      cs[it][3] = ldw(Q.sin_t + t + 64 + pd);
    }
#pragma unroll
    for (int it = 0; it < NPASS; it++) {
      const int r = RPI * it + 8 * wv + rr, t = m0 + r;
      const float* x = tile + r * QP;
      float x1[8], x2[8];
#pragma unroll
      for (int e = 0; e < 8; e += 4) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(x + pd + e);
        const f32x4 b = *reinterpret_cast<const f32x4*>(x + 64 + pd + e);
#pragma unroll
        for (int u = 0; u < 4; u++) {
          x1[e + u] = a[u];
          x2[e + u] = b[u];
        }
      }
      // sum of squares over the head in a fixed tree: v_d = x_d^2 + x_(d+64)^2, eight
      // consecutive d summed as ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)) in the lane,
      // then the eight lanes' sums as ((g0 + g1) + (g2 + g3)) + ((g4 + g5) + (g6 + g7)) by
      // xor 1, xor 2 and the half-row mirror (every lane of the row ends with the same sum)
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] = x1[e] * x1[e] + x2[e] * x2[e];
      float ss = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
      ss += dpp<0xB1>(ss);
      ss += dpp<0x4E>(ss);
      ss += dpp<0x141>(ss);
      const float rstd = 1.0f / sqrtf(ss * (1.0f / HD) + EPS);
      float c1[8], c2[8], s1[8], s2[8];
      bf8(cs[it][0], c1);
      bf8(cs[it][1], c2);
      bf8(cs[it][2], s1);
      bf8(cs[it][3], s2);
      uint32_t o1[4], o2[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float r1[2], r2[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const float n1 = rbf(w1[e + u] * rbf(x1[e + u] * rstd)), n2 = rbf(w2[e + u] * rbf(x2[e + u] * rstd));
          r1[u] = rbf(rbf(n1 * c1[e + u]) - rbf(n2 * s1[e + u]));
          r2[u] = rbf(rbf(n2 * c2[e + u]) + rbf(n1 * s2[e + u]));
        }
        o1[e / 2] = pack_bf2(r1[0], r1[1]);
        o2[e / 2] = pack_bf2(r2[0], r2[1]);
      }
      if (t >= G.m) continue;
      uint16_t* dst = si == 0 ? Q.q_out + (size_t)t * QS + HD * h : Q.kc + ((size_t)h * Q.max_seq + t) * HD;
      *reinterpret_cast<u32x4*>(dst + pd) = u32x4{o1[0], o1[1], o1[2], o1[3]};
      *reinterpret_cast<u32x4*>(dst + 64 + pd) = u32x4{o2[0], o2[1], o2[2], o2[3]};
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < RB; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int row = m0 + 16 * (RB * wm + i) + rq + e;
      if (row >= G.m) continue;
      if (EPI == EPI_RESADD) {
        // h = bf16(h + bf16(o)) (modeling_qwen3.py:316,322)
        uint16_t* hrow = S.out + (size_t)row * S.ldo + TN * nt;
#pragma unroll
        for (int j = 0; j < CB; j++) {
          const int cc = 16 * jb[j] + col;
          hrow[cc] = (uint16_t)f2bf(bf2f(hrow[cc]) + rbf(tot[i][j][e]));
        }
        continue;
      }
      if constexpr (EPI == EPI_PART) {
        static_assert(PART_HALF % TN == 0, "a tile lies in one column half");
        const int c0 = TN * nt;
        float* prow = (c0 < PART_HALF ? G.part.lo[z] : G.part.hi[z]) + (size_t)row * G.part.ld[z] + c0 % PART_HALF;
#pragma unroll
        for (int j = 0; j < CB; j++) prow[16 * jb[j] + col] = acc[i][j][e];
        continue;
      }
      uint16_t* orow = S.out + (size_t)row * S.ldo;
      if (EPI == EPI_SILU) {
        // HF Qwen3MLP (modeling_qwen3.py:81-83): down(bf16(silu(bf16 gate)) * bf16 up)
#pragma unroll
        for (int j = 0; j < CB / 2; j++) {
          const float g = rbf(acc[i][j][e]), u = rbf(acc[i][j + CB / 2][e]);
          const float sg = rbf(g / (1.0f + expf(-g)));
          orow[TN / 2 * nt + 16 * jb[j] + col] = (uint16_t)f2bf(sg * u);
        }
      } else {
#pragma unroll
        for (int j = 0; j < CB; j++) orow[TN * nt + 16 * jb[j] + col] = (uint16_t)f2bf(acc[i][j][e]);
      }
    }
}
template <int EPI, int TM, int TN, int NST, int KS, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN) gemm_nt(KernArgs<EPI> G) {
  gemm_tiles<EPI, TM, TN, NST, KS, WM, WN, false>(G, nullptr);
}
// the same product with a warm-up row of workgroups (blockIdx.y == W.row) after its tiles
template <int EPI, int TM, int TN, int NST, int KS, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN) gemm_nt_warm(KernArgs<EPI> G, WarmSet W) {
  gemm_tiles<EPI, TM, TN, NST, KS, WM, WN, true>(G, &W);
}

// ------------------------------------------------------------------ row-wise kernels
// Embedding rows of the prompt. An id outside the vocabulary sets the error word
// (reported as a negative token) and reads row 0.
__global__ void __launch_bounds__(128) embed_rows(const int* ids, const uint16_t* emb, uint16_t* h, uint32_t* err) {
  const int s = blockIdx.x;
  int id = ids[s];
  if (id < 0 || id >= VOCAB) {
    if (threadIdx.x == 0) __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    id = 0;
  }
  reinterpret_cast<u32x4*>(h + (size_t)s * H)[threadIdx.x] = ldw(emb + (size_t)id * H + 8 * threadIdx.x);
}

// HF Qwen3RMSNorm (modeling_qwen3.py:59-64) of each row: y = bf16(w * bf16(x * rstd)),
// rstd = 1 / sqrt(mean(x^2) + eps) in fp32. One single-wave workgroup per row.
__global__ void __launch_bounds__(64) rmsnorm_rows(const uint16_t* x, const uint16_t* w, uint16_t* y, int m) {
  const int row = blockIdx.x, lane = threadIdx.x;
  if (row < m) {
    const uint16_t* xr = x + (size_t)row * H;
    const u32x4 c[2] = {ldw(xr + 8 * lane), ldw(xr + 512 + 8 * lane)};
    const u32x4 wc[2] = {ldw(w + 8 * lane), ldw(w + 512 + 8 * lane)};
    float f[2][8];
    float ss = 0.f;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      unpack8(c[h], f[h]);
#pragma unroll
      for (int i = 0; i < 8; i++) ss = fmaf(f[h][i], f[h][i], ss);
    }
    ss = wave_sum(ss);
    const float rstd = 1.0f / sqrtf(ss * (1.0f / H) + EPS);
    uint16_t* yr = y + (size_t)row * H;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      float wf[8];
      unpack8(wc[h], wf);
      u32x4 o;
      o.x = pack_bf2(rbf(wf[0] * rbf(f[h][0] * rstd)), rbf(wf[1] * rbf(f[h][1] * rstd)));
      o.y = pack_bf2(rbf(wf[2] * rbf(f[h][2] * rstd)), rbf(wf[3] * rbf(f[h][3] * rstd)));
      o.z = pack_bf2(rbf(wf[4] * rbf(f[h][4] * rstd)), rbf(wf[5] * rbf(f[h][5] * rstd)));
      o.w = pack_bf2(rbf(wf[6] * rbf(f[h][6] * rstd)), rbf(wf[7] * rbf(f[h][7] * rstd)));
      reinterpret_cast<u32x4*>(yr + 512 * h)[lane] = o;
    }
  }
}

// The row step after a k-split residual product (o_proj or down_proj): the split's fp32
// partial sums of row r added in split order and rounded to bf16 (the Linear output),
// the residual add h = bf16(h + y) (modeling_qwen3.py:316,322), and, when w is given,
// the next RMSNorm of the new row into y_norm, as rmsnorm_rows computes it. One
// single-wave workgroup per row; lane l owns columns 8l .. 8l + 7 and 512 + 8l .. +7.
template <int NS>
__global__ void __launch_bounds__(64) resid_norm_rows(PartSet ps, uint16_t* h, const uint16_t* w, uint16_t* y, int m) {
  static_assert(2 * PART_HALF == H, "a partial set is two column halves");
  const int row = blockIdx.x, lane = threadIdx.x;
  if (row >= m) return;
  typedef const __attribute__((address_space(1))) f32x4 gf32x4;
  // every load first (the partials, the residual row, the norm weights): one memory
  // round trip for the row instead of one per partial set
  f32x4 pa[NS][2][2];
#pragma unroll
  for (int s = 0; s < NS; s++) {
    const float* half[2] = {ps.lo[s] + (size_t)row * ps.ld[s], ps.hi[s] + (size_t)row * ps.ld[s]};
#pragma unroll
    for (int hh = 0; hh < 2; hh++)
#pragma unroll
      for (int u = 0; u < 2; u++) pa[s][hh][u] = *(gf32x4*)(half[hh] + 8 * lane + 4 * u);
  }
  uint16_t* hr = h + (size_t)row * H;
  const u32x4 hc[2] = {ldw(hr + 8 * lane), ldw(hr + 512 + 8 * lane)};
  u32x4 wc[2] = {u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}};
  if (w) {
    wc[0] = ldw(w + 8 * lane);
    wc[1] = ldw(w + 512 + 8 * lane);
  }
  f32x4 a[2][2];
#pragma unroll
  for (int hh = 0; hh < 2; hh++)
#pragma unroll
    for (int u = 0; u < 2; u++) {
      a[hh][u] = pa[0][hh][u];
#pragma unroll
      for (int s = 1; s < NS; s++) a[hh][u] += pa[s][hh][u];  // split order
    }
  float f[2][8];
  float ss = 0.f;
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    float r[8];
    unpack8(hc[hh], r);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      f[hh][i] = rbf(r[i] + rbf(a[hh][i >> 2][i & 3]));
      ss = fmaf(f[hh][i], f[hh][i], ss);
    }
    u32x4 o;
    o.x = pack_bf2(f[hh][0], f[hh][1]);
    o.y = pack_bf2(f[hh][2], f[hh][3]);
    o.z = pack_bf2(f[hh][4], f[hh][5]);
    o.w = pack_bf2(f[hh][6], f[hh][7]);
    reinterpret_cast<u32x4*>(hr + 512 * hh)[lane] = o;
  }
  if (!w) return;
  ss = wave_sum(ss);
  const float rstd = 1.0f / sqrtf(ss * (1.0f / H) + EPS);
  uint16_t* yr = y + (size_t)row * H;
#pragma unroll
  for (int hh = 0; hh < 2; hh++) {
    float wf[8];
    unpack8(wc[hh], wf);
    u32x4 o;
    o.x = pack_bf2(rbf(wf[0] * rbf(f[hh][0] * rstd)), rbf(wf[1] * rbf(f[hh][1] * rstd)));
    o.y = pack_bf2(rbf(wf[2] * rbf(f[hh][2] * rstd)), rbf(wf[3] * rbf(f[hh][3] * rstd)));
    o.z = pack_bf2(rbf(wf[4] * rbf(f[hh][4] * rstd)), rbf(wf[5] * rbf(f[hh][5] * rstd)));
    o.w = pack_bf2(rbf(wf[6] * rbf(f[hh][6] * rstd)), rbf(wf[7] * rbf(f[hh][7] * rstd)));
    reinterpret_cast<u32x4*>(yr + 512 * hh)[lane] = o;
  }
}

// ------------------------------------------------------------------ causal attention
// Workgroup (q block, head h): query rows r0 .. r0+31 of head h against keys
// 0 .. min(S, r0 + 32) - 1 of KV head h / 2, in blocks of 512 keys. Per block:
// scores (MFMA) -> LDS; per-row max, exp and sum with the running maximum -> bf16
// probabilities in LDS; P.V on MFMA with the accumulator rescaled by exp(m_old - m_new).
//
// Eight waves. Scores: wave w takes keys 16 (w % 4) .. +15 of every other 64-key chunk
// (parity w / 4) and loads those K rows straight into registers as the MFMA operand, all
// four chunks' loads issued back to back before the first product (a short prompt's
// attention is latency-bound: one round trip for the whole block instead of one per
// chunk through an LDS ring); the scores go to LDS for the row-wise softmax (four rows a
// wave). P.V: wave w owns dims 16 w .. 16 w + 15. V rows reach LDS by 1 KB DMA instructions
// (four whole rows each): chunks 0..2 into three buffers at the block's start, chunks 3..6
// into the score rows' space once the softmax has read it, chunk 7 into buffer 0 once chunk
// 0 is consumed, so the whole block's V is in flight at once. A row's eight-dim chunk c sits
// in slot c ^ (row & 15), so the 16 rows of a fragment read hit distinct banks; P.V reads V
// with transpose reads (ds_read_b64_tr_b16), so V needs no transposed copy.
constexpr int AQ = 32;
constexpr int AKB = 512;
constexpr int ACK = 64;  // keys per LDS chunk
constexpr int AW = 8;    // waves a workgroup
// LDS row pitches: a P row is padded by 16 bytes so that the 16 rows a quarter-wave
// reads in one P.V fragment load fall in distinct bank groups (unpadded, 1 KB rows
// share their banks), and a score row by one word, which spreads the score writes
constexpr int SC_PITCH = AKB + 1, P_PITCH = AKB + 8;

__device__ __forceinline__ uint32_t akv_off(int row, int chunk) { return row * 256 + 16 * (chunk ^ (row & 15)); }

// exp(x) as 2^(x log2 e) on the hardware exp2 (v_exp_f32): about 2^-20 relative error for
// the arguments of the softmax (x <= 0), the accuracy class of the vectorised exp that
// torch's CPU flash-attention kernel uses (exp_u20); exp(-inf) = 0.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
// x, opaque to the compiler: a product passed through it is rounded on its own and never
// contracted with a later add into one fused multiply-add
__device__ __forceinline__ float unfused(float x) {
  asm("" : "+v"(x));
  return x;
}

// Rows k0 .. k0 + ACK - 1 of a K or V cache head (rows past klast repeat row klast) into
// the chunk buffer at LDS address `lds`: instruction q moves rows 4q .. 4q + 3, lane ->
// row 4q + lane / 16, slot lane % 16.
__device__ __forceinline__ void kv_chunk(const uint16_t* src, int k0, int klast, uint32_t lds, int wv, int lane) {
#pragma unroll
  for (int i = 0; i < ACK / 4 / AW; i++) {
    const int q = wv + AW * i, row = 4 * q + (lane >> 4), chunk = (lane & 15) ^ (row & 15);
    dma16(src + (size_t)min(k0 + row, klast) * HD + 8 * chunk, __builtin_amdgcn_readfirstlane(lds + 1024u * q));
  }
}
// Waits for this wave's chunk DMAs with at most n instructions still in flight, then a
// workgroup barrier (no vector-memory fence, so a prefetched chunk stays in flight).
#define AWAIT(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")
#define ABAR() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")

// TRIM (short prompts): the K loads, score products and exponentials stop at the block's
// last key instead of covering all 512 (the skipped scores are masked, so the sums and
// products are the same: same bits). Whole prefill, same box: S = 64 1.416 -> 1.368 ms, 128
// 1.462 -> 1.429, 256 1.636 -> 1.621; at S = 512 the branches cost more than they save
// (1.990 -> 2.015), so longer prompts keep the straight-line form.
template <bool TRIM>
__global__ void __launch_bounds__(64 * AW) attn_prefill(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                                                       uint16_t* out, int S, int max_seq, float scale) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  constexpr int RPW = AQ / AW;  // softmax rows per wave
  __shared__ float s_sc[AQ][SC_PITCH];
  __shared__ __align__(16) uint16_t s_p[AQ][P_PITCH];
  __shared__ __align__(16) uint8_t s_kv[3][ACK * 256];  // V chunk ring
  __shared__ float s_m[AQ], s_l[AQ], s_a[AQ];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // XCD-aware order: workgroup id runs on XCD id % 8, which is made the KV group g, so the
  // 32 workgroups reading one group's K/V rows share one L2; the longest query blocks
  // (the most keys) are dispatched first
  const int id = blockIdx.x, g = id & 7, r = id >> 3, h = 2 * g + (r & 1);
  const int r0 = ((S + AQ - 1) / AQ - 1 - (r >> 1)) * AQ;  // (the grid: NQ x that many blocks)
  const uint16_t* K = kc + (size_t)g * max_seq * HD;
  const uint16_t* V = vc + (size_t)g * max_seq * HD;
  const int nkey = min(S, r0 + AQ);
  const int r16 = lane & 15, kg = lane >> 4;
  const uint32_t kv0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_kv[0][0];
  MQ_PF_STAMP(0);
  // the scores: wave wv takes keys 16 (wv % 4) .. +15 of the chunks c with c % 2 == wv / 4
  const int kw = wv & 3, kpar = wv >> 2;

  u32x4 qf[2][4];
#pragma unroll
  for (int rb = 0; rb < 2; rb++) {
    const int row = r0 + 16 * rb + r16;
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
      qf[rb][ks] = ldw(q + (size_t)min(row, S - 1) * QS + HD * h + 32 * ks + 8 * kg);  // rows >= S: never stored
  }
  if (tid < AQ) {
    s_m[tid] = -INFINITY;
    s_l[tid] = 0.f;
  }
  f32x4 oacc[2];
#pragma unroll
  for (int rb = 0; rb < 2; rb++) oacc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int kb0 = 0; kb0 < nkey; kb0 += AKB) {
    const int kb1 = min(nkey, kb0 + AKB), nk = kb1 - kb0, nk32 = (nk + 31) & ~31;
    const int nch = (nk + ACK - 1) / ACK;
    // the block's first three V chunks into the three buffers, in flight during the scores
    // (issued before the K loads below, so they have landed once those have)
#pragma unroll
    for (int v = 0; v < 3; v++)
      if (v < nch) kv_chunk(V, kb0 + ACK * v, kb1 - 1, kv0 + v * ACK * 256, wv, lane);
    // ---- scores: the K rows go straight into registers as the MFMA operand (lane: key row
    // 16 kw + r16 of the chunk, dims 32 ks + 8 kg .. +7), all of the wave's chunks at once
    // (unconditional, past the block's keys too: those rows repeat its last key and their
    // scores are masked, and straight-line loads let the compiler keep them all in flight)
    u32x4 kf[AKB / ACK / 2][4];
#pragma unroll
    for (int i = 0; i < AKB / ACK / 2; i++) {
      const int c = 2 * i + kpar;
      if (TRIM && ACK * c >= nk) break;
      const int krow = min(kb0 + ACK * c + 16 * kw + r16, kb1 - 1);
#pragma unroll
      for (int ks = 0; ks < 4; ks++) kf[i][ks] = ldw(K + (size_t)krow * HD + 32 * ks + 8 * kg);
    }
    __builtin_amdgcn_sched_barrier(0);  // every K load issued before the first product
#pragma unroll
    for (int i = 0; i < AKB / ACK / 2; i++) {
      const int c = 2 * i + kpar;
      if (TRIM && ACK * c >= nk) break;  // (the unwritten score columns are past nk)
      {
        const int row = 16 * kw + r16, key = kb0 + ACK * c + row;
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
          f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ks++) a = mfma_16x16x32(qf[rb][ks], kf[i][ks], a);
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int rl = 16 * rb + 4 * kg + e;
            s_sc[rl][ACK * c + row] = (key <= r0 + rl && key < kb1) ? a[e] * scale : -INFINITY;
          }
        }
      }
    }
    ABAR();  // scores complete
    MQ_PF_STAMP(1);
    const int ncv = nk32 / ACK + ((nk32 & (ACK - 1)) != 0);
    // ---- softmax of rows RPW wv .. RPW wv + RPW - 1, all at once (the LDS reads of every
    // row are issued together and the reductions interleaved); lane takes keys lane + 64 u
    {
      float x[RPW][AKB / 64], mx[RPW], sum[RPW];
      const int nu = TRIM ? (nk + 63) >> 6 : AKB / 64;  // 64-key columns read
#pragma unroll
      for (int i = 0; i < RPW; i++)
#pragma unroll
        for (int u = 0; u < AKB / 64; u++) x[i][u] = u < nu ? s_sc[RPW * wv + i][lane + 64 * u] : -INFINITY;  // past nk: unused
#pragma unroll
      for (int i = 0; i < RPW; i++) {
        mx[i] = -INFINITY;
#pragma unroll
        for (int u = 0; u < AKB / 64; u++) mx[i] = fmaxf(mx[i], lane + 64 * u < nk ? x[i][u] : -INFINITY);
      }
      wave_max_n(mx);
#pragma unroll
      for (int i = 0; i < RPW; i++) {
        const int rl = RPW * wv + i;
        const float mn = fmaxf(s_m[rl], mx[i]);
        const float base = mn == -INFINITY ? 0.f : mn;
        sum[i] = 0.f;
        // branch-free: every lane evaluates all eight keys and selects 0 past nk (adding
        // +0 leaves the sum unchanged; P.V reads s_p only below nk32)
#pragma unroll
        for (int u = 0; u < AKB / 64; u++) {
          if (u >= nu) break;  // (P.V reads s_p below nk32 <= 64 nu only)
          const int cc = lane + 64 * u;
          const float ev = exp_fast(x[i][u] - base);
          const float e = cc < nk ? ev : 0.f;
          sum[i] += e;
          s_p[rl][cc] = (uint16_t)f2bf(e);
        }
        mx[i] = mn;
      }
      wave_sum_n(sum);
      if (lane == 0)
#pragma unroll
        for (int i = 0; i < RPW; i++) {
          const int rl = RPW * wv + i;
          const float mo = s_m[rl], mn = mx[i], base = mn == -INFINITY ? 0.f : mn;
          const float al = mo == -INFINITY ? 0.f : expf(mo - base);
          s_m[rl] = mn;
          s_l[rl] = sum[i] + al * s_l[rl];
          s_a[rl] = al;
        }
    }
    ABAR();  // s_p, s_a; every wave is done with s_sc
    MQ_PF_STAMP(2);
    // V chunks 3..6 into the score rows' LDS, now dead (chunk 7 follows into buffer 0 once
    // chunk 0 is consumed): the whole block's V rows in flight at once
    const uint32_t scb = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_sc[0][0];
    auto vslot = [&](int c) { return c < 3 ? kv0 + c * ACK * 256 : c < 7 ? scb + (c - 3) * ACK * 256 : kv0; };
#pragma unroll
    for (int c = 3; c < 7; c++)
      if (c < ncv) kv_chunk(V, kb0 + ACK * c, kb1 - 1, vslot(c), wv, lane);
    // ---- P.V: wave wv owns dims 16 wv .. 16 wv + 15
#pragma unroll
    for (int rb = 0; rb < 2; rb++)
#pragma unroll
      for (int e = 0; e < 4; e++) oacc[rb][e] *= s_a[16 * rb + 4 * kg + e];
    static_assert(AKB / ACK == 8 && ACK / 4 / AW == 2, "the V schedule below assumes 8 chunks, 2 DMAs a wave each");
    for (int c = 0; c < ncv; c++) {
      // chunk c landed: chunks 0..2 before the K loads did; for c >= 3 every later chunk of
      // the block has been issued after it (chunk 7 at c = 1), two DMAs a wave each
      if (c >= 3) {
        switch (ncv - 1 - c) {
          case 4: AWAIT(8); break;
          case 3: AWAIT(6); break;
          case 2: AWAIT(4); break;
          case 1: AWAIT(2); break;
          default: AWAIT(0); break;
        }
      }
      ABAR();  // ... for every wave, which are also done with chunk c - 1's buffer
      if (c == 1 && ncv > 7) kv_chunk(V, kb0 + ACK * 7, kb1 - 1, vslot(7), wv, lane);
      const uint32_t vb = vslot(c);
      for (int kk = 0; kk < 2 && ACK * c + 32 * kk < nk32; kk++) {
        // B operand (8 keys of one dim per lane) from two transpose reads: within each
        // 16-lane group, lane j addresses key base + j / 4, dims 4 (j % 4) .. +3 of the
        // 16-dim block, and lane i receives that dim's 4 keys
        const int ra = 32 * kk + 8 * kg + (r16 >> 2);
        const int dq = 16 * wv + 4 * (r16 & 3);
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(uintptr_t)(vb + akv_off(ra, dq >> 3) + 2 * (dq & 7)));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(uintptr_t)(vb + akv_off(ra + 4, dq >> 3) + 2 * (dq & 7)));
        const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
        const u32x4 vf = u32x4{l2.x, l2.y, h2.x, h2.y};
#pragma unroll
        for (int rb = 0; rb < 2; rb++) {
          const u32x4 pfr = *reinterpret_cast<const u32x4*>(&s_p[16 * rb + r16][ACK * c + 32 * kk + 8 * kg]);
          oacc[rb] = mfma_16x16x32(pfr, vf, oacc[rb]);
        }
      }
    }
    ABAR();  // V buffers and s_p free for the next key block
    MQ_PF_STAMP(3);
  }
#pragma unroll
  for (int rb = 0; rb < 2; rb++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int rl = 16 * rb + 4 * kg + e, row = r0 + rl;
      if (row >= S) continue;
      const float inv = 1.0f / s_l[rl];
      out[(size_t)row * QS + HD * h + 16 * wv + r16] = (uint16_t)f2bf(oacc[rb][e] * inv);
    }
}

// ------------------------------------------------------------------ causal attention, flash forms
// Long prompts (attn_prefill_fa2, attn_prefill_fa3). A workgroup takes a block of query rows of
// both query heads of KV group g (2g, 2g + 1); a wave holds 16 query rows of both heads. Keys
// run in blocks of 512 (torch's CPU flash blocks) with a running maximum, as attn_prefill.
//
// Scores are computed transposed, S^T = K Q^T (K rows from LDS as the A operand, the wave's
// Q rows as the B operand, in registers): lane (r16, kg) holds the scores of query row r16
// against keys 16 t + 4 kg + e of key tile t. So the softmax of a query row is the lane's own
// plus a reduction over its four lane groups, and the bf16 probabilities are already the B
// operand of O^T = V^T P^T: keys 4 kg + i of tiles 2j, 2j + 1 (i < 4) form k-slots 8 kg + i
// of key step j, and V^T is read in the same key order by LDS transpose reads. No score or
// probability goes through LDS. K and V rows move into LDS in 64-key chunks (16 KB, 1 KB DMA
// instructions).
constexpr int FLASH_MIN_S = 1024;  // prompts longer than this take a flash form

__device__ __forceinline__ float lane_group_max(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float lane_group_sum(float v) {
  // (g0 + g2) + (g1 + g3) in every lane group, the same order everywhere
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// ------------------------------------------------------------------ causal attention, two passes
// Workgroup (KV group g, query block): query rows r0 .. r0 + 127 of both query heads of the
// group, eight waves of 16 rows each, every wave holding both heads' rows, so that each K
// or V fragment read from LDS feeds two MFMAs. Keys run in blocks of 512 (torch's CPU flash
// blocks) with a running maximum; a block's softmax needs its row maxima before any
// exponential, so each block is swept twice over its 64-key chunks: pass 1 computes the
// scores and keeps only the row maxima, pass 2 recomputes them, takes the bf16
// probabilities (held in registers as the B operand of O^T = V^T P^T) and runs that
// chunk's P.V at once. The sums, the P.V chains and the rescaling happen in the same order
// as in attn_prefill_fa3, so both give the same bits.
//
// LDS: the block's 512 K rows (128 KB, resident for both passes) and a two-chunk V ring
// (32 KB). During pass 2 the next block's K chunk c - 1 is copied into the slot that
// chunk c - 1 has just left, and V runs one chunk ahead, so pass 1 of the next block finds
// its K rows in place.
constexpr int F2W = 8, F2Q = 16 * F2W, F2KB = 512, F2K = 64, F2NC = F2KB / F2K;
// prompts longer than this take the two-pass form; shorter ones run faster on
// attn_prefill_fa3 (8 S / 64 workgroups against 8 S / 128; same-box timings: 5121 tokens
// 258 against 258 us, 5600 304 against 285, 8192 545 against 452); the two give the same bits
constexpr int FLASH2_MIN_S = 5120;
// V rows live in LDS with their own chunk swizzle, chunk c of row r in slot c ^ vsw_pf(r):
// a P.V transpose read takes, per half wave, rows 4 kg + i (kg < 2, i < 4, plus a multiple
// of 16) at chunks 2 dt and 2 dt + 1, and vsw_pf = 2 (r % 8) puts those 16 (row, chunk)
// pairs in 16 distinct slots, so the read is free of bank conflicts
__device__ __forceinline__ int vsw_pf(int row) { return 2 * (row & 7); }
__device__ __forceinline__ uint32_t vkv_off_pf(int row, int chunk) { return row * 256 + 16 * (chunk ^ vsw_pf(row)); }

__global__ void __launch_bounds__(64 * F2W) attn_prefill_fa2(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                                                              uint16_t* out, int S, int max_seq, float scale) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  __shared__ __align__(16) uint8_t s_k[F2NC][F2K * 256];
  __shared__ __align__(16) uint8_t s_v[2][F2K * 256];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // XCD-aware order: workgroup id runs on XCD id % 8, made the KV group; the longest query
  // blocks (the most keys) are dispatched first
  const int id = blockIdx.x, g = id & 7, nqb = (S + F2Q - 1) / F2Q;  // (the grid: 8 x nqb blocks)
  const int r0 = (nqb - 1 - (id >> 3)) * F2Q;
  const int r16 = lane & 15, kg = lane >> 4;
  const int row = r0 + 16 * wv + r16;  // this lane's query row
  const int wrow0 = r0 + 16 * wv, wrow1 = wrow0 + 15;  // the wave's query rows
  const int nkey = min(S, r0 + F2Q);
  const int nblk = (nkey + F2KB - 1) / F2KB;
  const uint16_t* K = kc + (size_t)g * max_seq * HD;
  const uint16_t* V = vc + (size_t)g * max_seq * HD;
  const uint32_t lk = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_k[0][0];
  const uint32_t lv = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_v[0][0];

  // rows base .. base + 63 of a K or V head (rows past klast repeat row klast) into the
  // chunk buffer at `lds`: instruction i moves rows 4 qq .. 4 qq + 3, qq = wv + 8 i (lane ->
  // row 4 qq + lane / 16, slot lane % 16, which holds the row's 16-byte chunk slot ^ row % 16)
  // (K rows in slots chunk ^ row % 16, V rows in slots chunk ^ vsw_pf(row); rows 4 qq + r and
  // 4 qq + 32 + r share both, so one source chunk offset serves both instructions)
  const int drow0 = 4 * wv + (lane >> 4);
  const int dchk_k = 8 * ((lane & 15) ^ (drow0 & 15)), dchk_v = 8 * ((lane & 15) ^ vsw_pf(drow0));
  const uint32_t dl0 = __builtin_amdgcn_readfirstlane(1024u * wv), dl1 = dl0 + 1024u * F2W;
  auto dma_chunk = [&](const uint16_t* src, int base, int klast, uint32_t lds) {
    const int dchk = src == K ? dchk_k : dchk_v;
    dma16(src + (size_t)min(base + drow0, klast) * HD + dchk, lds + dl0);
    dma16(src + (size_t)min(base + drow0 + 32, klast) * HD + dchk, lds + dl1);
  };
  auto klast_of = [&](int b) { return min(nkey, F2KB * b + F2KB) - 1; };

  // Q^T (B operand) of both heads: lane (row r16, kg) holds dims 32 ks + 8 kg .. +7 of its row
  u32x4 qf[2][4];
#pragma unroll
  for (int hh = 0; hh < 2; hh++)
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
      qf[hh][ks] = ldw(q + (size_t)min(row, S - 1) * QS + HD * (2 * g + hh) + 32 * ks + 8 * kg);
  f32x4 o[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; hh++)
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[hh][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

  // block 0's K rows and V chunk 0
  for (int c = 0; c < F2NC; c++) dma_chunk(K, F2K * c, klast_of(0), lk + (uint32_t)c * (F2K * 256));
  dma_chunk(V, 0, klast_of(0), lv);
  // (a compiler-visible wait: the q loads are then known complete on every path, so no
  // wait for them, which would also wait for the DMAs in flight, lands inside the loops)
  wait_vmem();
  ABAR();

  // LDS byte offsets of this lane's fragment reads: K (A operand) row 16 j + r16, 16-byte
  // chunk 4 ks + kg -> 4096 j + koff[ks]; V^T (transpose reads) rows 32 j2 + 4 kg + r16 / 4
  // (+ 16), dims 16 dt + 4 (r16 % 4) .. +3 -> 8192 j2 + voff[dt] (+ 4096)
  uint32_t koff[4], voff[8];
#pragma unroll
  for (int ks = 0; ks < 4; ks++) koff[ks] = lk + akv_off(r16, 4 * ks + kg);
#pragma unroll
  for (int dt = 0; dt < 8; dt++) {
    const int dq = 16 * dt + 4 * (r16 & 3);
    voff[dt] = vkv_off_pf(4 * kg + (r16 >> 2), dq >> 3) + 2 * (dq & 7);
  }

  // raw scores (q . k, unscaled) of key tile j (16 keys; lane: query row r16, keys
  // 16 j + 4 kg + e) of K chunk slot c, both heads. The products run at a raised wave
  // priority, so that the SIMD's other wave, in its exponentials or LDS reads, yields to
  // them (same bits; S = 8192 22.56 -> 22.31 ms, S = 6000 18.00 -> 17.78 ms on one box, three
  // rounds each; the same around the P.V products as well: 22.40 ms)
  auto raw_scores = [&](uint32_t kbase, int j, f32x4 (&a)[2]) {
    u32x4 kf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
      kf[ks] = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(kbase + 4096u * j + koff[ks]);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      a[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ks++) a[hh] = mfma_16x16x32(kf[ks], qf[hh][ks], a[hh]);
    }
    __builtin_amdgcn_s_setprio(0);
  };

  for (int b = 0; b < nblk; b++) {
    const int kb0 = F2KB * b, kb1 = min(nkey, kb0 + F2KB), nchb = (kb1 - kb0 + F2K - 1) / F2K;
    const bool more = b + 1 < nblk;
    // ---- pass 1: the block's row maxima, over the unscaled scores (scale > 0 and rounding
    // is monotonic, so max(a * scale) = max(a) * scale, both rounded)
    float mx[2] = {-INFINITY, -INFINITY};
    for (int c = 0; c < nchb; c++) {
      const uint32_t kbase = (uint32_t)c * (F2K * 256);
      const int ck0 = kb0 + F2K * c;  // the chunk's first key
      if (ck0 + F2K - 1 < kb1 && ck0 + F2K - 1 <= wrow0) {
        // no score of the chunk is masked
#pragma unroll
        for (int j = 0; j < 4; j++) {
          f32x4 a[2];
          raw_scores(kbase, j, a);
#pragma unroll
          for (int hh = 0; hh < 2; hh++)
            mx[hh] = fmaxf(fmaxf(mx[hh], fmaxf(a[hh][0], a[hh][1])), fmaxf(a[hh][2], a[hh][3]));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int key0 = ck0 + 16 * j;
          if (key0 <= wrow1) {
            f32x4 a[2];
            raw_scores(kbase, j, a);
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
              for (int e = 0; e < 4; e++) {
                const int key = key0 + 4 * kg + e;
                mx[hh] = fmaxf(mx[hh], (key < kb1 && key <= row) ? a[hh][e] : -INFINITY);
              }
          }
        }
      }
    }
    float base[2], al[2], sum[2] = {0.f, 0.f};
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const float mn = fmaxf(m_run[hh], lane_group_max(mx[hh]) * scale);
      base[hh] = mn == -INFINITY ? 0.f : mn;
      al[hh] = m_run[hh] == -INFINITY ? 0.f : expf(m_run[hh] - base[hh]);
      m_run[hh] = mn;
#pragma unroll
      for (int dt = 0; dt < 8; dt++) o[hh][dt] *= al[hh];
    }
    // ---- pass 2: probabilities and P.V, chunk by chunk
    for (int c = 0; c < F2NC; c++) {
      // V chunk c has landed (the later DMAs of this wave: the next block's K chunk c - 2,
      // issued after it); every wave is done with chunk c - 1
      if (c >= 2 && more) AWAIT(2);
      else if (c >= 1) AWAIT(0);
      ABAR();
      // V runs one chunk ahead (the next block's chunk 0 after chunk 7); the next block's K
      // chunk c - 1 goes into the slot chunk c - 1 has left
      if (c + 1 < F2NC) {
        if (more || c + 1 < nchb) dma_chunk(V, kb0 + F2K * (c + 1), kb1 - 1, lv + (uint32_t)((c + 1) & 1) * (F2K * 256));
      } else if (more) {
        dma_chunk(V, kb0 + F2KB, klast_of(b + 1), lv);
      }
      if (c >= 1 && more)
        dma_chunk(K, kb0 + F2KB + F2K * (c - 1), klast_of(b + 1), lk + (uint32_t)(c - 1) * (F2K * 256));
      if (c >= nchb) continue;
      const uint32_t kbase = (uint32_t)c * (F2K * 256);
      const int ck0 = kb0 + F2K * c;
      u32x2 pb[2][4];
      if (ck0 + F2K - 1 < kb1 && ck0 + F2K - 1 <= wrow0) {
        // no score of the chunk is masked
#pragma unroll
        for (int j = 0; j < 4; j++) {
          f32x4 a[2];
          raw_scores(kbase, j, a);
#pragma unroll
          for (int hh = 0; hh < 2; hh++) {
            float e4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
              e4[e] = exp_fast(unfused(a[hh][e] * scale) - base[hh]);
              sum[hh] += e4[e];
            }
            pb[hh][j] = u32x2{pack_bf2(e4[0], e4[1]), pack_bf2(e4[2], e4[3])};
          }
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int key0 = ck0 + 16 * j;
          if (key0 <= wrow1) {
            f32x4 a[2];
            raw_scores(kbase, j, a);
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
              float e4[4];
#pragma unroll
              for (int e = 0; e < 4; e++) {
                // the score a * scale, or -inf where masked (exp(-inf) = 0)
                const int key = key0 + 4 * kg + e;
                const float sv = (key < kb1 && key <= row) ? unfused(a[hh][e] * scale) : -INFINITY;
                e4[e] = exp_fast(sv - base[hh]);
                sum[hh] += e4[e];
              }
              pb[hh][j] = u32x2{pack_bf2(e4[0], e4[1]), pack_bf2(e4[2], e4[3])};
            }
          } else {
            pb[0][j] = pb[1][j] = u32x2{0u, 0u};
          }
        }
      }
      const uint32_t vb = lv + (uint32_t)(c & 1) * (F2K * 256);
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) {
        if (ck0 + 32 * j2 <= wrow1) {
          const u32x4 pf0 = u32x4{pb[0][2 * j2].x, pb[0][2 * j2].y, pb[0][2 * j2 + 1].x, pb[0][2 * j2 + 1].y};
          const u32x4 pf1 = u32x4{pb[1][2 * j2].x, pb[1][2 * j2].y, pb[1][2 * j2 + 1].x, pb[1][2 * j2 + 1].y};
#pragma unroll
          for (int dt = 0; dt < 8; dt++) {
            const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(vb + 8192 * j2 + voff[dt]));
            const v4s hi =
                __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(vb + 8192 * j2 + 4096 + voff[dt]));
            const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
            const u32x4 vf = u32x4{l2.x, l2.y, h2.x, h2.y};
            o[0][dt] = mfma_16x16x32(vf, pf0, o[0][dt]);
            o[1][dt] = mfma_16x16x32(vf, pf1, o[1][dt]);
          }
        }
      }
    }
#pragma unroll
    for (int hh = 0; hh < 2; hh++) l_run[hh] = lane_group_sum(sum[hh]) + al[hh] * l_run[hh];
    // the next block's K chunk 7 (every wave is done with slot 7), then all of its K rows
    // and its V chunk 0 in place
    ABAR();
    if (more) dma_chunk(K, kb0 + F2KB + F2K * (F2NC - 1), klast_of(b + 1), lk + (uint32_t)(F2NC - 1) * (F2K * 256));
    AWAIT(0);
    ABAR();
  }
  if (row < S) {
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const float inv = 1.0f / l_run[hh];
      uint16_t* op = out + (size_t)row * QS + HD * (2 * g + hh) + 4 * kg;
#pragma unroll
      for (int dt = 0; dt < 8; dt++)
        *reinterpret_cast<u32x2*>(op + 16 * dt) =
            u32x2{pack_bf2(o[hh][dt][0] * inv, o[hh][dt][1] * inv), pack_bf2(o[hh][dt][2] * inv, o[hh][dt][3] * inv)};
    }
  }
}

// ------------------------------------------------------------------ causal attention, scores kept
// Workgroup (KV group g, query block): query rows r0 .. r0 + 63 of both query heads of the
// group, four waves (one per SIMD) of 16 rows each, every wave holding both heads' rows. Keys
// run in blocks of 512 with a running maximum, as in attn_prefill_fa2, but each score is
// computed once: a wave keeps its whole block of scores in registers (2 heads x 512 keys x 16
// rows: 256 registers a lane, which one wave per SIMD can hold), takes the row maxima, then
// the probabilities and P.V chunk by chunk. The operations and their order are those of
// attn_prefill_fa2 (scores, maxima, exponentials, in-lane sums, P.V chains, rescaling), so the
// two give the same bits; this one does a third less MFMA work and reads K from LDS once per
// block instead of twice.
//
// LDS: the workgroup's Q rows (32 KB, both heads, read back at the start of every block, so
// that the Q fragments hold no registers while the probabilities and P.V run), and a ring of
// F3R chunk buffers (16 KB: 64 K or V rows) through which each block streams its K chunks and
// then its V chunks ("items"), F3R - 1 items in flight. Before item n a wave
// waits for its own DMAs of item n; the barrier that follows tells that every wave's have
// landed and that every wave is done with item n - 1, whose buffer then takes item n + F3R - 1.
// Past the last item the ring takes dummy copies (K row 0), so every wave issues the same
// number of DMAs before each wait and the vmcnt count stays exact.
constexpr int F3W = 4, F3Q = 16 * F3W, F3R = 8, F3I = 4;  // waves, query rows, ring, DMAs per item and wave
// A block's scores are parked in accumulation registers (AGPRs) once the maxima have read
// them, and brought back to VGPRs chunk by chunk for the exponentials (an empty asm with an
// AGPR / VGPR operand: the compiler moves the value there), so that the 256 registers of
// scores sit in the AGPR file and the VGPRs keep the operands, accumulators and addresses.
__device__ __forceinline__ f32x4 park_agpr(f32x4 x) {
  f32x4 r;
  asm("; park %0" : "=a"(r) : "0"(x));
  return r;
}
__device__ __forceinline__ f32x4 unpark_agpr(f32x4 x) {
  f32x4 r;
  asm("; unpark %0" : "=v"(r) : "0"(x));
  return r;
}

// Item n of attn_prefill_fa3's ring (see there) into its buffer. A function of scalars: as a
// lambda over the kernel's locals, the compiler kept the selected pointer and chunk offset in
// scratch memory and reloaded them behind the DMAs in flight (a full vmcnt wait per item).
__device__ __forceinline__ void fa3_issue(const uint16_t* K, const uint16_t* V, int dchk_k, int dchk_v, int drow,
                                          uint32_t dl, int n, int nitems, int nblk, int nclast, int nkey) {
  const uint16_t* src = K;
  int dchk = dchk_k, base = 0, kl = 0;
  if (n < nitems) {
    const int b = n >> 4, r = n & 15, nc = b + 1 < nblk ? F2NC : nclast;
    const bool isv = r >= nc;
    src = isv ? V : K;
    dchk = isv ? dchk_v : dchk_k;
    base = F2KB * b + F2K * (isv ? r - nc : r);
    kl = min(nkey, F2KB * b + F2KB) - 1;
  }
  const uint32_t lds = dl + (uint32_t)(n % F3R) * (F2K * 256);
#pragma unroll
  for (int i = 0; i < F3I; i++) dma16(src + (size_t)min(base + drow + 16 * i, kl) * HD + dchk, lds + 4096u * i);
}

__global__ void __launch_bounds__(64 * F3W) attn_prefill_fa3(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                                                              uint16_t* out, int S, int max_seq, float scale) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  __shared__ __align__(16) uint8_t s_ring[F3R][F2K * 256];
  __shared__ __align__(16) uint8_t s_q[2][F3Q * 256];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // XCD-aware order as attn_prefill_fa2: KV group = XCD, longest query blocks first
  const int id = blockIdx.x, g = id & 7, nqb = (S + F3Q - 1) / F3Q;  // (the grid: 8 x nqb blocks)
  const int r0 = (nqb - 1 - (id >> 3)) * F3Q;
  const int r16 = lane & 15, kg = lane >> 4;
  const int row = r0 + 16 * wv + r16;                  // this lane's query row
  const int wrow0 = r0 + 16 * wv, wrow1 = wrow0 + 15;  // the wave's query rows
  const int nkey = min(S, r0 + F3Q);
  const int nblk = (nkey + F2KB - 1) / F2KB;
  const int nclast = (nkey - F2KB * (nblk - 1) + F2K - 1) / F2K;  // chunks of the last block
  const int nitems = 2 * F2NC * (nblk - 1) + 2 * nclast;
  const uint16_t* K = kc + (size_t)g * max_seq * HD;
  const uint16_t* V = vc + (size_t)g * max_seq * HD;
  const uint32_t lr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_ring[0][0];

  // item n: block n / 16, then its K chunks (n % 16 < chunks of the block), then its V chunks.
  // DMA instruction i of wave wv moves rows 16 i + 4 wv + lane / 16 of the chunk, lane -> slot
  // lane % 16 of its row, which holds the row's source chunk slot ^ (row % 16) for K and
  // slot ^ vsw_pf(row) for V; row % 16 is the same for the four instructions.
  const int drow = 4 * wv + (lane >> 4);
  const int dchk_k = 8 * ((lane & 15) ^ drow), dchk_v = 8 * ((lane & 15) ^ vsw_pf(drow));
  const uint32_t dl = __builtin_amdgcn_readfirstlane(lr + 1024u * wv);
  auto issue = [&](int n) { fa3_issue(K, V, dchk_k, dchk_v, drow, dl, n, nitems, nblk, nclast, nkey); };

  // the Q rows into LDS: [head][row][16-byte chunk slot], chunk c of row r in slot c ^ (r % 16);
  // instruction i of wave wv moves rows 4 (wv + 4 i) .. +3 of the [2][64] rows, lane -> slot
  // lane % 16 of row 4 (wv + 4 i) + lane / 16
  const uint32_t lq = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_q[0][0];
#pragma unroll
  for (int i = 0; i < 2 * F3Q / 16; i++) {
    const int rr = 4 * (wv + 4 * i) + (lane >> 4), hh = rr / F3Q, qr = rr % F3Q;
    dma16(q + (size_t)min(r0 + qr, S - 1) * QS + HD * (2 * g + hh) + 8 * ((lane & 15) ^ (qr & 15)),
          __builtin_amdgcn_readfirstlane(lq + 1024u * (wv + 4 * i)));
  }
  f32x4 o[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; hh++)
#pragma unroll
    for (int dt = 0; dt < 8; dt++) o[hh][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  for (int n = 0; n < F3R - 1; n++) issue(n);
  wait_vmem();
  // (the barrier that starts item 0 publishes every wave's Q rows)

  // LDS byte offsets of this lane's fragment reads within a chunk buffer: K (A operand) row
  // 16 j + r16, 16-byte chunk 4 ks + kg -> 4096 j + koff[ks]; V^T (transpose reads) rows
  // 32 j2 + 4 kg + r16 / 4 (+ 16), dims 16 dt + 4 (r16 % 4) .. +3 -> 8192 j2 + voff[dt] (+ 4096)
  uint32_t koff[4], voff[8];
#pragma unroll
  for (int ks = 0; ks < 4; ks++) koff[ks] = akv_off(r16, 4 * ks + kg);
#pragma unroll
  for (int dt = 0; dt < 8; dt++) {
    const int dq = 16 * dt + 4 * (r16 & 3);
    voff[dt] = vkv_off_pf(4 * kg + (r16 >> 2), dq >> 3) + 2 * (dq & 7);
  }
  // raw scores (q . k, unscaled) of key tile j of the K chunk at LDS address kbase, both heads
  auto raw_scores = [&](uint32_t kbase, int j, const u32x4 (&qf)[2][4], f32x4 (&a)[2]) {
    u32x4 kf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
      kf[ks] = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(kbase + 4096u * j + koff[ks]);
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      a[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ks++) a[hh] = mfma_16x16x32(kf[ks], qf[hh][ks], a[hh]);
    }
  };

  int n = 0;  // the next item
  for (int b = 0; b < nblk; b++) {
    const int kb0 = F2KB * b, kb1 = min(nkey, kb0 + F2KB), nc = (kb1 - kb0 + F2K - 1) / F2K;
    // ---- the block's scores, kept; the row maxima over the unscaled scores (scale > 0 and
    // rounding is monotonic, so max(a * scale) = max(a) * scale, both rounded)
    f32x4 sc[F2NC][4][2];
    float mx[2] = {-INFINITY, -INFINITY};
    // Q^T (B operand) of both heads: lane (row r16, kg) holds dims 32 ks + 8 kg .. +7 of its
    // row (the first item's barrier has published the Q rows; they are never overwritten)
    u32x4 qf[2][4];
#pragma unroll
    for (int c = 0; c < F2NC; c++) {
      if (c < nc) {
        AWAIT((F3R - 2) * F3I);
        ABAR();
        issue(n + F3R - 1);
        const uint32_t kbase = lr + (uint32_t)(n % F3R) * (F2K * 256);
        n++;
        if (c == 0) {
#pragma unroll
          for (int hh = 0; hh < 2; hh++)
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
              qf[hh][ks] = *(const __attribute__((address_space(3))) u32x4*)(uintptr_t)(
                  lq + 16384u * hh + 256u * 16 * wv + akv_off(r16, 4 * ks + kg));
        }
        const int ck0 = kb0 + F2K * c;  // the chunk's first key
        if (ck0 + F2K - 1 < kb1 && ck0 + F2K - 1 <= wrow0) {
          // no score of the chunk is masked
#pragma unroll
          for (int j = 0; j < 4; j++) {
            raw_scores(kbase, j, qf, sc[c][j]);
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
              mx[hh] = fmaxf(fmaxf(mx[hh], fmaxf(sc[c][j][hh][0], sc[c][j][hh][1])),
                             fmaxf(sc[c][j][hh][2], sc[c][j][hh][3]));
              sc[c][j][hh] = park_agpr(sc[c][j][hh]);
            }
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int key0 = ck0 + 16 * j;
            if (key0 <= wrow1) {
              raw_scores(kbase, j, qf, sc[c][j]);
#pragma unroll
              for (int hh = 0; hh < 2; hh++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                  const int key = key0 + 4 * kg + e;
                  mx[hh] = fmaxf(mx[hh], (key < kb1 && key <= row) ? sc[c][j][hh][e] : -INFINITY);
                }
                sc[c][j][hh] = park_agpr(sc[c][j][hh]);
              }
            }
          }
        }
      }
    }
    float base[2], al[2], sum[2] = {0.f, 0.f};
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const float mn = fmaxf(m_run[hh], lane_group_max(mx[hh]) * scale);
      base[hh] = mn == -INFINITY ? 0.f : mn;
      al[hh] = m_run[hh] == -INFINITY ? 0.f : expf(m_run[hh] - base[hh]);
      m_run[hh] = mn;
#pragma unroll
      for (int dt = 0; dt < 8; dt++) o[hh][dt] *= al[hh];
    }
    // ---- probabilities and P.V, chunk by chunk
#pragma unroll
    for (int c = 0; c < F2NC; c++) {
      if (c < nc) {
        AWAIT((F3R - 2) * F3I);
        ABAR();
        issue(n + F3R - 1);
        const uint32_t vb = lr + (uint32_t)(n % F3R) * (F2K * 256);
        n++;
        const int ck0 = kb0 + F2K * c;
        u32x2 pb[2][4];
        if (ck0 + F2K - 1 < kb1 && ck0 + F2K - 1 <= wrow0) {
#pragma unroll
          for (int j = 0; j < 4; j++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
              const f32x4 a = unpark_agpr(sc[c][j][hh]);
              float e4[4];
#pragma unroll
              for (int e = 0; e < 4; e++) {
                e4[e] = exp_fast(unfused(a[e] * scale) - base[hh]);
                sum[hh] += e4[e];
              }
              pb[hh][j] = u32x2{pack_bf2(e4[0], e4[1]), pack_bf2(e4[2], e4[3])};
            }
        } else {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int key0 = ck0 + 16 * j;
            if (key0 <= wrow1) {
#pragma unroll
              for (int hh = 0; hh < 2; hh++) {
                const f32x4 a = unpark_agpr(sc[c][j][hh]);
                float e4[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                  // the score a * scale, or -inf where masked (exp(-inf) = 0)
                  const int key = key0 + 4 * kg + e;
                  const float sv = (key < kb1 && key <= row) ? unfused(a[e] * scale) : -INFINITY;
                  e4[e] = exp_fast(sv - base[hh]);
                  sum[hh] += e4[e];
                }
                pb[hh][j] = u32x2{pack_bf2(e4[0], e4[1]), pack_bf2(e4[2], e4[3])};
              }
            } else {
              pb[0][j] = pb[1][j] = u32x2{0u, 0u};
            }
          }
        }
#pragma unroll
        for (int j2 = 0; j2 < 2; j2++) {
          // (the second half's V reads are not hoisted above the first half's products: one
          // half's 32 registers of V fragments at a time keeps the kernel within its VGPRs)
          if (j2 == 1) asm volatile("" ::: "memory");
          if (ck0 + 32 * j2 <= wrow1) {
            const u32x4 pf0 = u32x4{pb[0][2 * j2].x, pb[0][2 * j2].y, pb[0][2 * j2 + 1].x, pb[0][2 * j2 + 1].y};
            const u32x4 pf1 = u32x4{pb[1][2 * j2].x, pb[1][2 * j2].y, pb[1][2 * j2 + 1].x, pb[1][2 * j2 + 1].y};
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
              const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(vb + 8192 * j2 + voff[dt]));
              const v4s hi =
                  __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(uintptr_t)(vb + 8192 * j2 + 4096 + voff[dt]));
              const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
              const u32x4 vf = u32x4{l2.x, l2.y, h2.x, h2.y};
              o[0][dt] = mfma_16x16x32(vf, pf0, o[0][dt]);
              o[1][dt] = mfma_16x16x32(vf, pf1, o[1][dt]);
            }
          }
        }
      }
    }
#pragma unroll
    for (int hh = 0; hh < 2; hh++) l_run[hh] = lane_group_sum(sum[hh]) + al[hh] * l_run[hh];
  }
  wait_vmem();  // the ring's last (dummy) copies: no DMA may target this LDS after the exit
  if (row < S) {
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const float inv = 1.0f / l_run[hh];
      uint16_t* op = out + (size_t)row * QS + HD * (2 * g + hh) + 4 * kg;
#pragma unroll
      for (int dt = 0; dt < 8; dt++)
        *reinterpret_cast<u32x2*>(op + 16 * dt) =
            u32x2{pack_bf2(o[hh][dt][0] * inv, o[hh][dt][1] * inv), pack_bf2(o[hh][dt][2] * inv, o[hh][dt][3] * inv)};
    }
  }
}

#undef AWAIT
#undef ABAR

// ------------------------------------------------------------------ LM head
constexpr int LMB = 1184;  // partial-argmax blocks (the length of the reference's block_max_* buffers)

// Final norm of the last hidden row (every workgroup computes it), then the bf16 logits of
// rows [VOCAB * b / LMB, VOCAB * (b+1) / LMB) of the tied LM head and their argmax (lowest
// index on ties). Workgroup 0 also writes the row out, as each reference launcher does:
// - launch_prefill_float: the final-norm row (bf16) to final_hidden and to hidden_out (the
//   reference copies final_hidden into hidden_bf16_out, csrc/megakernel/fused_prefill.cu:843-849);
// - launch_prefill_megakernel: the final-norm row as fp32 to final_f32 and the pre-norm row
//   to hidden_out (csrc/megakernel/fused_prefill_megakernel.cu:723-728).
__global__ void __launch_bounds__(256) lm_partial(const uint16_t* hlast, const uint16_t* fnw, const uint16_t* lm,
                                                  uint16_t* final_hidden, float* final_f32, uint16_t* hidden_out,
                                                  int prenorm_out, float* bmv, int* bmi) {
  __shared__ __align__(16) uint32_t s_x[H / 2];
  __shared__ float s_ss[4], s_bv[4];
  __shared__ int s_bi[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, b = blockIdx.x;
  const u32x2 xw = ldw2(hlast + 4 * tid), ww = ldw2(fnw + 4 * tid);
  const float x[4] = {bflo(xw.x), bfhi(xw.x), bflo(xw.y), bfhi(xw.y)};
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++) ss = fmaf(x[i], x[i], ss);
  ss = wave_sum(ss);
  if (lane == 0) s_ss[wv] = ss;
  __syncthreads();
  const float rstd = 1.0f / sqrtf(((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3])) * (1.0f / H) + EPS);
  const uint32_t n0 = pack_bf2(rbf(bflo(ww.x) * rbf(x[0] * rstd)), rbf(bfhi(ww.x) * rbf(x[1] * rstd)));
  const uint32_t n1 = pack_bf2(rbf(bflo(ww.y) * rbf(x[2] * rstd)), rbf(bfhi(ww.y) * rbf(x[3] * rstd)));
  s_x[2 * tid] = n0;
  s_x[2 * tid + 1] = n1;
  if (b == 0) {
    if (final_hidden) reinterpret_cast<u32x2*>(final_hidden)[tid] = u32x2{n0, n1};
    if (final_f32)
      reinterpret_cast<f32x4*>(final_f32)[tid] = f32x4{bflo(n0), bfhi(n0), bflo(n1), bfhi(n1)};
    reinterpret_cast<u32x2*>(hidden_out)[tid] = prenorm_out ? xw : u32x2{n0, n1};
  }
  __syncthreads();
  const u32x4 xa = reinterpret_cast<const u32x4*>(s_x)[lane], xb = reinterpret_cast<const u32x4*>(s_x)[64 + lane];
  const int r0 = (int)((long long)VOCAB * b / LMB), r1 = (int)((long long)VOCAB * (b + 1) / LMB);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int r = r0 + wv; r < r1; r += 16) {
    u32x4 wa[4], wb[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int rr = min(r + 4 * u, r1 - 1);
      wa[u] = ldw(lm + (size_t)rr * H + 8 * lane);
      wb[u] = ldw(lm + (size_t)rr * H + 512 + 8 * lane);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const float lg = rbf(wave_sum(dot_chunk(wa[u], xa, dot_chunk(wb[u], xb, 0.f))));
      if (r + 4 * u < r1 && lg > bv) {
        bv = lg;
        bi = r + 4 * u;
      }
    }
  }
  if (lane == 0) {
    s_bv[wv] = bv;
    s_bi[wv] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int i = 1; i < 4; i++)
      if (s_bv[i] > bv || (s_bv[i] == bv && s_bi[i] < bi)) {
        bv = s_bv[i];
        bi = s_bi[i];
      }
    bmv[b] = bv;
    bmi[b] = bi;
  }
}

__global__ void __launch_bounds__(256) argmax_final(const float* bmv, const int* bmi, int* out, uint32_t* err) {
  __shared__ float s_bv[4];
  __shared__ int s_bi[4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  float v = -INFINITY;
  int i = 0x7fffffff;
  for (int b = tid; b < LMB; b += 256) {
    const float bv = bmv[b];
    const int bi = bmi[b];
    if (bv > v || (bv == v && bi < i)) {
      v = bv;
      i = bi;
    }
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
    s_bv[wv] = v;
    s_bi[wv] = i;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; w++)
      if (s_bv[w] > v || (s_bv[w] == v && s_bi[w] < i)) {
        v = s_bv[w];
        i = s_bi[w];
      }
    const uint32_t e = *err;
    *out = e ? -(int)(1u + e) : i;
    if (e) *err = 0u;
  }
}

}  // namespace pf
}  // namespace mq

using namespace mq;
using namespace mq::pf;

// GEMM shapes by prompt length (measured on MI355X, weights cold as each layer's are).
// Every shape computes each output with the same MFMA chain over k in the same order, and
// o_proj / down_proj always split k four ways, so the choice does not change any result.
// Longer prompts take larger tiles: a launch streams M N K 2 (1 / TM + 1 / TN) operand
// bytes from L2 into the CUs, and at S = 8192 the 256 x 256 tiles (sixteen waves, a
// two-step ring) run gate/up at 840-910 TFLOP/s against 650 for 128 x 128 ones. Short
// prompts keep smaller tiles so that the grid still fills the 256 CUs:
//   q/k/v (whole-head tiles, QK-norm/RoPE/K-V-append epilogue): 64 x 128 on 2 x 4 waves;
//     from S = 1024 128 x 128 on 4 x 2; from 2048 256 x 128 on 4 x 2 with a three-step ring;
//   gate/up: 128 x 128 on 4 x 4 waves; from S = 1024 128 x 256; from 2048 256 x 256;
//   o_proj, down_proj (k split four ways into fp32 partials): 128 x 64 on 4 x 2 waves;
//     from S = 1024 128 x 256 on 2 x 4; from 4096 256 x 256 on 4 x 4.
constexpr int RES_SPLIT = 4;

// one launch of gemm_nt over a [m, sum of the segments' widths] output, k split `split` ways
// The XCD order of a grid of nx column tiles by ny row tiles (XcdMap) with xg column bands and
// panels of at most xp row tiles (the largest that divides a band), or blockIdx order when
// the grid does not split into 8 such rectangles.
static XcdMap xcd_map(int nx, int ny, int xg, int xp) {
  const int gy = xg > 0 && xg <= 8 && 8 % xg == 0 ? 8 / xg : 0;
  if (gy == 0 || xp < 1 || nx % xg || ny % gy) return XcdMap{0, 0};
  const int rh = ny / gy;
  xp = xp < rh ? xp : rh;
  while (rh % xp) xp--;
  return XcdMap{xg, xp};
}
template <int EPI, int TM, int TN, int NST, int KS, int WM, int WN>
void gemm(GemmArgs g, int ntiles, hipStream_t stream, int split = 1, int xg = 0, int xp = 1,
          const WarmSet* warm = nullptr) {
  const int ny = (g.m + TM - 1) / TM;
  g.xm = xcd_map(ntiles, ny, xg, xp);
  // a warm-up row only where its workgroups land on CUs no tile uses, eight to an XCD
  // class, in blockIdx order
  KernArgs<EPI> ka{};
  ka.a = g.a; ka.lda = g.lda; ka.m = g.m; ka.k = g.k; ka.xm = g.xm;
  ka.nx = ntiles; ka.ny = ny; ka.kp = g.k / split;
  for (int i = 0; i < KernArgs<EPI>::NSEG; i++) ka.seg[i] = g.seg[i];
  if constexpr (EPI == EPI_PART) ka.part = g.part;
  if constexpr (EPI == EPI_QKN) ka.qkn = g.qkn;
  if (warm && warm->n > 0 && ntiles % 8 == 0 && split == 1 && g.xm.xg == 0 && ntiles * (ny + 1) <= NUM_CUS) {
    WarmSet W = *warm;
    W.row = ny;
    gemm_nt_warm<EPI, TM, TN, NST, KS, WM, WN><<<dim3(ntiles, ny + 1, split), 64 * WM * WN, 0, stream>>>(ka, W);
  } else {
    gemm_nt<EPI, TM, TN, NST, KS, WM, WN><<<dim3(ntiles, ny, split), 64 * WM * WN, 0, stream>>>(ka);
  }
}
// Prompts of at most SHORT_S tokens fill few CUs with the tiles of S = 512 (gate/up 48 x 2
// workgroups at S = 256), so they take smaller row tiles: q/k/v 32 x 128, gate/up 64 x 128
// (32 x 128 up to 128 tokens, 64 x 64 up to 64), the k-split residual products 64 x 64 (32 x
// 64 up to 128). Every tile sums its k range in the same order whatever its shape, so the
// outputs are the same bits. Whole prefill, same box, with the warm-up (ms): S = 64 1.600 ->
// 1.408, 96 1.644 -> 1.451, 128 1.699 -> 1.474, 192 1.706 -> 1.591, 256 1.780 -> 1.639.
constexpr int SHORT_S = 256;
static void gemm_qkv(GemmArgs g, hipStream_t stream) {
  // Long prompts: two heads a tile on sixteen waves (256 x 256, two stages; the epilogue stages
  // both heads through the ring as bf16), blockIdx order, the same bits as the one-head
  // 256 x 128 tiles. A two-head tile takes about 1.7 times as long as a one-head tile and there
  // are half as many, so it is used where its rounds of 256 workgroups, ceil(16 ny / 256), cost
  // less than the one-head tiles' ceil(32 ny / 256) (ny row tiles). Same box, the q/k/v launch
  // alone: S = 2600 49.9 -> 40.2 us, 3072 51.9 -> 41.7, 4096 55.0 -> 44.8, 6400 98.8 -> 76.5,
  // 7168 101.1 -> 80.1, 8192 98.1 -> 82.3; where the model says no: 2048 28.7 -> 39.0, 5000
  // 74.4 -> 74.0, and the whole S = 6000 prefill 16.58 -> 16.68 ms.
  const int ny = (g.m + 255) / 256;
  if (g.m >= 2048 && 17 * ((ny + 15) / 16) < 10 * ((ny + 7) / 8)) {
    g.seg[0].ntiles = QS / (2 * HD);
    g.seg[1].ntiles = g.seg[2].ntiles = KVS / (2 * HD);
    gemm<EPI_QKN, 256, 2 * HD, 2, 1, 4, 4>(g, (QS + 2 * KVS) / (2 * HD), stream);
    return;
  }
  if (g.m > 512 && g.m < 1024) {
    // 513..1023 tokens: two heads a tile on 64 x 256 tiles (eight waves, four stages), one round
    // of at most 256 workgroups where the one-head 64 x 128 tiles need two; same bits, the
    // launch alone, same box: S = 640 19.0 -> 17.1 us, 768 19.6 -> 17.4, 1000 21.2 -> 19.1
    // (up to 512 tokens the one-head tiles are faster: 11.3 against 16.6 us at S = 512)
    g.seg[0].ntiles = QS / (2 * HD);
    g.seg[1].ntiles = g.seg[2].ntiles = KVS / (2 * HD);
    gemm<EPI_QKN, 64, 2 * HD, 4, 1, 2, 4>(g, (QS + 2 * KVS) / (2 * HD), stream);
    return;
  }
  if (g.m > 1024 && g.m < 2048) {
    // 1025..2047 tokens: two heads a tile on 128 x 256 tiles (sixteen waves, three stages), one
    // round of at most 256 workgroups where the one-head 128 x 128 tiles need two (the same
    // rounds argument as above); same bits, the launch alone, same box: S = 1100 30.6 -> 23.5
    // us, 1536 31.6 -> 24.4, 2047 33.7 -> 27.2 (at 1024 both take one round)
    g.seg[0].ntiles = QS / (2 * HD);
    g.seg[1].ntiles = g.seg[2].ntiles = KVS / (2 * HD);
    gemm<EPI_QKN, 128, 2 * HD, 3, 1, 4, 4>(g, (QS + 2 * KVS) / (2 * HD), stream);
    return;
  }
  g.seg[0].ntiles = QS / HD;
  g.seg[1].ntiles = g.seg[2].ntiles = KVS / HD;
  const int nt = (QS + 2 * KVS) / HD;
  // long prompts: an XCD takes an eighth of the row tiles and every head, 4 row tiles by 8
  // heads at a time, so each A row tile is fetched from HBM by one XCD (S = 8192: 107.5 ->
  // 99.3 us against blockIdx order, same-box medians)
  if (g.m >= 2048) gemm<EPI_QKN, 256, HD, 3, 1, 4, 2>(g, nt, stream, 1, 1, 4);
  else if (g.m >= 1024) gemm<EPI_QKN, 128, HD, 4, 1, 4, 2>(g, nt, stream);
  else if (g.m > SHORT_S) gemm<EPI_QKN, 64, HD, 4, 1, 2, 4>(g, nt, stream);
  else gemm<EPI_QKN, 32, HD, 4, 1, 2, 2>(g, nt, stream);
}
// warm: the warm-up set of a prompt of at most WARM_MAX_S tokens, or null
static void gemm_gate_up(GemmArgs g, hipStream_t stream, const WarmSet* warm = nullptr) {
  static_assert(WARM_MAX_S <= 512, "the warm-up set's column tiles are those of the shapes up to 512 tokens");
  // 2049..3584 tokens: 128 x 256 tiles, twice the workgroups of the 256 x 256 tiles, each
  // taking about 0.6 of the time; they fill the last round of 256 workgroups better there
  // (same bits; the launch alone, same box: S = 3072 67.9 -> 61.1 us; at 2048, 5000, 6000
  // and 7000 the 256 x 256 tiles are as fast or faster, and at 4096 the launch alone gains
  // (72.0 -> 66.9) but the whole prefill loses, 9.99 -> 10.18 ms)
  if (g.m > 2048 && g.m <= 3584) {
    g.seg[0].ntiles = I / 128;
    gemm<EPI_SILU, 128, 256, 3, 1, 4, 4>(g, I / 128, stream);
  } else if (g.m > 1408) {
    // (from 1409 tokens the 128 x 256 tiles need more than one round of 256 workgroups; the
    // 256 x 256 tiles: S = 1536 38.2 -> 34.5 us, 2047 40.8 -> 38.8; at 1100 22.2 -> 34.5)
    g.seg[0].ntiles = I / 128;
    gemm<EPI_SILU, 256, 256, 2, 1, 4, 4>(g, I / 128, stream);  // (the XCD order measured no gain here)
  } else if (g.m >= 1024) {
    g.seg[0].ntiles = I / 128;
    gemm<EPI_SILU, 128, 256, 3, 1, 4, 4>(g, I / 128, stream);
  } else if (g.m > 640) {
    // (641..1023 tokens: the 128 x 128 tiles need a second round of 256 workgroups, the
    // 128 x 256 tiles one; S = 768 24.6 -> 20.5 us, 1000 25.3 -> 21.6; at 640 14.6 -> 19.9)
    g.seg[0].ntiles = I / 128;
    gemm<EPI_SILU, 128, 256, 3, 1, 4, 4>(g, I / 128, stream);
  } else if (g.m > 512) {
    g.seg[0].ntiles = I / 64;
    gemm<EPI_SILU, 128, 128, 3, 1, 4, 4>(g, I / 64, stream, 1, 0, 1, warm);
  } else if (g.m > SHORT_S) {
    // (257..512 tokens: 128 x 96 tiles on four waves, 64 column tiles, so 256 workgroups fill
    // the CUs where the 128 x 128 tiles leave 64 idle; same bits, whole prefill, same box:
    // S = 300 1.722 -> 1.714 ms, 384 1.774 -> 1.759, 512 1.923 -> 1.918; at 640 1.9x the
    // workgroups need two rounds, 2.414 -> 2.636; eight waves on two stages of two k-steps
    // 1-3% slower)
    g.seg[0].ntiles = I / 48;
    gemm<EPI_SILU, 128, 96, 3, 1, 4, 1>(g, I / 48, stream, 1, 0, 1, warm);
  } else if (g.m > 128) {
    g.seg[0].ntiles = I / 64;
    gemm<EPI_SILU, 64, 128, 3, 1, 2, 4>(g, I / 64, stream, 1, 0, 1, warm);
  } else if (g.m > 64) {
    g.seg[0].ntiles = I / 64;
    gemm<EPI_SILU, 32, 128, 4, 1, 2, 2>(g, I / 64, stream, 1, 0, 1, warm);
  } else {
    g.seg[0].ntiles = I / 32;
    gemm<EPI_SILU, 64, 64, 4, 1, 2, 2>(g, I / 32, stream, 1, 0, 1, warm);
  }
}
// Long prompts: o_proj / down_proj with the residual add in the epilogue (the four k quarters
// summed in order inside the workgroup: the same bits as the split-four partials and
// resid_norm_rows), on 256 x 128 tiles; out = h, updated in place
constexpr int RESADD_MIN_S = 7168;
static void gemm_residual_add(GemmArgs g, uint16_t* h, hipStream_t stream) {
  g.seg[0].out = h;
  g.seg[0].ldo = H;
  g.seg[0].ntiles = H / 128;
  // an XCD takes a quarter of the row tiles and half the column tiles, 4 row tiles at a time:
  // each A row tile is fetched by two XCDs instead of eight (S = 8192, same-box medians:
  // o_proj 49.3 -> 41.0 us, down_proj 67.8 -> 55.1 us)
  gemm<EPI_RESADD, 256, 128, 3, 1, 4, 2>(g, H / 128, stream, 1, 2, 4);
}
static void gemm_residual(GemmArgs g, hipStream_t stream) {
  // 256 x 256 tiles from 2049 tokens (at most one round of 256 workgroups up to 4096, where
  // the 128 x 256 tiles need two; same bits, down_proj's shape alone, same box: S = 3072
  // 37.8 -> 29.9 us; at 2048 the 128 x 256 tiles are faster, 23.1 against 25.1)
  if (g.m > 2048) {
    g.seg[0].ntiles = H / 256;
    gemm<EPI_PART, 256, 256, 2, 1, 4, 4>(g, H / 256, stream, RES_SPLIT);
  } else if (g.m >= 1024) {
    g.seg[0].ntiles = H / 256;
    gemm<EPI_PART, 128, 256, 3, 1, 2, 4>(g, H / 256, stream, RES_SPLIT);
  } else if (g.m > 512) {
    // (513..1023 tokens: one round of 256 workgroups on 128 x 128 tiles where 128 x 64 tiles
    // need two; S = 640 15.1 -> 12.5 us, 1000 17.1 -> 15.2)
    g.seg[0].ntiles = H / 128;
    gemm<EPI_PART, 128, 128, 4, 1, 4, 2>(g, H / 128, stream, RES_SPLIT);
  } else {
    g.seg[0].ntiles = H / 64;
    if (g.m > SHORT_S) gemm<EPI_PART, 128, 64, 4, 1, 4, 2>(g, H / 64, stream, RES_SPLIT);
    else if (g.m > 128) gemm<EPI_PART, 64, 64, 4, 1, 2, 2>(g, H / 64, stream, RES_SPLIT);
    else gemm<EPI_PART, 32, 64, 4, 1, 2, 2>(g, H / 64, stream, RES_SPLIT);
  }
}

// The buffers of one prefill run, carved from a launcher's scratch arguments: the bf16
// activations, the fp32 partial sums of the k-split o_proj and down_proj, and where the
// last row's final norm and hidden state go (see lm_partial).
struct PrefillBufs {
  uint16_t *h, *nrm, *qp, *att, *mln, *mid;
  PartSet parts;
  uint16_t* final_bf16;  // final-norm row (bf16), or null
  float* final_f32;      // final-norm row (fp32), or null
  uint16_t* hidden_out;  // the final-norm row, or with prenorm_out the pre-norm row
  int prenorm_out;
  float* bmv;  // per-block LM-head maxima and their indices
  int* bmi;
};

// Argument checks shared by the prefill launchers (before any HIP call).
static bool prefill_args_ok(const int* ids, const int* out, int S, const void* embed, const PrefillLayerWeights* lw,
                            const void* fnw, const void* lm, const void* cos_t, const void* sin_t, const void* kc,
                            const void* vc, int num_layers, int max_seq, float scale) {
  if (!ids || !out || !embed || !lw || !fnw || !lm || !cos_t || !sin_t || !kc || !vc) return false;
  if (S < 1 || max_seq < 1 || S > max_seq || num_layers < 1 || num_layers > MAX_LAYERS || !(scale > 0.f) ||
      !isfinite(scale))
    return false;
  for (int l = 0; l < num_layers; l++) {
    const PrefillLayerWeights& w = lw[l];
    if (!w.input_layernorm_weight || !w.q_proj_weight || !w.k_proj_weight || !w.v_proj_weight ||
        !w.q_norm_weight || !w.k_norm_weight || !w.o_proj_weight || !w.post_attn_layernorm_weight ||
        !w.gate_proj_weight || !w.up_proj_weight || !w.down_proj_weight)
      return false;
  }
  return true;
}

// One prefill: embedding, every layer, the LM head's argmax of the last row.
static int prefill_run(const int* input_token_ids, int* output_token_id, int seq_len, const void* embed_weight,
                       const PrefillLayerWeights* layer_weights, const void* final_norm_weight,
                       const void* lm_head_weight, const void* cos_table, const void* sin_table, void* k_cache,
                       void* v_cache, const PrefillBufs& B, int num_layers, int max_seq_len, float attn_scale,
                       hipStream_t stream) {
  uint32_t* ws = nullptr;
  const int st = current_workspace(&ws);
  if (st != MQ_OK) return st;
  uint32_t* err = ws + WS_PREFILL_ERR;

  const int S = seq_len;
  auto bf = [](const void* p) { return static_cast<const uint16_t*>(p); };
  auto bfm = [](void* p) { return static_cast<uint16_t*>(p); };
  uint16_t* h = B.h;
  uint16_t* nrm = B.nrm;
  uint16_t* qp = B.qp;
  uint16_t* att = B.att;
  uint16_t* mln = B.mln;
  uint16_t* mid = B.mid;
  const PartSet parts = B.parts;
  const size_t kv_layer = (size_t)NKV * max_seq_len * HD;

  hipError_t launch_err = hipSuccess;
  auto chk = [&]() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess && launch_err == hipSuccess) launch_err = e;
  };
  (void)hipGetLastError();  // clear an error left by an unrelated earlier call
  embed_rows<<<S, 128, 0, stream>>>(input_token_ids, bf(embed_weight), h, err);
  chk();
  rmsnorm_rows<<<S, 64, 0, stream>>>(h, bf(layer_weights[0].input_layernorm_weight), nrm, S);
  chk();
  for (int l = 0; l < num_layers; l++) {
    const PrefillLayerWeights& w = layer_weights[l];
    uint16_t* kcl = bfm(k_cache) + l * kv_layer;
    uint16_t* vcl = bfm(v_cache) + l * kv_layer;
    GemmArgs g{};
    g.a = nrm; g.lda = H; g.m = S; g.k = H;
    g.seg[0] = GemmSeg{bf(w.q_proj_weight), nullptr, nullptr, 0, QS};
    g.seg[1] = GemmSeg{bf(w.k_proj_weight), nullptr, nullptr, 0, KVS};
    g.seg[2] = GemmSeg{bf(w.v_proj_weight), nullptr, nullptr, 0, KVS};
    g.qkn = QknArgs{bf(w.q_norm_weight), bf(w.k_norm_weight), bf(cos_table), bf(sin_table), qp, kcl, vcl, max_seq_len};
    gemm_qkv(g, stream);
    chk();
    // long prompts: the two-pass flash form (128 rows of both heads a workgroup), then the
    // flash form with the scores kept (64 rows); short ones: 32 rows of one head a workgroup,
    // which fills more CUs (256 workgroups at S = 512)
    if (S > FLASH2_MIN_S)
      attn_prefill_fa2<<<NKV * ((S + F2Q - 1) / F2Q), 64 * F2W, 0, stream>>>(qp, kcl, vcl, att, S, max_seq_len,
                                                                             attn_scale);
    else if (S > FLASH_MIN_S)
      attn_prefill_fa3<<<NKV * ((S + F3Q - 1) / F3Q), 64 * F3W, 0, stream>>>(qp, kcl, vcl, att, S, max_seq_len,
                                                                             attn_scale);
    else if (S <= SHORT_S)
      attn_prefill<true><<<NQ * ((S + AQ - 1) / AQ), 64 * AW, 0, stream>>>(qp, kcl, vcl, att, S, max_seq_len, attn_scale);
    else
      attn_prefill<false><<<NQ * ((S + AQ - 1) / AQ), 64 * AW, 0, stream>>>(qp, kcl, vcl, att, S, max_seq_len, attn_scale);
    chk();
    GemmArgs go{};
    go.a = att; go.lda = QS; go.m = S; go.k = QS;
    go.seg[0] = GemmSeg{bf(w.o_proj_weight), nullptr, nullptr, 0, H};
    if (S >= RESADD_MIN_S) {
      gemm_residual_add(go, h, stream);
      chk();
      rmsnorm_rows<<<S, 64, 0, stream>>>(h, bf(w.post_attn_layernorm_weight), mln, S);
    } else {
      go.part = parts;
      gemm_residual(go, stream);
      chk();
      resid_norm_rows<RES_SPLIT><<<S, 64, 0, stream>>>(parts, h, bf(w.post_attn_layernorm_weight), mln, S);
    }
    chk();
    GemmArgs gu{};
    gu.a = mln; gu.lda = H; gu.m = S; gu.k = H;
    gu.seg[0] = GemmSeg{bf(w.gate_proj_weight), bf(w.up_proj_weight), mid, 0, I};
    WarmSet W{};
    if (S <= WARM_MAX_S) {
      // short prompts: the idle CUs of gate/up read down_proj's weights and the next layer's
      // q/k/v and o_proj weights, each column tile on the XCD of the launch that reads it
      // (q/k/v column tiles of one head: q 0-15, k 16-23, v 24-31; the k-split residual
      // products' 64-column tiles: 16)
      auto add = [&](const void* wp, int tile_bytes, int ntiles, int xcd0) {
        W.w[W.n] = bf(wp); W.tile_bytes[W.n] = tile_bytes; W.ntiles[W.n] = ntiles; W.xcd0[W.n] = xcd0; W.n++;
      };
      add(w.down_proj_weight, 64 * I * 2, H / 64, 0);
      if (l + 1 < num_layers) {
        const PrefillLayerWeights& wn = layer_weights[l + 1];
        add(wn.q_proj_weight, HD * H * 2, QS / HD, 0);
        add(wn.k_proj_weight, HD * H * 2, KVS / HD, (QS / HD) % 8);
        add(wn.v_proj_weight, HD * H * 2, KVS / HD, (QS / HD + KVS / HD) % 8);
        add(wn.o_proj_weight, 64 * QS * 2, H / 64, 0);
      }
    }
    gemm_gate_up(gu, stream, W.n > 0 ? &W : nullptr);
    chk();
    GemmArgs gd{};
    gd.a = mid; gd.lda = I; gd.m = S; gd.k = I;
    gd.seg[0] = GemmSeg{bf(w.down_proj_weight), nullptr, nullptr, 0, H};
    // then the next layer's input RMSNorm (none after the last: the final norm is the LM head's)
    if (S >= RESADD_MIN_S) {
      gemm_residual_add(gd, h, stream);
      chk();
      if (l + 1 < num_layers) rmsnorm_rows<<<S, 64, 0, stream>>>(h, bf(layer_weights[l + 1].input_layernorm_weight), nrm, S);
    } else {
      gd.part = parts;
      gemm_residual(gd, stream);
      chk();
      resid_norm_rows<RES_SPLIT><<<S, 64, 0, stream>>>(
          parts, h, l + 1 < num_layers ? bf(layer_weights[l + 1].input_layernorm_weight) : nullptr, nrm, S);
    }
    chk();
  }
  lm_partial<<<LMB, 256, 0, stream>>>(h + (size_t)(S - 1) * H, bf(final_norm_weight), bf(lm_head_weight),
                                      B.final_bf16, B.final_f32, B.hidden_out, B.prenorm_out, B.bmv, B.bmi);
  chk();
  argmax_final<<<1, 256, 0, stream>>>(B.bmv, B.bmi, output_token_id, err);
  chk();
  return launch_err == hipSuccess ? MQ_OK : MQ_ERR_HIP;
}

extern "C" int launch_prefill_float(const int* input_token_ids, int* output_token_id, int seq_len,
                                    const void* embed_weight, const PrefillLayerWeights* layer_weights,
                                    const void* final_norm_weight, const void* lm_head_weight, const void* cos_table,
                                    const void* sin_table, void* k_cache, void* v_cache, void* hidden_bf16,
                                    void* residual, void* normalized, void* q_proj, void* k_proj, void* v_proj,
                                    void* attn_out, void* o_proj_out, void* mlp_norm, void* gate_out, void* up_out,
                                    void* mlp_intermediate, void* down_out, void* final_hidden, void* block_max_vals,
                                    void* block_max_idxs, void* hidden_bf16_out, int num_layers, int max_seq_len,
                                    float attn_scale, hipStream_t stream) {
  (void)residual; (void)o_proj_out; (void)down_out;
  if (!prefill_args_ok(input_token_ids, output_token_id, seq_len, embed_weight, layer_weights, final_norm_weight,
                       lm_head_weight, cos_table, sin_table, k_cache, v_cache, num_layers, max_seq_len, attn_scale) ||
      !hidden_bf16 || !normalized || !q_proj || !k_proj || !v_proj || !attn_out || !mlp_norm || !gate_out ||
      !up_out || !mlp_intermediate || !final_hidden || !block_max_vals || !block_max_idxs || !hidden_bf16_out)
    return MQ_ERR_ARG;
  auto bfm = [](void* p) { return static_cast<uint16_t*>(p); };
  PrefillBufs B{};
  B.h = bfm(hidden_bf16);
  B.nrm = bfm(normalized);
  B.qp = bfm(q_proj);
  B.att = bfm(attn_out);
  B.mln = bfm(mlp_norm);
  B.mid = bfm(mlp_intermediate);
  // fp32 partial sums of the k-split o_proj and down_proj, [S, 1024] a split, in scratch
  // that is dead while they live: gate_out and up_out (unused otherwise), q_proj (read by
  // the attention before o_proj) and k_proj | v_proj as the two column halves of the
  // fourth set (unused: the q/k/v epilogue writes k and v straight to the caches)
  auto f32 = [](void* p) { return static_cast<float*>(p); };
  B.parts.n = RES_SPLIT;
  float* const whole[3] = {f32(gate_out), f32(up_out), f32(q_proj)};
  for (int z = 0; z < 3; z++) {
    B.parts.lo[z] = whole[z];
    B.parts.hi[z] = whole[z] + PART_HALF;
    B.parts.ld[z] = H;
  }
  B.parts.lo[3] = f32(k_proj);
  B.parts.hi[3] = f32(v_proj);
  B.parts.ld[3] = PART_HALF;
  B.final_bf16 = bfm(final_hidden);
  B.hidden_out = bfm(hidden_bf16_out);
  B.bmv = static_cast<float*>(block_max_vals);
  B.bmi = static_cast<int*>(block_max_idxs);
  return prefill_run(input_token_ids, output_token_id, seq_len, embed_weight, layer_weights, final_norm_weight,
                     lm_head_weight, cos_table, sin_table, k_cache, v_cache, B, num_layers, max_seq_len, attn_scale,
                     stream);
}

// The reference's fused-prefill launcher (csrc/megakernel/fused_prefill_megakernel.cu:938-1016),
// on the same MFMA prefill. Its scratch is fp32 ([seq_len, n] rows of 4 n bytes), twice the
// bytes of the bf16 activations, so the activations and the fp32 partial sums are carved from
// it: h, the post-attention norm output, the input norm output, q and the attention output in
// the first half of hidden, residual, normalized, q_proj and attn_out; the partial sums in
// k_proj and v_proj (whole), q_proj (once the attention has read q) and the second half of
// mlp_intermediate (whose first half holds the MLP activations). final_hidden receives the
// final-norm row as fp32 and hidden_bf16_out the pre-norm last row, as the reference writes.
extern "C" int launch_prefill_megakernel(const int* token_ids, int* output_token_id, int seq_len,
                                         const void* embed_weight, const PrefillLayerWeights* layer_weights,
                                         const void* final_norm_weight, const void* lm_head_weight,
                                         const void* cos_table, const void* sin_table, void* k_cache, void* v_cache,
                                         void* hidden, void* residual, void* normalized, void* q_proj, void* k_proj,
                                         void* v_proj, void* attn_out, void* mlp_intermediate, void* final_hidden,
                                         void* hidden_bf16_out, void* block_max_vals, void* block_max_idxs,
                                         int num_layers, int max_seq_len, float attn_scale, hipStream_t stream) {
  if (!prefill_args_ok(token_ids, output_token_id, seq_len, embed_weight, layer_weights, final_norm_weight,
                       lm_head_weight, cos_table, sin_table, k_cache, v_cache, num_layers, max_seq_len, attn_scale) ||
      !hidden || !residual || !normalized || !q_proj || !k_proj || !v_proj || !attn_out || !mlp_intermediate ||
      !final_hidden || !hidden_bf16_out || !block_max_vals || !block_max_idxs)
    return MQ_ERR_ARG;
  auto bfm = [](void* p) { return static_cast<uint16_t*>(p); };
  auto f32 = [](void* p) { return static_cast<float*>(p); };
  const size_t S = (size_t)seq_len;
  PrefillBufs B{};
  B.h = bfm(hidden);
  B.mln = bfm(residual);
  B.nrm = bfm(normalized);
  B.qp = bfm(q_proj);
  B.att = bfm(attn_out);
  B.mid = bfm(mlp_intermediate);  // [S, 3072] bf16: the first S * 6 KB of S * 12 KB
  B.parts.n = RES_SPLIT;
  float* const sets[RES_SPLIT] = {f32(k_proj), f32(v_proj), f32(q_proj),
                                  f32(mlp_intermediate) + S * (I / 2)};  // byte offset S * 6 KB
  for (int z = 0; z < RES_SPLIT; z++) {
    B.parts.lo[z] = sets[z];
    B.parts.hi[z] = sets[z] + PART_HALF;
    B.parts.ld[z] = H;
  }
  B.final_f32 = f32(final_hidden);
  B.hidden_out = bfm(hidden_bf16_out);
  B.prenorm_out = 1;
  B.bmv = f32(block_max_vals);
  B.bmi = static_cast<int*>(block_max_idxs);
  return prefill_run(token_ids, output_token_id, seq_len, embed_weight, layer_weights, final_norm_weight,
                     lm_head_weight, cos_table, sin_table, k_cache, v_cache, B, num_layers, max_seq_len, attn_scale,
                     stream);
}
