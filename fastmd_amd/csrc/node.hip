// Fused node-side update of the MACE-like interaction, forward and VJP: per workgroup a tile of
// 32 atoms runs the chain of small GEMMs and the symmetric contraction that otherwise takes six
// launches each way (two GEMMs of the aggregated messages, the contraction, three output GEMMs).
//
// A tile is 128 rows: block 0 = the 32 atoms' scalar rows ([N, C] matrices), blocks 1-3 = their
// 96 vector rows ([N, 3, C] matrices, 3 rows per atom). Each GEMM phase multiplies the tile by a
// weight per block (slot 0 for block 0, slot 1 for blocks 1-3), stored [columns, K]
// K-contiguous, fp32-accurate on the bf16 matrix cores (three bf16 planes per operand, six
// products: x3.h), in column passes of 128 and K slices of 16 through a double-buffered LDS
// (A planes + both weight slots: 72 KB, two workgroups per CU). Between phases the tile's rows go
// through global memory (they are L2 hits; P0/P1 are kept for the VJP anyway), ordered by the
// workgroup barrier.
//   forward  (phase 1)  [A0; A1] x [Wm0 | Wm1]                          -> P0, P1
//            (phase 2)  symmetric contraction                         -> B0, B1
//            (phase 3)  [B0 h0; B1 0] x [(Wo0 ; Wsc0) | (Wo1 ; 0)]    -> h0', h1'
//   VJP      (phase 1)  [g0; g1] x [(Wo0^T | Wsc0^T) | (Wo1^T | 0)]   -> gB0 | g_in0, gB1
//            (phase 2)  contraction VJP                               -> gP0, gP1
//            (phase 3)  [gP0; gP1] x [Wm0^T | Wm1^T]                  -> gA0, gA1
// (weights named as the model's [in, out] matrices; the host passes each phase's B already laid
// out [columns, K]). Deterministic: fixed summation order, no atomics.
#include "common.h"
#include "mace_math.h"
#include "x3.h"

namespace {

constexpr int kThreads = 256;
constexpr int kTA = 32;                 // atoms per workgroup
constexpr int kPL = 128 * 16;           // one bf16 plane of a 128 x 16 slice
constexpr int kBufA = 3 * kPL;          // A planes
constexpr int kBuf = kBufA + 2 * 3 * kPL;  // + two weight slots

// A rows of the tile: block 0 -> atom atom0 + r of s0 (ld C) for k < ksplit, of s0b (ld C) at
// k - ksplit beyond; blocks 1-3 -> row 3 atom0 + (r - 32) of s1 (ld C) for k < ksplit, zero beyond.
struct TileA {
  const float* s0;
  const float* s0b;
  const float* s1;
  int ksplit;
};

__device__ __forceinline__ float4 load4_or_zero(const float* p) {
  return p ? *reinterpret_cast<const float4*>(p) : make_float4(0.f, 0.f, 0.f, 0.f);
}

// acc = tile(A)[128, K] x W_slot[col0 .. col0 + 128, K]^T  (K and ksplit multiples of 16)
__device__ __forceinline__ void tile_gemm(const TileA& A, const float* w0, const float* w1, int64_t ldw, int ncols,
                                          int col0, int K, int64_t atom0, int64_t n_atoms, int C, __bf16* lds,
                                          fmd_f32x16 (&acc)[2][2]) {
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, rr = lane & 31;
  const int kc = (t & 3) * 4;
  // this thread's two rows of the A tile and of the weight tile (null: the row is zero)
  const float* alo[2];
  const float* ahi[2];
  const float* b0r[2];
  const float* b1r[2];
  int soff[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int r = (t + q * kThreads) >> 2;
    soff[q] = x3_lds_offset(r, kc);
    if (r < kTA) {
      const int64_t atom = atom0 + r;
      const bool ok = atom < n_atoms;
      alo[q] = ok ? A.s0 + atom * C + kc : nullptr;
      ahi[q] = ok && A.s0b ? A.s0b + atom * C + kc : nullptr;
    } else {
      const int64_t row = 3 * atom0 + (r - kTA);
      alo[q] = A.s1 && row < 3 * n_atoms ? A.s1 + row * C + kc : nullptr;
      ahi[q] = nullptr;
    }
    const int col = col0 + r;
    b0r[q] = w0 && col < ncols ? w0 + (int64_t)col * ldw + kc : nullptr;
    b1r[q] = w1 && col < ncols ? w1 + (int64_t)col * ldw + kc : nullptr;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  float4 ra[2], rb0[2], rb1[2];
  const int nk = K / 16;
  const int rd = x3_lds_offset(rr, h * 8);
  // slice kt -> registers
#define NODE_LOAD(KT)                                                                 \
  do {                                                                                \
    const int k0_ = (KT) * 16;                                                        \
    const bool hi_ = k0_ >= A.ksplit;                                                 \
    _Pragma("unroll") for (int q = 0; q < 2; ++q) {                                   \
      const float* pa_ = hi_ ? (ahi[q] ? ahi[q] + (k0_ - A.ksplit) : nullptr)         \
                             : (alo[q] ? alo[q] + k0_ : nullptr);                     \
      ra[q] = load4_or_zero(pa_);                                                     \
      rb0[q] = load4_or_zero(b0r[q] ? b0r[q] + k0_ : nullptr);                        \
      rb1[q] = load4_or_zero(b1r[q] ? b1r[q] + k0_ : nullptr);                        \
    }                                                                                 \
  } while (0)
  // registers -> LDS buffer (split into the three planes)
#define NODE_STORE(BUFI)                                                              \
  do {                                                                                \
    __bf16* sb_ = lds + (BUFI) * kBuf;                                                \
    _Pragma("unroll") for (int q = 0; q < 2; ++q) {                                   \
      fmd_bf16x4 x0_, x1_, x2_;                                                       \
      x3_split(ra[q], x0_, x1_, x2_);                                                 \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + 0 * kPL + soff[q]) = x0_;                  \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + 1 * kPL + soff[q]) = x1_;                  \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + 2 * kPL + soff[q]) = x2_;                  \
      x3_split(rb0[q], x0_, x1_, x2_);                                                \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + kBufA + 0 * kPL + soff[q]) = x0_;          \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + kBufA + 1 * kPL + soff[q]) = x1_;          \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + kBufA + 2 * kPL + soff[q]) = x2_;          \
      x3_split(rb1[q], x0_, x1_, x2_);                                                \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + kBufA + 3 * kPL + soff[q]) = x0_;          \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + kBufA + 4 * kPL + soff[q]) = x1_;          \
      *reinterpret_cast<fmd_bf16x4*>(sb_ + kBufA + 5 * kPL + soff[q]) = x2_;          \
    }                                                                                 \
  } while (0)
  NODE_LOAD(0);
  NODE_STORE(0);
  if (nk > 1) NODE_LOAD(1);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) {
      NODE_STORE(cur ^ 1);
      if (kt + 2 < nk) NODE_LOAD(kt + 2);
    }
    const __bf16* as = lds + cur * kBuf;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int gb = wm * 2 + i;  // block 0 multiplies weight slot 0, blocks 1-3 slot 1
      const __bf16* bs = as + kBufA + (gb == 0 ? 0 : 3 * kPL);
      fmd_bf16x8 av[3];
#pragma unroll
      for (int p = 0; p < 3; ++p) av[p] = *reinterpret_cast<const fmd_bf16x8*>(as + p * kPL + (gb * 32) * 16 + rd);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        fmd_bf16x8 bv[3];
#pragma unroll
        for (int p = 0; p < 3; ++p)
          bv[p] = *reinterpret_cast<const fmd_bf16x8*>(bs + p * kPL + ((wn * 2 + j) * 32) * 16 + rd);
        acc[i][j] = x3_mfma(av, bv, acc[i][j]);
      }
    }
    __syncthreads();
  }
#undef NODE_LOAD
#undef NODE_STORE
}

// Store a phase's tile: block 0 rows -> d0 (atoms, ld C) for columns < C and -> d0b for columns
// C .. 2C (accumulating when acc0b); blocks 1-3 -> d1 (3N rows, ld C) for columns < C.
__device__ __forceinline__ void tile_store(const fmd_f32x16 (&acc)[2][2], int col0, int64_t atom0, int64_t n_atoms,
                                           int C, float* d0, float* d0b, int acc0b, float* d1) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1, h = lane >> 5, rr = lane & 31;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int gb = wm * 2 + i;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = col0 + (wn * 2 + j) * 32 + rr;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = (v / 4) * 8 + h * 4 + (v % 4);  // row within the block
        const float x = acc[i][j][v];
        if (gb == 0) {
          const int64_t atom = atom0 + r;
          if (atom >= n_atoms) continue;
          if (col < C) {
            if (d0) d0[atom * C + col] = x;
          } else if (col < 2 * C && d0b) {
            float* p = d0b + atom * C + (col - C);
            *p = acc0b ? *p + x : x;
          }
        } else if (d1 && col < C) {
          const int64_t row = 3 * atom0 + (gb - 1) * 32 + r;
          if (row < 3 * n_atoms) d1[row * C + col] = x;
        }
      }
    }
  }
}

__global__ void __launch_bounds__(kThreads) node_fwd_kernel(const float* A0, const float* A1, const float* h0,
                                                            const int32_t* elem, const float* wm0t, const float* wm1t,
                                                            const float* Wc, const float* Wd, const float* wout0,
                                                            const float* wout1, int64_t n_atoms, int C, float* P0,
                                                            float* P1, float* B0, float* B1, float* h0n, float* h1n) {
  __shared__ __attribute__((aligned(16))) __bf16 lds[2 * kBuf];
  const int64_t atom0 = (int64_t)blockIdx.x * kTA;
  fmd_f32x16 acc[2][2];
  const bool vec = h1n != nullptr;
  // phase 1 (ph 0): P = [A0; A1] x [Wm0 | Wm1]; phase 3 (ph 1): [B0 h0; B1 0] x [(Wo0 ; Wsc0) | (Wo1 ; 0)]
  // (K = 2C; the vector rows only when h1n). One loop, so the tile GEMM is instantiated once.
  for (int ph = 0; ph < 2; ++ph) {
    const TileA a = ph == 0 ? TileA{A0, nullptr, A1, C} : TileA{B0, h0, vec ? B1 : nullptr, C};
    const float* w0 = ph == 0 ? wm0t : wout0;
    const float* w1 = ph == 0 ? wm1t : (vec ? wout1 : nullptr);
    const int K = ph == 0 ? C : 2 * C;
    for (int col0 = 0; col0 < C; col0 += 128) {
      tile_gemm(a, w0, w1, K, C, col0, K, atom0, n_atoms, C, lds, acc);
      tile_store(acc, col0, atom0, n_atoms, C, ph == 0 ? P0 : h0n, nullptr, 0, ph == 0 ? P1 : h1n);
    }
    if (ph == 1) break;
    __syncthreads();  // the tile's P rows (global, L2) are complete for the workgroup
    // phase 2: symmetric contraction of the tile's atoms
    for (int k = threadIdx.x; k < kTA * C; k += kThreads) {
      const int64_t i = atom0 + k / C;
      if (i >= n_atoms) continue;
      const int ch = k % C;
      const int el = elem[i];
      const float p0 = P0[i * C + ch];
      const float px = P1[(i * 3 + 0) * C + ch], py = P1[(i * 3 + 1) * C + ch], pz = P1[(i * 3 + 2) * C + ch];
      const float n1 = px * px + py * py + pz * pz;
      B0[i * C + ch] = symcon_b0(p0, n1, Wc + (int64_t)el * 5 * C + ch, C);
      if (vec) {
        const float q = symcon_q(p0, n1, Wd + (int64_t)el * 4 * C + ch, C);
        B1[(i * 3 + 0) * C + ch] = q * px;
        B1[(i * 3 + 1) * C + ch] = q * py;
        B1[(i * 3 + 2) * C + ch] = q * pz;
      }
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(kThreads) node_bwd_kernel(const float* g0, const float* g1, const float* P0,
                                                            const float* P1, const int32_t* elem, const float* wo0st,
                                                            const float* wo1st, const float* Wc, const float* Wd,
                                                            const float* wm0, const float* wm1, int64_t n_atoms, int C,
                                                            float* gB0, float* gB1, float* gin0, int acc_in0,
                                                            float* gP0, float* gP1, float* gA0, float* gA1) {
  __shared__ __attribute__((aligned(16))) __bf16 lds[2 * kBuf];
  const int64_t atom0 = (int64_t)blockIdx.x * kTA;
  fmd_f32x16 acc[2][2];
  // phase 1 (ph 0): [g0; g1] x [(Wo0^T | Wsc0^T) | (Wo1^T | 0)] -> gB0 | g_in0 (columns C .. 2C), gB1;
  // phase 3 (ph 1): [gP0; gP1] x [Wm0^T | Wm1^T] -> gA0, gA1. One loop: one tile GEMM instance.
  for (int ph = 0; ph < 2; ++ph) {
    const TileA a = ph == 0 ? TileA{g0, nullptr, g1, C} : TileA{gP0, nullptr, gP1, C};
    const float* w0 = ph == 0 ? wo0st : wm0;
    const float* w1 = ph == 0 ? (g1 ? wo1st : nullptr) : wm1;
    const int ncols = ph == 0 && gin0 ? 2 * C : C;  // no g_in0: phase 1 stops at gB
    for (int col0 = 0; col0 < ncols; col0 += 128) {
      tile_gemm(a, w0, w1, C, ncols, col0, C, atom0, n_atoms, C, lds, acc);
      if (ph == 0)
        tile_store(acc, col0, atom0, n_atoms, C, gB0, gin0, acc_in0, g1 ? gB1 : nullptr);
      else
        tile_store(acc, col0, atom0, n_atoms, C, gA0, nullptr, 0, gA1);
    }
    if (ph == 1) break;
    __syncthreads();
    // phase 2: contraction VJP
    for (int k = threadIdx.x; k < kTA * C; k += kThreads) {
      const int64_t i = atom0 + k / C;
      if (i >= n_atoms) continue;
      const int ch = k % C;
      const int el = elem[i];
      const float p[3] = {P1[(i * 3 + 0) * C + ch], P1[(i * 3 + 1) * C + ch], P1[(i * 3 + 2) * C + ch]};
      float gb1[3] = {0.f, 0.f, 0.f};
      if (g1) {
        gb1[0] = gB1[(i * 3 + 0) * C + ch];
        gb1[1] = gB1[(i * 3 + 1) * C + ch];
        gb1[2] = gB1[(i * 3 + 2) * C + ch];
      }
      float gp0, gp[3];
      symcon_vjp(P0[i * C + ch], p, Wc + (int64_t)el * 5 * C + ch, Wd + (int64_t)el * 4 * C + ch, C,
                 gB0[i * C + ch], g1 != nullptr, gb1, gp0, gp);
      gP0[i * C + ch] = gp0;
      gP1[(i * 3 + 0) * C + ch] = gp[0];
      gP1[(i * 3 + 1) * C + ch] = gp[1];
      gP1[(i * 3 + 2) * C + ch] = gp[2];
    }
    __syncthreads();
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

extern "C" {

int fmd_mace_node_fwd_f32(const float* A0, const float* A1, const float* h0, const int32_t* elem, const float* wm0t,
                          const float* wm1t, const float* Wc, const float* Wd, const float* wout0, const float* wout1,
                          int64_t n_atoms, int32_t channels, float* P0, float* P1, float* B0, float* B1, float* h0n,
                          float* h1n, hipStream_t stream) {
  FMD_REQUIRE(A0 && A1 && h0 && elem && wm0t && wm1t && Wc && wout0 && P0 && P1 && B0 && h0n && n_atoms >= 0);
  FMD_REQUIRE(!h1n || (Wd && wout1 && B1));
  if (channels % 64 || channels <= 0 || channels > 256) return FMD_EUNSUPPORTED;
  for (const void* p : {(const void*)A0, (const void*)A1, (const void*)h0, (const void*)wm0t, (const void*)wm1t,
                        (const void*)wout0})
    if (!aligned16(p)) return FMD_EUNSUPPORTED;
  if (h1n && !aligned16(wout1)) return FMD_EUNSUPPORTED;
  if (n_atoms == 0) return FMD_OK;
  hipLaunchKernelGGL(node_fwd_kernel, dim3((unsigned)fmd_cdiv(n_atoms, kTA)), dim3(kThreads), 0, stream, A0, A1, h0,
                     elem, wm0t, wm1t, Wc, Wd, wout0, wout1, n_atoms, channels, P0, P1, B0, B1, h0n, h1n);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_mace_node_bwd_f32(const float* g0, const float* g1, const float* P0, const float* P1, const int32_t* elem,
                          const float* wo0st, const float* wo1st, const float* Wc, const float* Wd, const float* wm0,
                          const float* wm1, int64_t n_atoms, int32_t channels, float* gB0, float* gB1, float* gin0,
                          int32_t accumulate_in0, float* gP0, float* gP1, float* gA0, float* gA1, hipStream_t stream) {
  FMD_REQUIRE(g0 && P0 && P1 && elem && wo0st && Wc && Wd && wm0 && wm1 && gB0 && gP0 && gP1 && gA0 && gA1);
  FMD_REQUIRE(!g1 || (wo1st && gB1));
  FMD_REQUIRE(n_atoms >= 0);
  if (channels % 64 || channels <= 0 || channels > 256) return FMD_EUNSUPPORTED;
  for (const void* p : {(const void*)g0, (const void*)wo0st, (const void*)wm0, (const void*)wm1, (const void*)gP0,
                        (const void*)gP1})
    if (!aligned16(p)) return FMD_EUNSUPPORTED;
  if (g1 && (!aligned16(g1) || !aligned16(wo1st))) return FMD_EUNSUPPORTED;
  if (n_atoms == 0) return FMD_OK;
  hipLaunchKernelGGL(node_bwd_kernel, dim3((unsigned)fmd_cdiv(n_atoms, kTA)), dim3(kThreads), 0, stream, g0, g1, P0,
                     P1, elem, wo0st, wo1st, Wc, Wd, wm0, wm1, n_atoms, channels, gB0, gB1, gin0, accumulate_in0, gP0,
                     gP1, gA0, gA1);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
