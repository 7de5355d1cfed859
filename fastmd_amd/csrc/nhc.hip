// (e) Nose-Hoover chain velocity Verlet (ASE NoseHooverChainNVT) on the float64 state.
//
// One workgroup integrates all atoms (no inter-block synchronization): the thermostat chain
// is a handful of fp64 scalars in registers that every thread advances alike, and the only
// reduction, ke2 = sum(p*p/m), is formed per thread in a fixed order, then over the wave by a
// butterfly and over the waves in wave order, so every thread sees the same bits (and computes
// the same chain and momentum scale factor). The operation order follows ASE / the reference port
// (gpu_nhc.py:315-425): p_eta_j sweeps backward, eta update, p scaling by exp(-delta p_eta0/Q0),
// ke2 recomputed, p_eta_j sweep forward; per Suzuki-Yoshida coefficient, tloop times.
// FP contraction is off (each op rounded like NumPy); exp is the HIP device library's.
// Momenta live in registers (KPT <= 4 atoms per thread; at KPT = 4, 1 024 threads, the 128-VGPR
// budget spills a few chain temporaries) up to 4096 atoms; beyond that the multi-block path
// below runs (two grid kernels per half step).
#pragma clang fp contract(off)

#include "common.h"

namespace {

constexpr int kMaxChain = 8;
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / FMD_WAVE;

// Thermostat chain in registers. Every thread of the single-workgroup kernels advances its own
// copy from the same inputs (ke2 reaches every thread with the same bits), so no thread waits
// for another to publish the momentum scale factor. The loops run over the constant index range
// of the arrays with the chain length M as a predicate: every array access has a constant index
// and the arrays stay in registers (one spare slot for the j + 1 read of the last link). The
// chain masses Q and the Suzuki-Yoshida constants are read from the constants vector once, at
// the start of a kernel (uniform loads ahead of its stores): the chain, a serial sequence of
// float64 divisions and exponentials, then waits on no memory.
struct Chain {
  double eta[kMaxChain + 1], pe[kMaxChain + 1], Q[kMaxChain + 1];
  double kT, ndof_kT;
  double delta[3], delta2[3], neg_delta4[3], neg_delta[3];  // per Suzuki-Yoshida sub-step
  int M;
};

__device__ __forceinline__ double sub_step(const double (&v)[3], int k) { return k == 0 ? v[0] : k == 1 ? v[1] : v[2]; }

__device__ __forceinline__ double block_sum(double v, double* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (FMD_WAVE - 1), wave = threadIdx.x / FMD_WAVE;
  __syncthreads();  // red[] may still be read from the previous reduction
  if (lane == 0) red[wave] = v;
  __syncthreads();
  const int nw = (blockDim.x + FMD_WAVE - 1) / FMD_WAVE;
  double s = red[0];
  for (int w = 1; w < nw; ++w) s = s + red[w];
  return s;
}

// ASE _integrate_p_eta_j; j is a constant after unrolling
__device__ __forceinline__ void p_eta_j(Chain& c, int j, double ke2, double delta2, double neg_delta4) {
  double pj = c.pe[j];
  double s = 1.0;
  const bool inner = j < c.M - 1;
  if (inner) {
    s = exp((neg_delta4 * c.pe[j + 1]) / c.Q[j + 1]);
    pj = pj * s;
  }
  double g;
  if (j == 0)
    g = ke2 - c.ndof_kT;
  else
    g = (c.pe[j - 1] * c.pe[j - 1]) / c.Q[j - 1] - c.kT;
  pj = pj + delta2 * g;
  if (inner) pj = pj * s;
  c.pe[j] = pj;
}

// consts: [dt, dt/2, kT, ndof kT, 3 x (delta, delta/2, -delta/4, -delta), Q[0 .. M-1], ...];
// links past M load link M - 1 (in bounds) and hold zeros
__device__ __forceinline__ void load_chain(Chain& c, int M, const double* eta, const double* pe,
                                           const double* consts) {
  c.M = M;
  c.kT = consts[2];
  c.ndof_kT = consts[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    c.delta[k] = consts[4 + 4 * k];
    c.delta2[k] = consts[5 + 4 * k];
    c.neg_delta4[k] = consts[6 + 4 * k];
    c.neg_delta[k] = consts[7 + 4 * k];
  }
#pragma unroll
  for (int j = 0; j <= kMaxChain; ++j) {
    const int jj = j < M ? j : M - 1;
    const double e = eta[jj], p = pe[jj];
    c.Q[j] = consts[16 + jj];
    c.eta[j] = j < M ? e : 0.0;
    c.pe[j] = j < M ? p : 0.0;
  }
}

__device__ __forceinline__ void store_chain(const Chain& c, double* eta, double* pe) {
#pragma unroll
  for (int j = 0; j < kMaxChain; ++j) {
    if (j < c.M) {
      eta[j] = c.eta[j];
      pe[j] = c.pe[j];
    }
  }
}

// Suzuki-Yoshida sub-step k before the momentum scaling: the p_eta_j sweep backward (j = M-1 .. 0),
// the eta update; returns the momentum scale factor exp(-delta p_eta_0 / Q_0)
__device__ __forceinline__ double chain_before_scale(Chain& c, double ke2, int k) {
  const double delta = sub_step(c.delta, k), delta2 = sub_step(c.delta2, k);
  const double neg_delta4 = sub_step(c.neg_delta4, k), neg_delta = sub_step(c.neg_delta, k);
#pragma unroll
  for (int j = kMaxChain - 1; j >= 0; --j)
    if (j < c.M) p_eta_j(c, j, ke2, delta2, neg_delta4);
#pragma unroll
  for (int j = 0; j < kMaxChain; ++j)
    if (j < c.M) c.eta[j] = c.eta[j] + (delta * c.pe[j]) / c.Q[j];
  return exp((neg_delta * c.pe[0]) / c.Q[0]);
}

// ... and after it, with the new ke2: the p_eta_j sweep forward (j = 0 .. M-1)
__device__ __forceinline__ void chain_after_scale(Chain& c, double ke2, int k) {
  const double delta2 = sub_step(c.delta2, k), neg_delta4 = sub_step(c.neg_delta4, k);
#pragma unroll
  for (int j = 0; j < kMaxChain; ++j)
    if (j < c.M) p_eta_j(c, j, ke2, delta2, neg_delta4);
}

// Momentum storage: registers (KPT > 0) or global memory (KPT == 0).
template <int KPT>
struct Momenta {
  double p[KPT > 0 ? KPT : 1][3];
  double mv[KPT > 0 ? KPT : 1];  // the atoms' masses (registers: ke2 is summed once per sub-step)
  double* gp;
  const double* m;
  int64_t n;

  __device__ void load(double* p_ptr, const double* masses, int64_t n_atoms) {
    gp = p_ptr;
    m = masses;
    n = n_atoms;
    if constexpr (KPT > 0) {
#pragma unroll
      for (int r = 0; r < KPT; ++r) {
        const int64_t a = threadIdx.x + (int64_t)r * blockDim.x;
#pragma unroll
        for (int d = 0; d < 3; ++d) p[r][d] = a < n ? p_ptr[3 * a + d] : 0.0;
        mv[r] = a < n ? masses[a] : 1.0;
      }
    }
  }
  template <typename F>
  __device__ __forceinline__ void for_each(F f) {  // f(atom, double (&)[3] p)
    if constexpr (KPT > 0) {
#pragma unroll
      for (int r = 0; r < KPT; ++r) {
        const int64_t a = threadIdx.x + (int64_t)r * blockDim.x;
        if (a < n) f(a, p[r]);
      }
    } else {
      for (int64_t a = threadIdx.x; a < n; a += blockDim.x) {
        double v[3] = {gp[3 * a], gp[3 * a + 1], gp[3 * a + 2]};
        f(a, v);
        gp[3 * a] = v[0];
        gp[3 * a + 1] = v[1];
        gp[3 * a + 2] = v[2];
      }
    }
  }
  __device__ void store() {
    if constexpr (KPT > 0) {
#pragma unroll
      for (int r = 0; r < KPT; ++r) {
        const int64_t a = threadIdx.x + (int64_t)r * blockDim.x;
        if (a < n) {
#pragma unroll
          for (int d = 0; d < 3; ++d) gp[3 * a + d] = p[r][d];
        }
      }
    }
  }
};

template <int KPT>
__device__ double ke2_of(Momenta<KPT>& mom, double* red) {
  static_assert(KPT > 0, "the single-workgroup kernels keep the momenta in registers");
  double s = 0.0;
#pragma unroll
  for (int r = 0; r < KPT; ++r) {
    const int64_t a = threadIdx.x + (int64_t)r * blockDim.x;
    if (a >= mom.n) continue;
    const double(&p)[3] = mom.p[r];
    const double m = mom.mv[r];
    s = s + (p[0] * p[0]) / m;
    s = s + (p[1] * p[1]) / m;
    s = s + (p[2] * p[2]) / m;
  }
  return block_sum(s, red);
}

// ASE integrate_nhc over half a time step (every thread advances its copy of the chain), from
// ke2 = sum(p*p/m) of the momenta on entry; returns that sum of the momenta on return (the
// recomputation after the last scaling: a pre half that follows directly starts from it).
template <int KPT>
__device__ double nhc_half(Momenta<KPT>& mom, Chain& c, int tloop, double* red, double ke2) {
  for (int tl = 0; tl < tloop; ++tl) {
    for (int k = 0; k < 3; ++k) {
      const double scale = chain_before_scale(c, ke2, k);
      mom.for_each([&](int64_t, double (&p)[3]) {
        p[0] = p[0] * scale;
        p[1] = p[1] * scale;
        p[2] = p[2] * scale;
      });
      ke2 = ke2_of(mom, red);
      chain_after_scale(c, ke2, k);
    }
  }
  return ke2;
}

__device__ __forceinline__ double kick_of(double dt2, double f, int f32_kick) {
  if (f32_kick) return (double)((float)dt2 * (float)f);
  return dt2 * f;
}

template <int KPT>
__global__ void __launch_bounds__(kThreads) nhc_pre_kernel(double* q, double* p, const double* f, const double* masses,
                                                           double* eta, double* pe, const double* consts, int64_t n,
                                                           int M, int tloop, int f32_kick) {
  __shared__ double red[kWaves];
  Chain c;
  load_chain(c, M, eta, pe, consts);
  Momenta<KPT> mom;
  mom.load(p, masses, n);
  nhc_half(mom, c, tloop, red, ke2_of(mom, red));
  const double dt = consts[0], dt2 = consts[1];
  mom.for_each([&](int64_t a, double (&pv)[3]) {
    const double m = masses[a];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      pv[d] = pv[d] + kick_of(dt2, f[3 * a + d], f32_kick);
      q[3 * a + d] = q[3 * a + d] + (dt * pv[d]) / m;
    }
  });
  mom.store();
  if (threadIdx.x == 0) store_chain(c, eta, pe);
}

template <int KPT>
__global__ void __launch_bounds__(kThreads) nhc_post_kernel(double* p, const void* f_in, int f_in_64, double* f_cache,
                                                            const double* masses, double* eta, double* pe,
                                                            const double* consts, const void* e_in, int e_kind,
                                                            double* e_out, int64_t n, int M, int tloop, int f32_kick) {
  __shared__ double red[kWaves];
  Chain c;
  load_chain(c, M, eta, pe, consts);
  Momenta<KPT> mom;
  mom.load(p, masses, n);
  const double dt2 = consts[1];
  mom.for_each([&](int64_t a, double (&pv)[3]) {
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const double fv = f_in_64 ? static_cast<const double*>(f_in)[3 * a + d]
                                : (double)static_cast<const float*>(f_in)[3 * a + d];
      pv[d] = pv[d] + kick_of(dt2, fv, f32_kick);
      f_cache[3 * a + d] = fv;
    }
  });
  nhc_half(mom, c, tloop, red, ke2_of(mom, red));
  mom.store();
  if (threadIdx.x == 0) store_chain(c, eta, pe);
  if (threadIdx.x == 0 && e_kind != 0)
    e_out[0] = e_kind == 2 ? static_cast<const double*>(e_in)[0] : (double)static_cast<const float*>(e_in)[0];
}


// Step n's post-force half followed by step n + 1's pre-force half in one launch (consecutive in a
// window of steps): momenta and chain stay in registers between the halves; every operation is
// the one nhc_post_kernel and nhc_pre_kernel perform, in the same order (the same bits), the pre
// half's kick reading the forces the post half just cached.
template <int KPT>
__global__ void __launch_bounds__(kThreads) nhc_post_pre_kernel(double* q, double* p, const void* f_in, int f_in_64,
                                                                double* f_cache, const double* masses, double* eta,
                                                                double* pe, const double* consts, const void* e_in,
                                                                int e_kind, double* e_out, int64_t n, int M, int tloop,
                                                                int f32_kick) {
  __shared__ double red[kWaves];
  Chain c;
  load_chain(c, M, eta, pe, consts);
  Momenta<KPT> mom;
  mom.load(p, masses, n);
  const double dt = consts[0], dt2 = consts[1];
  mom.for_each([&](int64_t a, double (&pv)[3]) {
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const double fv = f_in_64 ? static_cast<const double*>(f_in)[3 * a + d]
                                : (double)static_cast<const float*>(f_in)[3 * a + d];
      pv[d] = pv[d] + kick_of(dt2, fv, f32_kick);
      f_cache[3 * a + d] = fv;
    }
  });
  const double ke2 = nhc_half(mom, c, tloop, red, ke2_of(mom, red));
  if (threadIdx.x == 0 && e_kind != 0)
    e_out[0] = e_kind == 2 ? static_cast<const double*>(e_in)[0] : (double)static_cast<const float*>(e_in)[0];
  nhc_half(mom, c, tloop, red, ke2);  // the same momenta: the post half's last sum
  mom.for_each([&](int64_t a, double (&pv)[3]) {
    const double m = masses[a];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      pv[d] = pv[d] + kick_of(dt2, f_cache[3 * a + d], f32_kick);
      q[3 * a + d] = q[3 * a + d] + (dt * pv[d]) / m;
    }
  });
  mom.store();
  if (threadIdx.x == 0) store_chain(c, eta, pe);
}


// ------------------------------------------------------------------------------------------
// Multi-block path (systems beyond the register path): a half step is two grid kernels --
// per-block partial sums of p*p/m (fixed order), after which the last workgroup to finish
// reduces them in block order and integrates the chain, recording the momentum scale factor of
// every Suzuki-Yoshida sub-step -> an elementwise pass multiplies p by those factors in sequence
// (the same roundings as the single-workgroup path). After a scaling, ke2 is updated as ke2 * s^2 instead of a new
// reduction (the reference's "scaled" ke2 update, gpu_nhc.py:520-706), which differs from the
// recomputed sum in the last bits only.
// work layout (float64): [0, kMaxScales) scale factors, then the block partials.
// ------------------------------------------------------------------------------------------
constexpr int kMbThreads = 256;
constexpr int kMaxScales = 3 * 16;

// p times the nscale factors in sequence; one Suzuki-Yoshida loop (three factors, the usual
// case) from registers the caller loaded before its atom's loads
__device__ __forceinline__ double apply_scales(double pv, const double (&s3)[3], int nscale, const double* work) {
  if (nscale == 3) return ((pv * s3[0]) * s3[1]) * s3[2];
  for (int k = 0; k < nscale; ++k) pv = pv * work[k];
  return pv;
}

__device__ __forceinline__ double block_sum_mb(double v, double* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & (FMD_WAVE - 1), wave = threadIdx.x / FMD_WAVE;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  double s = red[0];
  for (int w = 1; w < (int)(blockDim.x / FMD_WAVE); ++w) s = s + red[w];
  return s;
}

// ke2 from the partials (lane-strided, then the wave sum: a fixed order), the chain half step
// and the scale factors; run by one wave (its lane 0 does the chain)
__device__ __forceinline__ void mb_chain(double* eta, double* pe, const double* consts, int M, int tloop,
                                         int64_t nblocks, double* work) {
  const int lane = threadIdx.x & (FMD_WAVE - 1);
  double s = 0.0;
  for (int64_t b = lane; b < nblocks; b += FMD_WAVE) s = s + work[kMaxScales + b];
  s = wave_sum(s);
  if (lane != 0) return;
  Chain c;
  load_chain(c, M, eta, pe, consts);
  double ke2 = s;
  int ns = 0;
  for (int tl = 0; tl < tloop; ++tl) {
    for (int k = 0; k < 3; ++k) {
      const double scale = chain_before_scale(c, ke2, k);
      work[ns++] = scale;
      ke2 = ke2 * (scale * scale);
      chain_after_scale(c, ke2, k);
    }
  }
  store_chain(c, eta, pe);
}

// p += kick (post half: kick first, cache F) then the block partial of p*p/m; the chain half
// step is run by the workgroup that finishes last (a completion counter after the partials; every workgroup publishes its partial
// with a device-scope fence before it counts itself, the last one fences again before it reads
// them, then sets the counter back to zero for the next launch): a half step is this launch and
// the elementwise pass.
__global__ void __launch_bounds__(kMbThreads) nhc_mb_partials_chain_kernel(
    double* p, const void* f_in, int f_in_64, double* f_cache, const double* masses, const double* consts, int kick,
    int f32_kick, int64_t n, double* work, unsigned int* counter, double* eta, double* pe, int M, int tloop) {
  __shared__ double red[kMbThreads / FMD_WAVE];
  __shared__ int last;
  const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  double s = 0.0;
  if (a < n) {
    const double m = masses[a];
    const double dt2 = consts[1];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      double pv = p[3 * a + d];
      if (kick) {
        const double fv = f_in_64 ? static_cast<const double*>(f_in)[3 * a + d]
                                  : (double)static_cast<const float*>(f_in)[3 * a + d];
        pv = pv + kick_of(dt2, fv, f32_kick);
        p[3 * a + d] = pv;
        f_cache[3 * a + d] = fv;
      }
      s = s + (pv * pv) / m;
    }
  }
  s = block_sum_mb(s, red);
  if (threadIdx.x == 0) {
    work[kMaxScales + blockIdx.x] = s;
    __threadfence();
    last = atomicAdd(counter, 1u) == gridDim.x - 1 ? 1 : 0;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (threadIdx.x < FMD_WAVE) mb_chain(eta, pe, consts, M, tloop, gridDim.x, work);
  if (threadIdx.x == 0) atomicExch(counter, 0u);
}

// p *= scale factors in sequence; pre half: then kick with the cached F and drift
__global__ void __launch_bounds__(kMbThreads) nhc_mb_apply_kernel(double* q, double* p, const double* f,
                                                                  const double* masses, const double* consts,
                                                                  int nscale, int pre, int f32_kick, int64_t n,
                                                                  const double* work, const void* e_in, int e_kind,
                                                                  double* e_out) {
  const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (a == 0 && e_kind != 0)
    e_out[0] = e_kind == 2 ? static_cast<const double*>(e_in)[0] : (double)static_cast<const float*>(e_in)[0];
  if (a >= n) return;
  const double s3[3] = {work[0], work[1], work[2]};
  const double m = masses[a];
  const double dt = consts[0], dt2 = consts[1];
#pragma unroll
  for (int d = 0; d < 3; ++d) {
    double pv = apply_scales(p[3 * a + d], s3, nscale, work);
    if (pre) {
      pv = pv + kick_of(dt2, f[3 * a + d], f32_kick);
      q[3 * a + d] = q[3 * a + d] + (dt * pv) / m;
    }
    p[3 * a + d] = pv;
  }
}

// The multi-block form of the same pair: between nhc_mb_partials_chain_kernel (post half: kick,
// partials, chain) and nhc_mb_apply_kernel (pre half: scales, kick, drift), one launch applies the
// post half's scales to p and forms the pre half's partials from the scaled p, its last workgroup
// running the pre half's chain (the work the post half's apply launch and the pre half's partials
// launch did, in the same order: the same bits). The last workgroup overwrites the scale factors
// only after every workgroup has read them (each reads them before it counts itself).
__global__ void __launch_bounds__(kMbThreads) nhc_mb_apply_partials_chain_kernel(
    double* p, const double* masses, const double* consts, int nscale, int64_t n, double* work, unsigned int* counter,
    double* eta, double* pe, int M, int tloop, const void* e_in, int e_kind, double* e_out) {
  __shared__ double red[kMbThreads / FMD_WAVE];
  __shared__ int last;
  const int64_t a = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (a == 0 && e_kind != 0)
    e_out[0] = e_kind == 2 ? static_cast<const double*>(e_in)[0] : (double)static_cast<const float*>(e_in)[0];
  double s = 0.0;
  if (a < n) {
    const double s3[3] = {work[0], work[1], work[2]};
    const double m = masses[a];
#pragma unroll
    for (int d = 0; d < 3; ++d) {
      const double pv = apply_scales(p[3 * a + d], s3, nscale, work);
      p[3 * a + d] = pv;
      s = s + (pv * pv) / m;
    }
  }
  s = block_sum_mb(s, red);
  if (threadIdx.x == 0) {
    work[kMaxScales + blockIdx.x] = s;
    __threadfence();
    last = atomicAdd(counter, 1u) == gridDim.x - 1 ? 1 : 0;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (threadIdx.x < FMD_WAVE) mb_chain(eta, pe, consts, M, tloop, gridDim.x, work);
  if (threadIdx.x == 0) atomicExch(counter, 0u);
}

unsigned int* mb_counter(double* work, int64_t n) {
  return reinterpret_cast<unsigned int*>(work + kMaxScales + fmd_cdiv(n > 0 ? n : 1, kMbThreads));
}

int pick_kpt(int64_t n, int threads) {
  const int64_t per = fmd_cdiv(n, threads);
  if (per <= 1) return 1;
  if (per <= 2) return 2;
  if (per <= 4) return 4;
  return 0;
}

int nhc_threads(int64_t n) {
  int64_t t = fmd_cdiv(n, FMD_WAVE) * FMD_WAVE;
  return (int)(t < kThreads ? (t < FMD_WAVE ? FMD_WAVE : t) : kThreads);
}

}  // namespace

#define FMD_NHC_DISPATCH(KERNEL, ...)                                                                    \
  switch (kpt) {                                                                                         \
    case 1: hipLaunchKernelGGL(KERNEL<1>, dim3(1), dim3(threads), 0, stream, __VA_ARGS__); break;       \
    case 2: hipLaunchKernelGGL(KERNEL<2>, dim3(1), dim3(threads), 0, stream, __VA_ARGS__); break;       \
    case 4: hipLaunchKernelGGL(KERNEL<4>, dim3(1), dim3(threads), 0, stream, __VA_ARGS__); break;       \
    default: return FMD_EUNSUPPORTED;                                                                    \
  }

extern "C" {

// the completion counter of nhc_mb_partials_chain_kernel: the last float64 slot of `work`
// (zero-initialized by the caller, and zero again after every launch)
int64_t fmd_nhc_work_size(int64_t n_atoms) {
  return kMaxScales + fmd_cdiv(n_atoms > 0 ? n_atoms : 1, kMbThreads) + 1;
}

int fmd_nhc_pre_force(double* q, double* p, const double* f, const double* masses, double* eta, double* p_eta,
                      const double* consts, int64_t n_atoms, int32_t tchain, int32_t tloop, int32_t f32_kick,
                      double* work, hipStream_t stream) {
  FMD_REQUIRE(q && p && f && masses && eta && p_eta && consts && n_atoms > 0);
  FMD_REQUIRE(tchain >= 1 && tchain <= kMaxChain && tloop >= 1);
  const int threads = nhc_threads(n_atoms);
  const int kpt = pick_kpt(n_atoms, threads);
  if (kpt == 0) {
    FMD_REQUIRE(work && 3 * tloop <= kMaxScales);
    const int64_t nb = fmd_cdiv(n_atoms, kMbThreads);
    hipLaunchKernelGGL(nhc_mb_partials_chain_kernel, dim3((unsigned)nb), dim3(kMbThreads), 0, stream, p,
                       (const void*)f, 1, (double*)nullptr, masses, consts, 0, f32_kick, n_atoms, work,
                       mb_counter(work, n_atoms), eta, p_eta, tchain, tloop);
    FMD_CHECK_LAUNCH();
    hipLaunchKernelGGL(nhc_mb_apply_kernel, dim3((unsigned)nb), dim3(kMbThreads), 0, stream, q, p, f, masses, consts,
                       3 * tloop, 1, f32_kick, n_atoms, (const double*)work, (const void*)nullptr, 0, (double*)nullptr);
    FMD_CHECK_LAUNCH();
    return FMD_OK;
  }
  FMD_NHC_DISPATCH(nhc_pre_kernel, q, p, f, masses, eta, p_eta, consts, n_atoms, tchain, tloop, f32_kick);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_nhc_post_force(double* p, const void* f_in, int32_t f_in_is_f64, double* f_cache, const double* masses,
                       double* eta, double* p_eta, const double* consts, const void* e_in, int32_t e_kind,
                       double* e_out, int64_t n_atoms, int32_t tchain, int32_t tloop, int32_t f32_kick, double* work,
                       hipStream_t stream) {
  FMD_REQUIRE(p && f_in && f_cache && masses && eta && p_eta && consts && n_atoms > 0);
  FMD_REQUIRE(tchain >= 1 && tchain <= kMaxChain && tloop >= 1);
  FMD_REQUIRE(e_kind == 0 || (e_in && e_out && (e_kind == 1 || e_kind == 2)));
  const int threads = nhc_threads(n_atoms);
  const int kpt = pick_kpt(n_atoms, threads);
  if (kpt == 0) {
    FMD_REQUIRE(work && 3 * tloop <= kMaxScales);
    const int64_t nb = fmd_cdiv(n_atoms, kMbThreads);
    hipLaunchKernelGGL(nhc_mb_partials_chain_kernel, dim3((unsigned)nb), dim3(kMbThreads), 0, stream, p, f_in,
                       f_in_is_f64, f_cache, masses, consts, 1, f32_kick, n_atoms, work, mb_counter(work, n_atoms),
                       eta, p_eta, tchain, tloop);
    FMD_CHECK_LAUNCH();
    hipLaunchKernelGGL(nhc_mb_apply_kernel, dim3((unsigned)nb), dim3(kMbThreads), 0, stream, (double*)nullptr, p,
                       (const double*)nullptr, masses, consts, 3 * tloop, 0, f32_kick, n_atoms, (const double*)work,
                       e_in, e_kind, e_out);
    FMD_CHECK_LAUNCH();
    return FMD_OK;
  }
  FMD_NHC_DISPATCH(nhc_post_kernel, p, f_in, f_in_is_f64, f_cache, masses, eta, p_eta, consts, e_in, e_kind, e_out,
                   n_atoms, tchain, tloop, f32_kick);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

int fmd_nhc_post_pre(double* q, double* p, const void* f_in, int32_t f_in_is_f64, double* f_cache,
                     const double* masses, double* eta, double* p_eta, const double* consts, const void* e_in,
                     int32_t e_kind, double* e_out, int64_t n_atoms, int32_t tchain, int32_t tloop, int32_t f32_kick,
                     double* work, hipStream_t stream) {
  FMD_REQUIRE(q && p && f_in && f_cache && masses && eta && p_eta && consts && n_atoms > 0);
  FMD_REQUIRE(tchain >= 1 && tchain <= kMaxChain && tloop >= 1);
  FMD_REQUIRE(e_kind == 0 || (e_in && e_out && (e_kind == 1 || e_kind == 2)));
  const int threads = nhc_threads(n_atoms);
  const int kpt = pick_kpt(n_atoms, threads);
  if (kpt == 0) {
    FMD_REQUIRE(work && 3 * tloop <= kMaxScales);
    const int64_t nb = fmd_cdiv(n_atoms, kMbThreads);
    unsigned int* counter = mb_counter(work, n_atoms);
    hipLaunchKernelGGL(nhc_mb_partials_chain_kernel, dim3((unsigned)nb), dim3(kMbThreads), 0, stream, p, f_in,
                       f_in_is_f64, f_cache, masses, consts, 1, f32_kick, n_atoms, work, counter, eta, p_eta, tchain,
                       tloop);
    FMD_CHECK_LAUNCH();
    hipLaunchKernelGGL(nhc_mb_apply_partials_chain_kernel, dim3((unsigned)nb), dim3(kMbThreads), 0, stream, p, masses,
                       consts, 3 * tloop, n_atoms, work, counter, eta, p_eta, tchain, tloop, e_in, e_kind, e_out);
    FMD_CHECK_LAUNCH();
    hipLaunchKernelGGL(nhc_mb_apply_kernel, dim3((unsigned)nb), dim3(kMbThreads), 0, stream, q, p,
                       (const double*)f_cache, masses, consts, 3 * tloop, 1, f32_kick, n_atoms, (const double*)work,
                       (const void*)nullptr, 0, (double*)nullptr);
    FMD_CHECK_LAUNCH();
    return FMD_OK;
  }
  FMD_NHC_DISPATCH(nhc_post_pre_kernel, q, p, f_in, f_in_is_f64, f_cache, masses, eta, p_eta, consts, e_in, e_kind,
                   e_out, n_atoms, tchain, tloop, f32_kick);
  FMD_CHECK_LAUNCH();
  return FMD_OK;
}

}  // extern "C"
