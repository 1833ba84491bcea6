// asm_fft.hip — fused band-limited ASM propagation with hand-written LDS
// FFTs for gfx950 (the per-frame multi-plane forward and adjoint).
//
// A 2-D transform is two 1-D passes.  The zero padding, the transfer
// function multiply-accumulate over planes and the centred crops are folded
// into the passes, so every (plane, wavelength) grid crosses HBM about three
// times instead of the ~12 M x M passes of pad -> FFT (with transposes) ->
// shift -> multiply -> shift -> iFFT -> crop:
//
//   forward  (fields (P,C,H,W) -> hologram (C,S,S)), M = 2S:
//     A  row FFT of the H nonzero rows of each padded field  -> X (PC,H,M)
//     B  per channel and block of 4 columns: for each plane, column FFT of
//        the implicitly padded column, times T[p,c] x aperture, summed over
//        planes; inverse column FFT; keep the S cropped rows  -> Z (C,S,M)
//     C  inverse row FFT of those rows, keep S columns, x 1/M^2 -> hologram
//   adjoint (grad hologram (C,S,S) -> grad fields (P,C,H,W)): the mirror
//     A' row FFT of the S rows -> X (C,S,M); B' column FFT once per channel,
//     then per plane conj(T) x aperture and inverse column FFT, keep H rows
//     -> Z (PC,H,M); C' inverse row FFT, keep W columns, x 1/M^2.
//
// The 1-D FFT is a radix-{2,4,8,3,5,7} Stockham autosort transform on a
// batch of B rows or columns held in LDS: each stage reads all butterfly
// inputs into registers, applies table twiddles (double-precision table,
// rounded to float), does the R-point DFT, and writes the outputs back to
// their Stockham positions between two barriers.  Transform lengths
// without a plan here use the hipFFT path.
#include <hip/hip_runtime.h>

#include <cmath>
#include <map>
#include <mutex>
#include <vector>

#include "fast_trig.h"
#include "hrf_internal.h"

namespace hrf {
namespace {

constexpr int kFftThreads = 512;   // column passes
constexpr int kFftBatch = 4;  // columns per column-pass block; columns of an intermediate tile
// Rows per row-pass block and its threads: four rows in 1024 threads up to
// 1600 points, two in 512 above, where a four-row batch takes 73-147 KB of
// LDS (two or one blocks per CU; two-row blocks measured slower at 1600).
template <int N>
constexpr int kRowBatch = N > 1600 ? 2 : 4;
template <int N>
constexpr int kRowThreads = 256 * kRowBatch<N>;
// Column-pass threads and the occupancy they are compiled for: the longest
// transforms (N >= 3840: a 138-147 KB LDS batch, one block per CU) run
// twice the waves per block, which also halves each thread's share of the
// per-element transfer state.
template <int N>
constexpr int kColThreads = N >= 3840 ? 1024 : kFftThreads;
// Columns per column-pass block: two (half an intermediate tile) above
// 1600 points, where a four-column batch takes 73-147 KB of LDS (one or two
// blocks per CU) and, at 3840/4096, 16 spectrum and transfer entries per
// thread (spilled); four at 1600 and below (two columns measured no faster
// at 1600).
template <int N>
constexpr int kColBatch = N > 1600 ? 2 : kFftBatch;
template <int N>
constexpr int kColMinBlocks = N <= 1600 ? 4 : 2;
constexpr double kTwoPiD = 2.0 * 3.14159265358979323846;

__device__ __forceinline__ float2 cadd(float2 a, float2 b) { return make_float2(a.x + b.x, a.y + b.y); }
__device__ __forceinline__ float2 csub(float2 a, float2 b) { return make_float2(a.x - b.x, a.y - b.y); }
// Twiddle product with explicit fused multiply-adds (the library is built
// with contraction off for the bit-exact geometry code; the transforms only
// need fp32 accuracy).
__device__ __forceinline__ float2 cmulf(float2 a, float2 b) {
  return make_float2(fmaf(a.x, b.x, -(a.y * b.y)), fmaf(a.x, b.y, a.y * b.x));
}
__device__ __forceinline__ float2 cscale(float2 a, float s) { return make_float2(a.x * s, a.y * s); }
// multiply by -i (forward) or +i (inverse)
template <bool INV>
__device__ __forceinline__ float2 mul_mi(float2 a) {
  return INV ? make_float2(-a.y, a.x) : make_float2(a.y, -a.x);
}

template <int R, bool INV>
struct Dft;

template <bool INV>
struct Dft<2, INV> {
  __device__ __forceinline__ static void run(float2 (&x)[2]) {
    const float2 a = x[0], b = x[1];
    x[0] = cadd(a, b);
    x[1] = csub(a, b);
  }
};

template <bool INV>
struct Dft<4, INV> {
  __device__ __forceinline__ static void run(float2 (&x)[4]) {
    const float2 a0 = cadd(x[0], x[2]), a1 = csub(x[0], x[2]);
    const float2 a2 = cadd(x[1], x[3]), a3 = mul_mi<INV>(csub(x[1], x[3]));
    x[0] = cadd(a0, a2);
    x[1] = cadd(a1, a3);
    x[2] = csub(a0, a2);
    x[3] = csub(a1, a3);
  }
};

template <bool INV>
struct Dft<8, INV> {
  __device__ __forceinline__ static void run(float2 (&x)[8]) {
    float2 e[4] = {x[0], x[2], x[4], x[6]};
    float2 o[4] = {x[1], x[3], x[5], x[7]};
    Dft<4, INV>::run(e);
    Dft<4, INV>::run(o);
    // o1 * e^{-/+ i pi/4} and o3 * e^{-/+ 3i pi/4}: two adds and two
    // multiplies each.
    constexpr float c = 0.70710678118654752f;
    const float2 o1 = INV ? make_float2((o[1].x - o[1].y) * c, (o[1].x + o[1].y) * c)
                          : make_float2((o[1].x + o[1].y) * c, (o[1].y - o[1].x) * c);
    const float2 o3 = INV ? make_float2(-(o[3].x + o[3].y) * c, (o[3].x - o[3].y) * c)
                          : make_float2((o[3].y - o[3].x) * c, -(o[3].x + o[3].y) * c);
    const float2 o2 = mul_mi<INV>(o[2]);
    x[0] = cadd(e[0], o[0]);
    x[4] = csub(e[0], o[0]);
    x[1] = cadd(e[1], o1);
    x[5] = csub(e[1], o1);
    x[2] = cadd(e[2], o2);
    x[6] = csub(e[2], o2);
    x[3] = cadd(e[3], o3);
    x[7] = csub(e[3], o3);
  }
};

// DFT-8 of inputs that are zero at t = 0, 1, 6, 7 (the first stage of a
// transform whose nonzero input lies in [N/4, 3N/4)): the two DFT-4 halves
// of (0, a, c, 0) reduce to sums and differences of a and c.
template <bool INV>
__device__ __forceinline__ void dft8_half(float2 (&x)[8]) {
  const float2 a = x[2], b = x[3], c = x[4], d = x[5];
  const float2 ma = mul_mi<INV>(a), mb = mul_mi<INV>(b);
  float2 e[4] = {cadd(c, a), csub(ma, c), csub(c, a), csub(make_float2(-c.x, -c.y), ma)};
  float2 o[4] = {cadd(d, b), csub(mb, d), csub(d, b), csub(make_float2(-d.x, -d.y), mb)};
  constexpr float k = 0.70710678118654752f;
  const float2 o1 = INV ? make_float2((o[1].x - o[1].y) * k, (o[1].x + o[1].y) * k)
                        : make_float2((o[1].x + o[1].y) * k, (o[1].y - o[1].x) * k);
  const float2 o3 = INV ? make_float2(-(o[3].x + o[3].y) * k, (o[3].x - o[3].y) * k)
                        : make_float2((o[3].y - o[3].x) * k, -(o[3].x + o[3].y) * k);
  const float2 o2 = mul_mi<INV>(o[2]);
  x[0] = cadd(e[0], o[0]);
  x[4] = csub(e[0], o[0]);
  x[1] = cadd(e[1], o1);
  x[5] = csub(e[1], o1);
  x[2] = cadd(e[2], o2);
  x[6] = csub(e[2], o2);
  x[3] = cadd(e[3], o3);
  x[7] = csub(e[3], o3);
}

// DFT-16 as two DFT-8 (even and odd inputs) combined with the twiddles
// w16^k, k < 8.  HALF: the inputs are zero at t < 4 and t >= 12 (the
// first stage of a transform whose nonzero input lies in [N/4, 3N/4)): the
// even and odd halves are then both DFT-8s of inputs zero at 0, 1, 6, 7.
template <bool INV, bool HALF>
__device__ __forceinline__ void dft16(float2 (&x)[16]) {
  float2 e[8], o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (!HALF || (j >= 2 && j <= 5)) {
      e[j] = x[2 * j];
      o[j] = x[2 * j + 1];
    }
  }
  if constexpr (HALF) {
    dft8_half<INV>(e);
    dft8_half<INV>(o);
  } else {
    Dft<8, INV>::run(e);
    Dft<8, INV>::run(o);
  }
  // o[k] * w16^k: k = 2, 6 are the DFT-8's 1/sqrt(2) products, k = 4 is
  // -/+ i, k odd a full complex product with cos/sin(pi k/8).
  constexpr float c1 = 0.92387953251128676f;  // cos(pi/8)
  constexpr float s1 = 0.38268343236508977f;  // sin(pi/8)
  constexpr float h = 0.70710678118654752f;
  const float sg = INV ? 1.0f : -1.0f;
  float2 t[8];
  t[0] = o[0];
  t[1] = cmulf(o[1], make_float2(c1, sg * s1));
  t[2] = INV ? make_float2((o[2].x - o[2].y) * h, (o[2].x + o[2].y) * h)
             : make_float2((o[2].x + o[2].y) * h, (o[2].y - o[2].x) * h);
  t[3] = cmulf(o[3], make_float2(s1, sg * c1));
  t[4] = mul_mi<INV>(o[4]);
  t[5] = cmulf(o[5], make_float2(-s1, sg * c1));
  t[6] = INV ? make_float2(-(o[6].x + o[6].y) * h, (o[6].x - o[6].y) * h)
             : make_float2((o[6].y - o[6].x) * h, -(o[6].x + o[6].y) * h);
  t[7] = cmulf(o[7], make_float2(-c1, sg * s1));
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    x[k] = cadd(e[k], t[k]);
    x[k + 8] = csub(e[k], t[k]);
  }
}
template <bool INV>
struct Dft<16, INV> {
  __device__ __forceinline__ static void run(float2 (&x)[16]) { dft16<INV, false>(x); }
};

// Odd radix by symmetric pairing: X_m = x0 + sum_j cos(2 pi jm/R)(x_j+x_{R-j})
//   -/+ i sum_j sin(2 pi jm/R)(x_j-x_{R-j}),  X_{R-m} with the opposite sign.
template <int R>
struct OddConsts;
template <>
struct OddConsts<3> {
  // only k = 1 occurs for R = 3 (j = m = 1)
  __device__ static constexpr float c(int) { return -0.5f; }
  __device__ static constexpr float s(int) { return 0.86602540378443865f; }
};
template <>
struct OddConsts<5> {
  // index (j*m) mod 5 in 1..4 -> cos/sin(2 pi k / 5)
  __device__ static constexpr float c(int k) {
    return (k == 1 || k == 4) ? 0.30901699437494742f : -0.80901699437494742f;
  }
  __device__ static constexpr float s(int k) {
    return k == 1 ? 0.95105651629515357f
                  : (k == 2 ? 0.58778525229247313f
                            : (k == 3 ? -0.58778525229247313f : -0.95105651629515357f));
  }
};
template <>
struct OddConsts<7> {
  __device__ static constexpr float c(int k) {
    return (k == 1 || k == 6) ? 0.62348980185873353f
                              : ((k == 2 || k == 5) ? -0.22252093395631440f : -0.90096886790241913f);
  }
  __device__ static constexpr float s(int k) {
    return k == 1 ? 0.78183148246802981f
                  : (k == 2 ? 0.97492791218182361f
                            : (k == 3 ? 0.43388373911755812f
                                      : (k == 4 ? -0.43388373911755812f
                                                : (k == 5 ? -0.97492791218182361f
                                                          : -0.78183148246802981f))));
  }
};

template <>
struct OddConsts<9> {
  // cos/sin(2 pi k / 9), k = 0..8 (9 is not prime: j m = 9 at j = m = 3
  // gives k = 0): c(9 - k) = c(k), s(9 - k) = -s(k)
  __device__ static constexpr float c(int k) {
    return k == 0 ? 1.0f
           : (k == 1 || k == 8) ? 0.76604444311897804f
                              : ((k == 2 || k == 7) ? 0.17364817766693035f
                                                    : ((k == 3 || k == 6) ? -0.5f
                                                                          : -0.93969262078590838f));
  }
  __device__ static constexpr float s(int k) {
    return k == 0   ? 0.0f
           : k == 1 ? 0.64278760968653933f
           : k == 2 ? 0.98480775301220806f
           : k == 3 ? 0.86602540378443865f
           : k == 4 ? 0.34202014332566873f
           : k == 5 ? -0.34202014332566873f
           : k == 6 ? -0.86602540378443865f
           : k == 7 ? -0.98480775301220806f
                    : -0.64278760968653933f;
  }
};

template <int R, bool INV>
struct DftOdd {
  __device__ __forceinline__ static void run(float2 (&x)[R]) {
    constexpr int H = (R - 1) / 2;
    float2 sp[H + 1], dm[H + 1];
    float2 x0 = x[0];
    float2 X0 = x0;
#pragma unroll
    for (int j = 1; j <= H; ++j) {
      sp[j] = cadd(x[j], x[R - j]);
      dm[j] = csub(x[j], x[R - j]);
      X0 = cadd(X0, sp[j]);
    }
    float2 out[R];
    out[0] = X0;
#pragma unroll
    for (int m = 1; m <= H; ++m) {
      float2 re = x0, im = make_float2(0.0f, 0.0f);
#pragma unroll
      for (int j = 1; j <= H; ++j) {
        const int k = (j * m) % R;
        re = make_float2(fmaf(OddConsts<R>::c(k), sp[j].x, re.x), fmaf(OddConsts<R>::c(k), sp[j].y, re.y));
        im = make_float2(fmaf(OddConsts<R>::s(k), dm[j].x, im.x), fmaf(OddConsts<R>::s(k), dm[j].y, im.y));
      }
      // X_m = re - i*im (forward), X_{R-m} = re + i*im
      const float2 mi = mul_mi<INV>(im);
      out[m] = cadd(re, mi);
      out[R - m] = csub(re, mi);
    }
#pragma unroll
    for (int t = 0; t < R; ++t) x[t] = out[t];
  }
};
template <bool INV>
struct Dft<3, INV> : DftOdd<3, INV> {};
template <bool INV>
struct Dft<5, INV> : DftOdd<5, INV> {};
template <bool INV>
struct Dft<7, INV> : DftOdd<7, INV> {};
template <bool INV>
struct Dft<9, INV> : DftOdd<9, INV> {};
// DFT-10 by the prime-factor mapping 10 = 2 x 5 (no inner twiddles): input
// n = (5 n1 + 2 n2) mod 10 and output k = (5 k1 + 6 k2) mod 10, i.e. a
// DFT-2 over (x[2j], x[2j+5 mod 10]) for each j, then a DFT-5 over each of
// the two results.
template <bool INV>
struct Dft<10, INV> {
  __device__ __forceinline__ static void run(float2 (&x)[10]) {
    float2 a[5], b[5];
#pragma unroll
    for (int j = 0; j < 5; ++j) {
      const float2 u = x[2 * j], v = x[(2 * j + 5) % 10];
      a[j] = cadd(u, v);
      b[j] = csub(u, v);
    }
    Dft<5, INV>::run(a);
    Dft<5, INV>::run(b);
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      x[(6 * k) % 10] = a[k];
      x[(5 + 6 * k) % 10] = b[k];
    }
  }
};

// LDS layout.  A batch of B transforms of length N is interleaved: element
// i of transform b is at B*i + b, so rows and columns share one layout and
// one thread's butterfly inputs (and outputs) sit at a base address plus a
// stride.  K padding slots follow every 32 elements (K per plan and batch,
// below): the first stage's strided stores then spread over the banks, and
// for every stride that is a multiple of 32 the padded addresses stay a
// base plus a compile-time offset.
template <int K = 4>
__device__ __forceinline__ constexpr int pad(int a) { return a + (a >> 5) * K; }
// Padding slots per 32 elements for a batch of B transforms whose plan
// starts with radix R1: 2 for radix 16 over two transforms, whose first
// stage's 32-word output runs would otherwise put a half-wave's stores on 16
// of the 32 banks (4-way conflicts; config 4's passes 1-2% faster with 2),
// else 4 (at 1600 points, four transforms, 4 measured faster than 2 though
// a half-wave's radix-16 stores then meet 2-way conflicts).
template <int R1, int B>
constexpr int kPadSlots = (R1 == 16 && B == 2) ? 2 : 4;
template <int N, int B = kFftBatch, int K = 4>
constexpr int lds_elems() {
  return pad<K>(B * N - 1) + 1;
}

// Twiddles are stored per stage, in the order the butterflies use them:
// the stage with radix R after NS points have been combined holds
// w(k, t) = exp(-2 pi i t k / (NS R)) at OFF + k (R - 1) + t - 1 for
// k < NS, 1 <= t < R (OFF = sum of NS (R - 1) over the earlier stages; N - 1
// entries in all).  A butterfly then reads its R - 1 twiddles at one base
// address plus constant offsets.
// HALF (first stage only, R = 8 or 16): the inputs at t < R/4 and t >= 3R/4
// are zero and are neither read nor stored by the caller.
template <int N, int R, int NS, bool INV, int OFF, int T, bool HALF, int B, int K>
__device__ __forceinline__ void fft_stage(float2* lds, const float2* __restrict__ tw) {
  static_assert(!HALF || ((R == 8 || R == 16) && NS == 1), "pruned first stage is radix 8 or 16");
  static_assert(B > 0 && (B & (B - 1)) == 0, "the batch is a power of two");
  constexpr int NR = N / R;
  constexpr int NB = B * NR;
  constexpr int BPT = (NB + T - 1) / T;
  constexpr int LS = B * NR;  // load stride between butterfly inputs
  constexpr int SS = B * NS;  // store stride between butterfly outputs
  constexpr bool lin_load = LS % 32 == 0;
  constexpr bool lin_store = SS % 32 == 0 || (NS == 1 && (B * R) % 32 == 0);
  constexpr int LSP = LS / 32 * (32 + K);
  // First stage (NS = 1, B R a multiple of 32): butterfly j's outputs are
  // the B R words from B R j + b on (b < B) at stride B, so the padded
  // address of output t is pad<K>(a0) + pad<K>(t B) (a run of 64 crosses one
  // padding gap, at t B = 32).
  constexpr int SSP = SS % 32 == 0 ? SS / 32 * (32 + K) : SS;
  // The thread index and a zero twiddle offset pass through empty asm
  // statements, so a caller that runs the transform inside a loop (the plane
  // loop of the column passes) cannot hoist this stage's addresses and
  // twiddle loads out of the loop and hold them in registers throughout.
  // Indices are unsigned: the empty asm hides that the thread index is
  // non-negative, and signed division and remainder by the batch and the
  // stage span would cost three or four extra instructions each.
  unsigned tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  int twoff = 0;
  asm volatile("" : "+s"(twoff));
  float2 y[BPT][R];
  int ob[BPT];
#pragma unroll
  for (int u = 0; u < BPT; ++u) {
    const unsigned q = tid + u * T;
    ob[u] = -1;
    if (BPT * T == NB || q < static_cast<unsigned>(NB)) {
      const unsigned j = q / B;  // butterfly index within its transform
      const int k = static_cast<int>(j % NS);
      float2 x[R];
      if (lin_load) {
        const int base = pad<K>(static_cast<int>(q));
#pragma unroll
        for (int t = 0; t < R; ++t)
          if (!HALF || (t >= R / 4 && t < 3 * R / 4)) x[t] = lds[base + t * LSP];
      } else {
#pragma unroll
        for (int t = 0; t < R; ++t)
          if (!HALF || (t >= R / 4 && t < 3 * R / 4))
            x[t] = lds[pad<K>(static_cast<int>(q + t * LS))];
      }
      if (NS > 1) {
        const float2* wk = tw + (twoff + OFF + k * (R - 1) - 1);
#pragma unroll
        for (int t = 1; t < R; ++t) {
          float2 w = wk[t];
          if (INV) w.y = -w.y;
          x[t] = cmulf(x[t], w);
        }
      }
      if constexpr (HALF && R == 8)
        dft8_half<INV>(x);
      else if constexpr (HALF)
        dft16<INV, true>(x);
      else
        Dft<R, INV>::run(x);
#pragma unroll
      for (int t = 0; t < R; ++t) y[u][t] = x[t];
      // Stockham output position (j/NS)*NS*R + k + t*NS, interleaved.
      const int a0 = static_cast<int>(q + B * (j / NS) * NS * (R - 1));
      ob[u] = lin_store ? pad<K>(a0) : a0;
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < BPT; ++u) {
    if (ob[u] >= 0) {
      if (lin_store) {
#pragma unroll
        for (int t = 0; t < R; ++t)
          lds[ob[u] + (SS % 32 == 0 ? t * SSP : pad<K>(t * SS))] = y[u][t];
      } else {
#pragma unroll
        for (int t = 0; t < R; ++t) lds[pad<K>(ob[u] + t * SS)] = y[u][t];
      }
    }
  }
  __syncthreads();
}

template <int T, int B, int K, int N, bool INV, bool HALF, int NS, int OFF, int R, int... Rest>
__device__ __forceinline__ void run_stages(float2* lds, const float2* __restrict__ tw) {
  fft_stage<N, R, NS, INV, OFF, T, HALF && NS == 1, B, K>(lds, tw);
  if constexpr (sizeof...(Rest) > 0)
    run_stages<T, B, K, N, INV, false, NS * R, OFF + NS * (R - 1), Rest...>(lds, tw);
}

// First stage of a transform with its inputs taken from in(pos, b) (pos:
// the input's index within transform b of the batch) instead of a staged
// batch: butterfly j reads pos = j + t N/R, so for each t a wave's lanes
// fetch 64 / B consecutive positions of each of the B transforms, straight
// into the registers the butterfly uses (no LDS store, barrier or LDS read
// of a staged copy).  HALF: as in fft_stage, the inputs at t < R/4 and
// t >= 3R/4 are zero and are not fetched.  The caller guarantees that no
// thread still reads the batch from an earlier phase.
template <int N, int R, bool INV, int T, bool HALF, int B, int K, class In>
__device__ __forceinline__ void fft_stage_in(float2* lds, In& in) {
  static_assert(!HALF || R == 8 || R == 16, "pruned first stage is radix 8 or 16");
  constexpr int NR = N / R;
  constexpr int NB = B * NR;
  constexpr int BPT = (NB + T - 1) / T;
  constexpr bool lin_store = B % 32 == 0 || (B * R) % 32 == 0;
  constexpr int SSP = B % 32 == 0 ? B / 32 * (32 + K) : B;
  unsigned tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
#pragma unroll
  for (int u = 0; u < BPT; ++u) {
    const unsigned q = tid + u * T;
    if (BPT * T == NB || q < static_cast<unsigned>(NB)) {
      const unsigned j = q / B;
      const int b = static_cast<int>(q % B);
      float2 x[R];
#pragma unroll
      for (int t = 0; t < R; ++t)
        if (!HALF || (t >= R / 4 && t < 3 * R / 4)) x[t] = in(static_cast<int>(j) + t * NR, b);
      if constexpr (HALF && R == 8)
        dft8_half<INV>(x);
      else if constexpr (HALF)
        dft16<INV, true>(x);
      else
        Dft<R, INV>::run(x);
      // Stockham output position j R + t, interleaved (NS = 1).
      const int a0 = static_cast<int>(q + B * j * (R - 1));
      if (lin_store) {
        const int ob = pad<K>(a0);
#pragma unroll
        for (int t = 0; t < R; ++t) lds[ob + (B % 32 == 0 ? t * SSP : pad<K>(t * B))] = x[t];
      } else {
#pragma unroll
        for (int t = 0; t < R; ++t) lds[pad<K>(a0 + t * B)] = x[t];
      }
    }
  }
  __syncthreads();
}

// The first stage split in two for a caller that overlaps the loads with
// other work (one butterfly per thread): first_stage_load fetches thread
// q's inputs (the q < B N/R that own a butterfly) into x, first_stage_finish
// transforms and stores them as fft_stage_in does.
template <int N, int R, int T, bool HALF, int B, class In>
__device__ __forceinline__ void first_stage_load(In& in, float2 (&x)[R]) {
  constexpr int NR = N / R;
  static_assert(B * NR <= T, "one butterfly per thread");
  const unsigned q = threadIdx.x;
  if (q < static_cast<unsigned>(B * NR)) {
    const int j = static_cast<int>(q / B), b = static_cast<int>(q % B);
#pragma unroll
    for (int t = 0; t < R; ++t)
      if (!HALF || (t >= R / 4 && t < 3 * R / 4)) x[t] = in(j + t * NR, b);
  }
}
template <int N, int R, bool INV, int T, bool HALF, int B, int K>
__device__ __forceinline__ void first_stage_finish(float2* lds, float2 (&x)[R]) {
  static_assert(!HALF || R == 8 || R == 16, "pruned first stage is radix 8 or 16");
  constexpr int NB = B * (N / R);
  static_assert(NB <= T, "one butterfly per thread");
  constexpr bool lin_store = B % 32 == 0 || (B * R) % 32 == 0;
  constexpr int SSP = B % 32 == 0 ? B / 32 * (32 + K) : B;
  unsigned q = threadIdx.x;
  asm volatile("" : "+v"(q));
  if (q < static_cast<unsigned>(NB)) {
    const unsigned j = q / B;
    if constexpr (HALF && R == 8)
      dft8_half<INV>(x);
    else if constexpr (HALF)
      dft16<INV, true>(x);
    else
      Dft<R, INV>::run(x);
    const int a0 = static_cast<int>(q + B * j * (R - 1));
    if (lin_store) {
      const int ob = pad<K>(a0);
#pragma unroll
      for (int t = 0; t < R; ++t) lds[ob + (B % 32 == 0 ? t * SSP : pad<K>(t * B))] = x[t];
    } else {
#pragma unroll
      for (int t = 0; t < R; ++t) lds[pad<K>(a0 + t * B)] = x[t];
    }
  }
  __syncthreads();
}
template <int T, int B, int K, int N, bool INV, bool HALF, int R, int... Rest>
__device__ __forceinline__ void run_stages_from(float2* lds, const float2* __restrict__ tw,
                                                float2 (&x)[R]) {
  first_stage_finish<N, R, INV, T, HALF, B, K>(lds, x);
  if constexpr (sizeof...(Rest) > 0)
    run_stages<T, B, K, N, INV, false, R, R - 1, Rest...>(lds, tw);
}

template <int T, int B, int K, int N, bool INV, bool HALF, class In, int R, int... Rest>
__device__ __forceinline__ void run_stages_in(float2* lds, const float2* __restrict__ tw, In& in) {
  fft_stage_in<N, R, INV, T, HALF, B, K>(lds, in);
  if constexpr (sizeof...(Rest) > 0)
    run_stages<T, B, K, N, INV, false, R, R - 1, Rest...>(lds, tw);
}

// Last stage of a transform with its outputs handed to out(pos, b, value)
// (pos: the output's index within transform b of the batch) instead of
// stored back: the crop a caller keeps goes straight to memory, with no
// LDS store, no barriers and no LDS read-back.  In the last stage j < NS,
// so butterfly j's outputs are pos = j + t NS: for each t a wave's lanes
// (B consecutive transforms per butterfly) hand over 64 / B consecutive
// positions of each transform.  The caller synchronises before it reuses
// the batch.
template <int N, int R, int NS, bool INV, int OFF, int T, int B, int K, class Out>
__device__ __forceinline__ void fft_stage_out(const float2* lds, const float2* __restrict__ tw,
                                              Out& out) {
  static_assert(NS * R == N, "the last stage of the plan");
  constexpr int NB = B * NS;
  constexpr int BPT = (NB + T - 1) / T;
  constexpr int LS = B * NS;
  constexpr bool lin_load = LS % 32 == 0;
  constexpr int LSP = LS / 32 * (32 + K);
  unsigned tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  int twoff = 0;
  asm volatile("" : "+s"(twoff));
#pragma unroll
  for (int u = 0; u < BPT; ++u) {
    const unsigned q = tid + u * T;
    if (BPT * T == NB || q < static_cast<unsigned>(NB)) {
      const unsigned j = q / B;
      const int b = static_cast<int>(q % B);
      float2 x[R];
      if (lin_load) {
        const int base = pad<K>(static_cast<int>(q));
#pragma unroll
        for (int t = 0; t < R; ++t) x[t] = lds[base + t * LSP];
      } else {
#pragma unroll
        for (int t = 0; t < R; ++t) x[t] = lds[pad<K>(static_cast<int>(q + t * LS))];
      }
      if (NS > 1) {
        const float2* wk = tw + (twoff + OFF + static_cast<int>(j) * (R - 1) - 1);
#pragma unroll
        for (int t = 1; t < R; ++t) {
          float2 w = wk[t];
          if (INV) w.y = -w.y;
          x[t] = cmulf(x[t], w);
        }
      }
      Dft<R, INV>::run(x);
#pragma unroll
      for (int t = 0; t < R; ++t) out(static_cast<int>(j) + t * NS, b, x[t]);
    }
  }
}

template <int T, int B, int K, int N, bool INV, int NS, int OFF, class Out, int R, int... Rest>
__device__ __forceinline__ void run_stages_out(float2* lds, const float2* __restrict__ tw,
                                               Out& out) {
  if constexpr (sizeof...(Rest) > 0) {
    fft_stage<N, R, NS, INV, OFF, T, false, B, K>(lds, tw);
    run_stages_out<T, B, K, N, INV, NS * R, OFF + NS * (R - 1), Out, Rest...>(lds, tw, out);
  } else {
    fft_stage_out<N, R, NS, INV, OFF, T, B, K>(lds, tw, out);
  }
}
// First stage from in(), last stage to out() (plans of two or more stages).
template <int T, int B, int K, int N, bool INV, bool HALF, class In, class Out, int R,
          int... Rest>
__device__ __forceinline__ void run_stages_in_out(float2* lds, const float2* __restrict__ tw,
                                                  In& in, Out& out) {
  static_assert(sizeof...(Rest) > 0, "a plan of two or more stages");
  fft_stage_in<N, R, INV, T, HALF, B, K>(lds, in);
  run_stages_out<T, B, K, N, INV, R, R - 1, Out, Rest...>(lds, tw, out);
}
template <typename... A>
constexpr int first_radix(int r, A...) {
  return r;
}

// The plans (radix sequence per length), shared by the device transforms
// and the host's twiddle tables.
#define HRF_FFT_PLANS(X) \
  X(128, 8, 4, 4)        \
  X(160, 8, 4, 5)        \
  X(192, 8, 8, 3)        \
  X(512, 8, 8, 8)        \
  X(1024, 8, 8, 4, 4)    \
  X(1600, 16, 10, 10)    \
  X(2016, 8, 4, 7, 9)    \
  X(2048, 8, 8, 8, 4)    \
  X(3840, 16, 16, 5, 3)  \
  X(4096, 16, 16, 16)

template <int N>
struct Plan;
#define HRF_FFT_PLAN(NN, ...)                                                       \
  template <>                                                                       \
  struct Plan<NN> {                                                                 \
    template <int B>                                                                \
    static constexpr int kPad = kPadSlots<first_radix(__VA_ARGS__), B>;             \
    template <bool INV, int T = kFftThreads, bool HALF = false, int B = kFftBatch>  \
    __device__ __forceinline__ static void run(float2* lds, const float2* tw) {     \
      run_stages<T, B, kPad<B>, NN, INV, HALF, 1, 0, __VA_ARGS__>(lds, tw);         \
    }                                                                               \
    template <bool INV, int T, bool HALF, int B, class In>                          \
    __device__ __forceinline__ static void run_in(float2* lds, const float2* tw,    \
                                                  In& in) {                         \
      run_stages_in<T, B, kPad<B>, NN, INV, HALF, In, __VA_ARGS__>(lds, tw, in);    \
    }                                                                               \
    static constexpr int kR1 = first_radix(__VA_ARGS__);                            \
    template <int T, bool HALF, int B, class In>                                    \
    __device__ __forceinline__ static void load_first(In& in, float2 (&x)[kR1]) {   \
      first_stage_load<NN, kR1, T, HALF, B>(in, x);                                 \
    }                                                                               \
    template <bool INV, int T, bool HALF, int B>                                    \
    __device__ __forceinline__ static void run_from(float2* lds, const float2* tw,  \
                                                    float2 (&x)[kR1]) {             \
      run_stages_from<T, B, kPad<B>, NN, INV, HALF, __VA_ARGS__>(lds, tw, x);       \
    }                                                                               \
    template <bool INV, int T, bool HALF, int B, class In, class Out>               \
    __device__ __forceinline__ static void run_in_out(float2* lds, const float2* tw,\
                                                      In& in, Out& out) {           \
      run_stages_in_out<T, B, kPad<B>, NN, INV, HALF, In, Out, __VA_ARGS__>(lds, tw,\
                                                                 in, out);          \
    }                                                                               \
    template <bool INV, int T, int B, class Out>                                    \
    __device__ __forceinline__ static void run_out(float2* lds, const float2* tw,   \
                                                   Out& out) {                      \
      run_stages_out<T, B, kPad<B>, NN, INV, 1, 0, Out, __VA_ARGS__>(lds, tw, out); \
    }                                                                               \
  };
HRF_FFT_PLANS(HRF_FFT_PLAN)
#undef HRF_FFT_PLAN

// Plans of the column passes where they differ from the length's: at 4096
// points the column blocks (1024 threads, two transforms) would leave half
// their waves idle in every radix-16 stage (512 butterflies), so they keep
// 8 8 8 8, while the row passes (512 threads) take 16 16 16.
#define HRF_FFT_COL_PLANS(X) X(4096, 8, 8, 8, 8)
template <int N>
struct PlanCol : Plan<N> {};
#define HRF_FFT_PLAN(NN, ...)                                                       \
  template <>                                                                       \
  struct PlanCol<NN> {                                                              \
    template <int B>                                                                \
    static constexpr int kPad = kPadSlots<first_radix(__VA_ARGS__), B>;             \
    template <bool INV, int T = kFftThreads, bool HALF = false, int B = kFftBatch>  \
    __device__ __forceinline__ static void run(float2* lds, const float2* tw) {     \
      run_stages<T, B, kPad<B>, NN, INV, HALF, 1, 0, __VA_ARGS__>(lds, tw);         \
    }                                                                               \
    template <bool INV, int T, bool HALF, int B, class In>                          \
    __device__ __forceinline__ static void run_in(float2* lds, const float2* tw,    \
                                                  In& in) {                         \
      run_stages_in<T, B, kPad<B>, NN, INV, HALF, In, __VA_ARGS__>(lds, tw, in);    \
    }                                                                               \
    static constexpr int kR1 = first_radix(__VA_ARGS__);                            \
    template <int T, bool HALF, int B, class In>                                    \
    __device__ __forceinline__ static void load_first(In& in, float2 (&x)[kR1]) {   \
      first_stage_load<NN, kR1, T, HALF, B>(in, x);                                 \
    }                                                                               \
    template <bool INV, int T, bool HALF, int B>                                    \
    __device__ __forceinline__ static void run_from(float2* lds, const float2* tw,  \
                                                    float2 (&x)[kR1]) {             \
      run_stages_from<T, B, kPad<B>, NN, INV, HALF, __VA_ARGS__>(lds, tw, x);       \
    }                                                                               \
    template <bool INV, int T, bool HALF, int B, class In, class Out>               \
    __device__ __forceinline__ static void run_in_out(float2* lds, const float2* tw,\
                                                      In& in, Out& out) {           \
      run_stages_in_out<T, B, kPad<B>, NN, INV, HALF, In, Out, __VA_ARGS__>(lds, tw,\
                                                                 in, out);          \
    }                                                                               \
    template <bool INV, int T, int B, class Out>                                    \
    __device__ __forceinline__ static void run_out(float2* lds, const float2* tw,   \
                                                   Out& out) {                      \
      run_stages_out<T, B, kPad<B>, NN, INV, 1, 0, Out, __VA_ARGS__>(lds, tw, out); \
    }                                                                               \
  };
HRF_FFT_COL_PLANS(HRF_FFT_PLAN)
#undef HRF_FFT_PLAN

// Host: the radix sequence of a plan (empty for lengths without one); col:
// the column passes' plan.
std::vector<int> plan_radices(int N, bool col) {
#define HRF_FFT_RADICES(NN, ...) \
  if (N == NN) return std::vector<int>{__VA_ARGS__};
  if (col) {
    HRF_FFT_COL_PLANS(HRF_FFT_RADICES)
  }
  HRF_FFT_PLANS(HRF_FFT_RADICES)
#undef HRF_FFT_RADICES
  return {};
}

// Lengths whose twiddle table (N - 1 entries) is copied into LDS at block
// start: it fits beside the batch without costing a block per CU.
template <int N>
constexpr bool kTwInLds = N <= 1600;
template <int N>
constexpr int kTwLdsElems = kTwInLds<N> ? N : 1;

// Copies the table into LDS (when kTwInLds) and returns the pointer the
// transforms read; the caller's next __syncthreads publishes it.
template <int N, int T = kFftThreads>
__device__ __forceinline__ const float2* stage_twiddles(float2* s_tw,
                                                        const float2* __restrict__ tw) {
  if constexpr (kTwInLds<N>) {
    for (int i = threadIdx.x; i < N - 1; i += T) s_tw[i] = tw[i];
    return s_tw;
  } else {
    return tw;
  }
}

// Transfer-function geometry of natural-order spectral element (row i,
// column k): frequencies as torch.fft.fftfreq float32 values and the
// aperture on the fftshifted grid (same mapping as asm_prop.hip).
__device__ __forceinline__ void coords(int i, int kcol, int M, float sfreq, float ap,
                                       float* fxv, float* fyv, bool* inap) {
  const int h = M / 2;
  int kr = i + h;
  if (kr >= M) kr -= M;
  int kc = kcol + h;
  if (kc >= M) kc -= M;
  *fxv = static_cast<float>(kr - h) * sfreq;
  *fyv = static_cast<float>(kc - h) * sfreq;
  bool a = true;
  if (ap > 0.0f) {
    const float off = static_cast<float>(M) / 2.0f - 0.5f;
    const float x = static_cast<float>(kc) - off;
    const float y = static_cast<float>(kr) - off;
    a = x * x + y * y < ap * ap;
  }
  *inap = a;
}

// kz^2 and kz exactly as the reference kernel evaluates them
// (bandlimited_propagation_cuda.cu:60,65-67); kz2 <= 0 -> evanescent.
__device__ __forceinline__ float kz_of(float k, float fxv, float fyv, bool* prop) {
  const double a = kTwoPiD * static_cast<double>(fxv);
  const double b = kTwoPiD * static_cast<double>(fyv);
  const float kz2 = static_cast<float>((static_cast<double>(k * k) - a * a) - b * b);
  *prop = kz2 > 0.0f;
  return *prop ? sqrtf(kz2) : 0.0f;
}

struct AsmFftConsts {
  float k[kMaxChannels];
  float d[kMaxPlanes];
  float fxmax[kMaxPlanes * kMaxChannels];
  float fymax[kMaxPlanes * kMaxChannels];
  // 1 when the band limit of (plane, channel) passes every frequency of the
  // grid (decided on the host with the device's float arithmetic), so the
  // per-element test can be skipped.
  unsigned char band_all[kMaxPlanes * kMaxChannels];
};

// Intermediate spectra are stored tile-major: image `img` (h rows of N
// columns) as N/B column tiles, each h x B with the B columns innermost, at
// ((img * N/B + tile) * h + row) * B + col.  A column pass then reads and
// writes one contiguous h*B*8-byte run per tile, and a row pass touches
// B*B*8 = 128-byte runs.
__device__ __forceinline__ int64_t tile_off(int img, int ncb, int cb, int h, int r, int b, int B) {
  return ((static_cast<int64_t>(img) * ncb + cb) * h + r) * B + b;
}

// A / A': forward FFT of kRowBatch rows of a plain (nimg, h, w_in) image
// placed at column c_in of the zero-padded N-length row -> tiled (nimg, h,
// N).  HALF: [c_in, c_in + w_in) lies in [N/4, 3N/4); only that half is
// staged and the first stage is pruned.
template <int N, bool HALF>
__global__ __launch_bounds__(kRowThreads<N>) void k_rows_in(const float2* __restrict__ src,
                                                         float2* __restrict__ dst, int nimg,
                                                         int h, int w_in, int c_in,
                                                         const float2* __restrict__ tw) {
  constexpr int RB = kRowBatch<N>;  // rows (transforms) of this block
  constexpr int T = kRowThreads<N>;
  constexpr int TB = kFftBatch;     // columns of an intermediate tile
  constexpr int ncb = N / TB;
  __shared__ float2 lds[lds_elems<N, RB, Plan<N>::template kPad<RB>>()];
  __shared__ float2 s_tw[kTwLdsElems<N>];
  const float2* twp = stage_twiddles<N, T>(s_tw, tw);
  const int blocks_per_img = (h + RB - 1) / RB;
  const int img = blockIdx.x / blocks_per_img;
  const int r0 = (blockIdx.x - img * blocks_per_img) * RB;
  // The first stage reads the rows straight from memory: position pos of
  // row rr is column pos - c_in of the image (zero outside [0, w_in)).
  const float2* srow = src + static_cast<int64_t>(img) * h * w_in;
  auto in = [&](int pos, int rr) -> float2 {
    const unsigned col = static_cast<unsigned>(pos - c_in);
    const int r = r0 + rr;
    return (r < h && col < static_cast<unsigned>(w_in))
               ? srow[static_cast<int64_t>(r) * w_in + col]
               : make_float2(0.0f, 0.0f);
  };
  // The last stage stores the spectrum rows tile-major itself (for each
  // output index a wave covers 64 / RB columns of the RB rows: runs of
  // RB TB words, tile cb's rows r0 .. r0 + RB - 1).
  auto out = [&](int pos, int rr, float2 v) {
    const int r = r0 + rr;
    if (r < h) dst[tile_off(img, ncb, pos / TB, h, r, pos % TB, TB)] = v;
  };
  Plan<N>::template run_in_out<false, T, HALF, RB>(lds, twp, in, out);
}

// C / C': inverse FFT of kRowBatch rows of a tiled (nimg, h, N) spectrum;
// keeps columns [c_out, c_out + w_out) times `scale` -> plain (nimg, h,
// w_out).
template <int N>
__global__ __launch_bounds__(kRowThreads<N>) void k_rows_out(const float2* __restrict__ src,
                                                          float2* __restrict__ dst, int nimg,
                                                          int h, int w_out, int c_out,
                                                          float scale,
                                                          const float2* __restrict__ tw) {
  constexpr int RB = kRowBatch<N>;
  constexpr int T = kRowThreads<N>;
  constexpr int TB = kFftBatch;
  constexpr int ncb = N / TB;
  __shared__ float2 lds[lds_elems<N, RB, Plan<N>::template kPad<RB>>()];
  __shared__ float2 s_tw[kTwLdsElems<N>];
  const float2* twp = stage_twiddles<N, T>(s_tw, tw);
  const int blocks_per_img = (h + RB - 1) / RB;
  const int img = blockIdx.x / blocks_per_img;
  const int r0 = (blockIdx.x - img * blocks_per_img) * RB;
  // The first stage reads the tile-major spectrum rows straight from
  // memory, the last stores the kept columns [c_out, c_out + w_out).
  auto in = [&](int pos, int rr) -> float2 {
    const int r = r0 + rr;
    return r < h ? src[tile_off(img, ncb, pos / TB, h, r, pos % TB, TB)]
                 : make_float2(0.0f, 0.0f);
  };
  float2* drow = dst + static_cast<int64_t>(img) * h * w_out;
  auto out = [&](int pos, int rr, float2 v) {
    const unsigned i = static_cast<unsigned>(pos - c_out);
    const int r = r0 + rr;
    if (i < static_cast<unsigned>(w_out) && r < h)
      drow[static_cast<int64_t>(r) * w_out + i] = cscale(v, scale);
  };
  Plan<N>::template run_in_out<true, T, false, RB>(lds, twp, in, out);
}

__device__ __forceinline__ void map_cblock(int bid, int nblk, int* chan, int* cb, int ncb) {
  // XCD-aware: consecutive column tiles of a channel go to one XCD, so the
  // tiles of neighbouring blocks stream through the same L2.
  const int q = nblk >> 3, r = nblk & 7;
  const int x = bid & 7, i = bid >> 3;
  const int logical = (x < r) ? x * (q + 1) + i : r * (q + 1) + (x - r) * q + i;
  *chan = logical / ncb;
  *cb = logical - (*chan) * ncb;
}

// B: forward column pass for one channel and one column tile.  X tiled
// (P*C, H, N) row spectra of the fields (rows r_pad..r_pad+H of the padded
// grid; the other rows are zero); Z tiled (C, S, N) receives rows
// [s_crop, s_crop+S) of iFFTcol(sum_p FFTcol(X[p,c]) * T[p,c] * A), or
// adds them to what Z holds (accumulate != 0).
// HALF: the field rows lie in [N/4, 3N/4); only that half is staged and the
// forward transforms' first stage is pruned.
template <int N, bool HALF>
__global__ __launch_bounds__(kColThreads<N>, kColMinBlocks<N>) void k_col_fwd(
    const float2* __restrict__ X, float2* __restrict__ Z, int P, int C, int H, int r_pad, int S,
    int s_crop, float sfreq, float ap, AsmFftConsts mc, const float2* __restrict__ tw,
    int accumulate) {
  constexpr int B = kColBatch<N>;  // columns of this block
  constexpr int TB = kFftBatch;    // columns of an intermediate tile
  constexpr int T = kColThreads<N>;
  constexpr int ncb = N / TB;
  __shared__ float2 lds[lds_elems<N, B, PlanCol<N>::template kPad<B>>()];
  __shared__ float2 s_tw[kTwLdsElems<N>];
  const float2* twp = stage_twiddles<N, T>(s_tw, tw);
  int c, hb;
  map_cblock(blockIdx.x, gridDim.x, &c, &hb, N / B);
  const int cb = hb / (TB / B), col0 = (hb % (TB / B)) * B;  // tile, first column in it
  const int k0 = hb * B;

  // Row mirrors: the transfer function depends on the row frequency only
  // through its square, and rows i and N - i hold frequencies f and -f
  // exactly, so a slot q = i B + b with i in [0, N/2] owns element q and,
  // for 0 < i < N/2, its mirror (N - i) B + b, both with one kz and one
  // sine and cosine per plane (the values the per-element evaluation gives
  // each).  The aperture (centred between samples) is tested per element:
  // bits 2u and 2u + 1 of amask.  kz is -1 where the evanescent cut or the
  // aperture zeroes the transfer function of both elements for every plane.
  // kSplit: the first plane's first-stage loads are issued before the kz
  // prologue, so its arithmetic overlaps their latency (half-grid inputs at
  // the lengths where the registers the loads hold cost no occupancy).
  constexpr bool kSplit = HALF && (N == 1600 || N == 3840 || N == 4096);
  const float2* src = X + tile_off(c, ncb, cb, H, 0, 0, TB) + col0;
  auto in = [&](int pos, int b) -> float2 {
    const unsigned r = static_cast<unsigned>(pos - r_pad);
    return r < static_cast<unsigned>(H) ? src[r * TB + b] : make_float2(0.0f, 0.0f);
  };
  float2 xin[PlanCol<N>::kR1];
  if constexpr (kSplit) PlanCol<N>::template load_first<T, HALF, B>(in, xin);
  constexpr int NS = (N / 2 + 1) * B;  // slots
  constexpr int SPT = (NS + T - 1) / T;
  static_assert(2 * SPT <= 32, "two aperture bits per slot in one word");
  float kz[SPT];
  float2 acc[SPT], acc2[SPT];
  uint32_t amask = 0;
#pragma unroll
  for (int u = 0; u < SPT; ++u) {
    const int q = threadIdx.x + u * T;
    acc[u] = make_float2(0.0f, 0.0f);
    acc2[u] = make_float2(0.0f, 0.0f);
    kz[u] = -1.0f;
    if (q < NS) {
      const int i = q / B, b = q % B;
      float fxv, fyv;
      bool in1, in2 = false, prop;
      coords(i, k0 + b, N, sfreq, ap, &fxv, &fyv, &in1);
      const float kk = kz_of(mc.k[c], fxv, fyv, &prop);
      if (i != 0 && i != N / 2) {
        float fx2, fy2;
        coords(N - i, k0 + b, N, sfreq, ap, &fx2, &fy2, &in2);
      }
      if (prop && (in1 || in2)) kz[u] = kk;
      amask |= (in1 ? 1u : 0u) << (2 * u) | (in2 ? 1u : 0u) << (2 * u + 1);
    }
  }
  for (int p = 0; p < P; ++p) {
    // The previous plane's reads of the batch end here; the transform's
    // first stage then reads the plane's column tile straight from memory
    // (rows outside [r_pad, r_pad + H) are zero); with kSplit the first
    // plane's loads were issued before the kz prologue.
    __syncthreads();
    src = X + tile_off(p * C + c, ncb, cb, H, 0, 0, TB) + col0;
    if (kSplit && p == 0)
      PlanCol<N>::template run_from<false, T, HALF, B>(lds, twp, xin);
    else
      PlanCol<N>::template run_in<false, T, HALF, B>(lds, twp, in);
    const float fxm = mc.fxmax[p * kMaxChannels + c], fym = mc.fymax[p * kMaxChannels + c];
    const bool band_all = mc.band_all[p * kMaxChannels + c] != 0;
    const float d = mc.d[p];
    // At 1600 points the thread index is opaque per plane: the band-limit
    // coordinates below are then recomputed here rather than hoisted out of
    // the plane loop and held through the transforms, which spilled 66
    // registers with the 16 10 10 plan.  (At the other lengths holding them
    // measured faster.)
    int tid = static_cast<int>(threadIdx.x);
    if constexpr (N == 1600) asm volatile("" : "+v"(tid));
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
      const int q = tid + u * T;
      if (q < NS && kz[u] >= 0.0f) {
        bool within = band_all;
        if (!within) {
          const int i = q / B, b = q % B;
          float fxv, fyv;
          bool inap;
          coords(i, k0 + b, N, sfreq, -1.0f, &fxv, &fyv, &inap);
          within = fabsf(fxv) < fxm && fabsf(fyv) < fym;
        }
        if (within) {
          float sn, cs;
          sincos_big_ff(d * kz[u], &sn, &cs);
          if ((amask >> (2 * u)) & 1u) {
            const float2 x = lds[pad<PlanCol<N>::template kPad<B>>(q)];
            acc[u].x += x.x * cs - x.y * sn;
            acc[u].y += x.x * sn + x.y * cs;
          }
          if ((amask >> (2 * u + 1)) & 1u) {
            const float2 x2 =
                lds[pad<PlanCol<N>::template kPad<B>>((N - q / B) * B + q % B)];
            acc2[u].x += x2.x * cs - x2.y * sn;
            acc2[u].y += x2.x * sn + x2.y * cs;
          }
        }
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < SPT; ++u) {
    const int q = threadIdx.x + u * T;
    if (q < NS) {
      lds[pad<PlanCol<N>::template kPad<B>>(q)] = acc[u];
      const int i = q / B;
      if (i != 0 && i != N / 2) lds[pad<PlanCol<N>::template kPad<B>>((N - i) * B + q % B)] = acc2[u];
    }
  }
  __syncthreads();
  // The inverse transform's last stage stores the kept rows
  // [s_crop, s_crop + S) itself.
  float2* dst = Z + tile_off(c, ncb, cb, S, 0, 0, TB) + col0;
  auto out = [&](int pos, int b, float2 v) {
    const unsigned r = static_cast<unsigned>(pos - s_crop);
    if (r < static_cast<unsigned>(S)) {
      float2* o = dst + r * TB + b;
      *o = accumulate ? cadd(*o, v) : v;
    }
  };
  PlanCol<N>::template run_out<true, T, B>(lds, twp, out);
}

// B': adjoint column pass.  X tiled (C, S, N) row spectra of the padded
// hologram gradient (rows s_pad..s_pad+S of the grid); Z tiled (P*C, H, N)
// receives rows [r_crop, r_crop+H) of iFFTcol(FFTcol(X[c]) conj(T[p,c]) A).
// HALF: the S gradient rows lie in [N/4, 3N/4) (always, with N = 2S); only
// that half is staged and the forward transform's first stage is pruned.
template <int N, bool HALF>
__global__ __launch_bounds__(kColThreads<N>, kColMinBlocks<N>) void k_col_adj(
    const float2* __restrict__ X, float2* __restrict__ Z, int P, int C, int S, int s_pad, int H,
    int r_crop, float sfreq, float ap, AsmFftConsts mc, const float2* __restrict__ tw) {
  constexpr int B = kColBatch<N>;
  constexpr int TB = kFftBatch;
  constexpr int T = kColThreads<N>;
  constexpr int ncb = N / TB;
  __shared__ float2 lds[lds_elems<N, B, PlanCol<N>::template kPad<B>>()];
  __shared__ float2 s_tw[kTwLdsElems<N>];
  const float2* twp = stage_twiddles<N, T>(s_tw, tw);
  int c, hb;
  map_cblock(blockIdx.x, gridDim.x, &c, &hb, N / B);
  const int cb = hb / (TB / B), col0 = (hb % (TB / B)) * B;
  const int k0 = hb * B;

  // The forward transform's first stage reads the column tile straight
  // from memory (rows outside [s_pad, s_pad + S) are zero).
  const float2* src = X + tile_off(c, ncb, cb, S, 0, 0, TB) + col0;
  auto in = [&](int pos, int b) -> float2 {
    const unsigned r = static_cast<unsigned>(pos - s_pad);
    return r < static_cast<unsigned>(S) ? src[r * TB + b] : make_float2(0.0f, 0.0f);
  };
  // kSplit: the first stage's loads are issued before the kz prologue, so
  // its arithmetic overlaps their latency (half-grid inputs at the lengths
  // where the registers the loads hold cost no occupancy).
  constexpr bool kSplit = HALF && (N == 1600 || N == 3840 || N == 4096);
  float2 xin[PlanCol<N>::kR1];
  if constexpr (kSplit)
    PlanCol<N>::template load_first<T, HALF, B>(in, xin);
  else
    PlanCol<N>::template run_in<false, T, HALF, B>(lds, twp, in);
  // Slots own an element and its row mirror, as in k_col_fwd.
  constexpr int NS = (N / 2 + 1) * B;
  constexpr int SPT = (NS + T - 1) / T;
  static_assert(2 * SPT <= 32, "two aperture bits per slot in one word");
  float kz[SPT];
  float2 gs[SPT], gs2[SPT];
  uint32_t amask = 0;
#pragma unroll
  for (int u = 0; u < SPT; ++u) {
    const int q = threadIdx.x + u * T;
    kz[u] = -1.0f;
    if (q < NS) {
      const int i = q / B, b = q % B;
      float fxv, fyv;
      bool in1, in2 = false, prop;
      coords(i, k0 + b, N, sfreq, ap, &fxv, &fyv, &in1);
      const float kk = kz_of(mc.k[c], fxv, fyv, &prop);
      if (i != 0 && i != N / 2) {
        float fx2, fy2;
        coords(N - i, k0 + b, N, sfreq, ap, &fx2, &fy2, &in2);
      }
      if (prop && (in1 || in2)) kz[u] = kk;
      amask |= (in1 ? 1u : 0u) << (2 * u) | (in2 ? 1u : 0u) << (2 * u + 1);
    }
  }
  if constexpr (kSplit) PlanCol<N>::template run_from<false, T, HALF, B>(lds, twp, xin);
#pragma unroll
  for (int u = 0; u < SPT; ++u) {
    const int q = threadIdx.x + u * T;
    gs[u] = make_float2(0.0f, 0.0f);
    gs2[u] = make_float2(0.0f, 0.0f);
    if (q < NS) {
      const int i = q / B, b = q % B;
      gs[u] = lds[pad<PlanCol<N>::template kPad<B>>(q)];
      if (i != 0 && i != N / 2) gs2[u] = lds[pad<PlanCol<N>::template kPad<B>>((N - i) * B + b)];
    }
  }
  for (int p = 0; p < P; ++p) {
    __syncthreads();
    const float fxm = mc.fxmax[p * kMaxChannels + c], fym = mc.fymax[p * kMaxChannels + c];
    const bool band_all = mc.band_all[p * kMaxChannels + c] != 0;
    const float nd = -mc.d[p];
#pragma unroll
    for (int u = 0; u < SPT; ++u) {
      const int q = threadIdx.x + u * T;
      if (q < NS) {
        float2 r = make_float2(0.0f, 0.0f), r2 = make_float2(0.0f, 0.0f);
        if (kz[u] >= 0.0f) {
          bool within = band_all;
          if (!within) {
            const int i = q / B, b = q % B;
            float fxv, fyv;
            bool inap;
            coords(i, k0 + b, N, sfreq, -1.0f, &fxv, &fyv, &inap);
            within = fabsf(fxv) < fxm && fabsf(fyv) < fym;
          }
          if (within) {
            float sn, cs;
            sincos_big_ff(nd * kz[u], &sn, &cs);
            if ((amask >> (2 * u)) & 1u)
              r = make_float2(gs[u].x * cs - gs[u].y * sn, gs[u].x * sn + gs[u].y * cs);
            if ((amask >> (2 * u + 1)) & 1u)
              r2 = make_float2(gs2[u].x * cs - gs2[u].y * sn, gs2[u].x * sn + gs2[u].y * cs);
          }
        }
        lds[pad<PlanCol<N>::template kPad<B>>(q)] = r;
        const int i = q / B;
        if (i != 0 && i != N / 2) lds[pad<PlanCol<N>::template kPad<B>>((N - i) * B + q % B)] = r2;
      }
    }
    __syncthreads();
    // The last stage stores the kept rows [r_crop, r_crop + H) itself; the
    // next plane's barrier orders its LDS reads before the batch is rewritten.
    float2* dst = Z + tile_off(p * C + c, ncb, cb, H, 0, 0, TB) + col0;
    auto out = [&](int pos, int b, float2 v) {
      const unsigned r = static_cast<unsigned>(pos - r_crop);
      if (r < static_cast<unsigned>(H)) dst[r * TB + b] = v;
    };
    PlanCol<N>::template run_out<true, T, B>(lds, twp, out);
  }
}

// ------------------------------------------------------------ host side --
std::mutex g_tw_mu;
std::map<std::pair<int, int>, float2*>& tw_tables() {
  static std::map<std::pair<int, int>, float2*> m;
  return m;
}

// The twiddle table of the length-N plan (col: the column passes' plan),
// built once per device.
int twiddles(int N, const float2** out, bool col = false) {
  int dev = 0;
  HRF_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_tw_mu);
  auto key = std::make_pair(dev, 2 * N + (col ? 1 : 0));
  auto it = tw_tables().find(key);
  if (it != tw_tables().end()) {
    *out = it->second;
    return HRF_OK;
  }
  // Per-stage tables (see fft_stage): w(k, t) = exp(-2 pi i t k / (NS R)),
  // computed in double as exp(-2 pi i m / N) with m = t k N / (NS R).
  std::vector<float2> h;
  h.reserve(N);
  int ns = 1;
  for (int r : plan_radices(N, col)) {
    for (int k = 0; k < ns; ++k)
      for (int t = 1; t < r; ++t) {
        const long long m = static_cast<long long>(t) * k * (N / (ns * r));
        const double a = -kTwoPiD * static_cast<double>(m) / static_cast<double>(N);
        h.push_back(make_float2(static_cast<float>(std::cos(a)),
                                static_cast<float>(std::sin(a))));
      }
    ns *= r;
  }
  if (ns != N || static_cast<int>(h.size()) != N - 1) {
    set_error("internal: FFT plan for %d does not multiply out", N);
    return HRF_ERR_INVALID;
  }
  h.push_back(make_float2(1.0f, 0.0f));  // pad to N entries
  float2* d = nullptr;
  HRF_HIP(hipMalloc(&d, N * sizeof(float2)));
  HRF_HIP(hipMemcpy(d, h.data(), N * sizeof(float2), hipMemcpyHostToDevice));
  tw_tables()[key] = d;
  *out = d;
  return HRF_OK;
}

AsmFftConsts fft_consts(int P, int C, int M, double pitch, const float* wl, const float* dist) {
  AsmFftConsts mc{};
  for (int c = 0; c < C; ++c) mc.k[c] = asm_consts(wl[c], 0.0f, static_cast<float>(pitch), M, M).k;
  for (int p = 0; p < P; ++p) {
    mc.d[p] = dist[p];
    for (int c = 0; c < C; ++c) {
      const AsmConsts a = asm_consts(wl[c], dist[p], static_cast<float>(pitch), M, M);
      mc.fxmax[p * kMaxChannels + c] = a.fx_max;
      mc.fymax[p * kMaxChannels + c] = a.fy_max;
      // |fx| on the grid is at most float(M/2) * (float)(1/(M*pitch)), the
      // value of the most negative bin; the device tests |f| < f_max.
      const float fmax_grid = static_cast<float>(M / 2) *
                              static_cast<float>(1.0 / (static_cast<double>(M) * pitch));
      mc.band_all[p * kMaxChannels + c] = (fmax_grid < a.fx_max && fmax_grid < a.fy_max) ? 1 : 0;
    }
  }
  return mc;
}

// Launches of the four passes for a length-N plan.  Inputs of width w (or
// height h) sit centred in the padded length-N line, at N/2 - w/2; when
// 2w <= N they lie in [N/4, 3N/4) and the pruned first stage is taken.
template <int N>
int pass_rows_in(const float2* src, float2* X, int nimg, int h, int w, const float2* tw,
                 hipStream_t s) {
  const int B = kRowBatch<N>;
  const dim3 grid(nimg * ((h + B - 1) / B));
  if (2 * w <= N)
    hipLaunchKernelGGL((k_rows_in<N, true>), grid, dim3(kRowThreads<N>), 0, s, src, X, nimg, h, w,
                       N / 2 - w / 2, tw);
  else
    hipLaunchKernelGGL((k_rows_in<N, false>), grid, dim3(kRowThreads<N>), 0, s, src, X, nimg, h, w,
                       N / 2 - w / 2, tw);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

// Keeps rows [N/2 - h/2, +h) and columns [N/2 - w/2, +w), times 1/N^2.
template <int N>
int pass_rows_out(const float2* Z, float2* dst, int nimg, int h, int w, const float2* tw,
                  hipStream_t s) {
  const int B = kRowBatch<N>;
  const float scale = static_cast<float>(1.0 / (static_cast<double>(N) * N));
  hipLaunchKernelGGL((k_rows_out<N>), dim3(nimg * ((h + B - 1) / B)), dim3(kRowThreads<N>), 0, s, Z,
                     dst, nimg, h, w, N / 2 - w / 2, scale, tw);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

// B with P transfer functions summed: X (P*C, h_in, N) -> Z (C, h_out, N).
template <int N>
int pass_col_fwd(const float2* X, float2* Z, int P, int C, int h_in, int h_out, float sfreq,
                 float ap, const AsmFftConsts& mc, bool accumulate, hipStream_t s) {
  const float2* tw = nullptr;
  HRF_TRY(twiddles(N, &tw, true));
  const dim3 grid(C * (N / kColBatch<N>)), block(kColThreads<N>);
  if (2 * h_in <= N)
    hipLaunchKernelGGL((k_col_fwd<N, true>), grid, block, 0, s, X, Z, P, C, h_in,
                       N / 2 - h_in / 2, h_out, N / 2 - h_out / 2, sfreq, ap, mc, tw,
                       accumulate ? 1 : 0);
  else
    hipLaunchKernelGGL((k_col_fwd<N, false>), grid, block, 0, s, X, Z, P, C, h_in,
                       N / 2 - h_in / 2, h_out, N / 2 - h_out / 2, sfreq, ap, mc, tw,
                       accumulate ? 1 : 0);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

// B' with P transfer functions applied one by one: X (C, h_in, N) ->
// Z (P*C, h_out, N).
template <int N>
int pass_col_adj(const float2* X, float2* Z, int P, int C, int h_in, int h_out, float sfreq,
                 float ap, const AsmFftConsts& mc, hipStream_t s) {
  const float2* tw = nullptr;
  HRF_TRY(twiddles(N, &tw, true));
  const dim3 grid(C * (N / kColBatch<N>)), block(kColThreads<N>);
  if (2 * h_in <= N)
    hipLaunchKernelGGL((k_col_adj<N, true>), grid, block, 0, s, X, Z, P, C, h_in,
                       N / 2 - h_in / 2, h_out, N / 2 - h_out / 2, sfreq, ap, mc, tw);
  else
    hipLaunchKernelGGL((k_col_adj<N, false>), grid, block, 0, s, X, Z, P, C, h_in,
                       N / 2 - h_in / 2, h_out, N / 2 - h_out / 2, sfreq, ap, mc, tw);
  HRF_LAUNCH_CHECK();
  return HRF_OK;
}

float freq_step_of(int N, double pitch) {
  return static_cast<float>(1.0 / (static_cast<double>(N) * pitch));
}

// The transfer constants with the propagation direction reversed: k_col_fwd
// applies exp(+i d kz) and k_col_adj exp(-i d kz), so negated distances give
// the conjugate transfer function in the one and the plain one in the other.
// The band limits depend on d^2 and stay those of the given distances.
AsmFftConsts fft_consts_reversed(int P, int C, int M, double pitch, const float* wl,
                                 const float* dist) {
  AsmFftConsts mc = fft_consts(P, C, M, pitch, wl, dist);
  for (int p = 0; p < P; ++p) mc.d[p] = -mc.d[p];
  return mc;
}

template <int N>
int run_forward(const float2* fields, int P, int C, int H, int W, int S, double pitch,
                const float* wl, const float* dist, float ap, float2* holo, float2* X, float2* Z,
                hipStream_t s) {
  const float2* tw = nullptr;
  HRF_TRY(twiddles(N, &tw));
  const AsmFftConsts mc = fft_consts(P, C, N, pitch, wl, dist);
  {
    HRF_STAGE("asm_rows_in", s);
    HRF_TRY(pass_rows_in<N>(fields, X, P * C, H, W, tw, s));
  }
  {
    HRF_STAGE("asm_col_fwd", s);
    HRF_TRY(pass_col_fwd<N>(X, Z, P, C, H, S, freq_step_of(N, pitch), ap, mc, false, s));
  }
  {
    HRF_STAGE("asm_rows_out", s);
    HRF_TRY(pass_rows_out<N>(Z, holo, C, S, S, tw, s));
  }
  return HRF_OK;
}

template <int N>
int run_adjoint(const float2* gholo, int P, int C, int H, int W, int S, double pitch,
                const float* wl, const float* dist, float ap, float2* gfields, float2* X,
                float2* Z, hipStream_t s) {
  const float2* tw = nullptr;
  HRF_TRY(twiddles(N, &tw));
  const AsmFftConsts mc = fft_consts(P, C, N, pitch, wl, dist);
  {
    HRF_STAGE("asm_rows_in", s);
    HRF_TRY(pass_rows_in<N>(gholo, X, C, S, S, tw, s));
  }
  {
    HRF_STAGE("asm_col_adj", s);
    HRF_TRY(pass_col_adj<N>(X, Z, P, C, S, H, freq_step_of(N, pitch), ap, mc, s));
  }
  {
    HRF_STAGE("asm_rows_out", s);
    HRF_TRY(pass_rows_out<N>(Z, gfields, P * C, H, W, tw, s));
  }
  return HRF_OK;
}

// Multi-distance forward, (C,H,W) -> (D,C,S,S): the structure of the
// adjoint above with the plain transfer function, one forward column
// transform per group of distances.  X holds (C,H,N); Z holds `group`
// distances' (C,S,N) spectra.
template <int N>
int run_md_forward(const float2* field, int D, int C, int H, int W, int S, double pitch,
                   const float* wl, const float* dist, float ap, float2* out, float2* X,
                   float2* Z, int group, hipStream_t s) {
  const float2* tw = nullptr;
  HRF_TRY(twiddles(N, &tw));
  const int64_t SS = static_cast<int64_t>(S) * S;
  {
    HRF_STAGE("asm_rows_in", s);
    HRF_TRY(pass_rows_in<N>(field, X, C, H, W, tw, s));
  }
  for (int d0 = 0; d0 < D; d0 += group) {
    const int g = D - d0 < group ? D - d0 : group;
    const AsmFftConsts mc = fft_consts_reversed(g, C, N, pitch, wl, dist + d0);
    {
      HRF_STAGE("asm_col_adj", s);
      HRF_TRY(pass_col_adj<N>(X, Z, g, C, H, S, freq_step_of(N, pitch), ap, mc, s));
    }
    {
      HRF_STAGE("asm_rows_out", s);
      HRF_TRY(pass_rows_out<N>(Z, out + d0 * C * SS, g * C, S, S, tw, s));
    }
  }
  return HRF_OK;
}

// Multi-distance adjoint, (D,C,S,S) -> (C,H,W): the structure of the forward
// above with the conjugate transfer function, summed over the distances;
// each group of distances adds its column-pass result into Z (C,H,N).
template <int N>
int run_md_adjoint(const float2* gout, int D, int C, int H, int W, int S, double pitch,
                   const float* wl, const float* dist, float ap, float2* gfield, float2* X,
                   float2* Z, int group, hipStream_t s) {
  const float2* tw = nullptr;
  HRF_TRY(twiddles(N, &tw));
  const int64_t SS = static_cast<int64_t>(S) * S;
  for (int d0 = 0; d0 < D; d0 += group) {
    const int g = D - d0 < group ? D - d0 : group;
    const AsmFftConsts mc = fft_consts_reversed(g, C, N, pitch, wl, dist + d0);
    {
      HRF_STAGE("asm_rows_in", s);
      HRF_TRY(pass_rows_in<N>(gout + d0 * C * SS, X, g * C, S, S, tw, s));
    }
    {
      HRF_STAGE("asm_col_fwd", s);
      HRF_TRY(pass_col_fwd<N>(X, Z, g, C, S, H, freq_step_of(N, pitch), ap, mc, d0 > 0, s));
    }
  }
  {
    HRF_STAGE("asm_rows_out", s);
    HRF_TRY(pass_rows_out<N>(Z, gfield, C, H, W, tw, s));
  }
  return HRF_OK;
}

}  // namespace

bool fused_fft_supported(int M) {
#define HRF_FFT_SUPPORTED(NN, ...) \
  if (M == NN) return true;
  HRF_FFT_PLANS(HRF_FFT_SUPPORTED)
#undef HRF_FFT_SUPPORTED
  return false;
}

// One case per plan: `case NN: return RUNNER<NN> ARGS;` (RUNNER and ARGS
// are defined around each use).
#define HRF_FFT_CASE(NN, ...) \
  case NN:                    \
    return RUNNER<NN> ARGS;

int fused_asm_forward(const float2* fields, int P, int C, int H, int W, int S, double pitch,
                      const float* wl, const float* dist, float ap, float2* holo, float2* X,
                      float2* Z, hipStream_t s) {
#define RUNNER run_forward
#define ARGS (fields, P, C, H, W, S, pitch, wl, dist, ap, holo, X, Z, s)
  switch (2 * S) {
    HRF_FFT_PLANS(HRF_FFT_CASE)
    default:
      break;
  }
#undef ARGS
#undef RUNNER
  set_error("fused ASM: unsupported grid %d", 2 * S);
  return HRF_ERR_INVALID;
}

int fused_asm_adjoint(const float2* gholo, int P, int C, int H, int W, int S, double pitch,
                      const float* wl, const float* dist, float ap, float2* gfields, float2* X,
                      float2* Z, hipStream_t s) {
#define RUNNER run_adjoint
#define ARGS (gholo, P, C, H, W, S, pitch, wl, dist, ap, gfields, X, Z, s)
  switch (2 * S) {
    HRF_FFT_PLANS(HRF_FFT_CASE)
    default:
      break;
  }
#undef ARGS
#undef RUNNER
  set_error("fused ASM: unsupported grid %d", 2 * S);
  return HRF_ERR_INVALID;
}

int fused_md_forward(const float2* field, int D, int C, int H, int W, int S, double pitch,
                     const float* wl, const float* dist, float ap, float2* out, float2* X,
                     float2* Z, int group, hipStream_t s) {
  if (group < 1) {
    set_error("internal: multi-distance group of %d", group);
    return HRF_ERR_INVALID;
  }
#define RUNNER run_md_forward
#define ARGS (field, D, C, H, W, S, pitch, wl, dist, ap, out, X, Z, group, s)
  switch (2 * S) {
    HRF_FFT_PLANS(HRF_FFT_CASE)
    default:
      break;
  }
#undef ARGS
#undef RUNNER
  set_error("fused ASM: unsupported grid %d", 2 * S);
  return HRF_ERR_INVALID;
}

int fused_md_adjoint(const float2* gout, int D, int C, int H, int W, int S, double pitch,
                     const float* wl, const float* dist, float ap, float2* gfield, float2* X,
                     float2* Z, int group, hipStream_t s) {
  if (group < 1) {
    set_error("internal: multi-distance group of %d", group);
    return HRF_ERR_INVALID;
  }
#define RUNNER run_md_adjoint
#define ARGS (gout, D, C, H, W, S, pitch, wl, dist, ap, gfield, X, Z, group, s)
  switch (2 * S) {
    HRF_FFT_PLANS(HRF_FFT_CASE)
    default:
      break;
  }
#undef ARGS
#undef RUNNER
  set_error("fused ASM: unsupported grid %d", 2 * S);
  return HRF_ERR_INVALID;
}
#undef HRF_FFT_CASE

void fused_fft_release_all() {
  std::lock_guard<std::mutex> lock(g_tw_mu);
  for (auto& kv : tw_tables()) (void)hipFree(kv.second);
  tw_tables().clear();
}

}  // namespace hrf
