// Uniform draws from the reference's one global generator, on the host and
// on the device, bit for bit the same stream.  The reference keeps a
// std::mt19937_64 seeded from std::random_device unless manual_seed is
// called (src/cpp/random.h:5-13) and fills a tensor by drawing
// std::uniform_real_distribution<T>(0, 1) element by element on the host,
// then copying to the device (src/cpp/factory.cu:73-83).
//
// Generator: MT19937-64 with the published parameters (Matsumoto and
// Nishimura; the std::mt19937_64 of C++11).  Raw words obey
//   x_{k+312} = x_{k+156} ^ next(x_k, x_{k+1}),
// a draw tempers one raw word, and libstdc++ turns it into T(u) / 2^64,
// kept below 1, then (r * (b - a)) + a.
//
// Device generation in parallel: the one-word step T is linear over GF(2),
// and on every state reached after at least one step P(T) = 0 for its
// characteristic polynomial P (degree 19937).  With g = x^J mod P,
//   x_{k+J+m} = XOR over {i : g_i = 1} of x_{k+i+m},
// so the window of 312 words J steps past a base window is a GF(2)
// correlation of the 20280 raw words that follow the base with the bits of
// g.  A call cuts its draws into substreams of SUB_WORDS raw words; the
// start window of substream w is the base jumped by w * SUB_WORDS, from a
// table g_w = x^(w SUB_WORDS) mod P built once per process on the host.
// Per launch round: one wave steps the 20280 raw words after the base
// (rng_raw_kernel); one wave per (bit chunk, substream) correlates them
// with g_w (rng_jump_kernel); one workgroup per substream runs its
// recurrence half a block (156 words) per step in a producer wave and
// tempers, converts and stores in consumer waves (rng_gen_kernel).
#include <algorithm>
#include <memory>
#include <mutex>
#include <random>

#include "nt_internal.h"
#include "rng_poly.h"

namespace nt {
namespace {

// ------------------------------------------------------------ MT19937-64

constexpr int MT_N = 312;  // state words
constexpr int MT_M = 156;  // middle offset; also half a block
constexpr uint64_t MT_A = 0xB5026F5AA96619E9ull;
constexpr uint64_t MT_UPPER = 0xFFFFFFFF80000000ull; // top 33 bits
constexpr uint64_t MT_LOWER = 0x7FFFFFFFull;         // low 31 bits
constexpr uint64_t MT_F = 6364136223846793005ull;    // seeding multiplier
constexpr int MT_DEGREE = 19937;

// x_{k+312} from x_k, x_{k+1} and x_{k+156}.
__host__ __device__ inline uint64_t mt_next(uint64_t xk, uint64_t xk1,
                                            uint64_t xkm) {
  const uint64_t y = (xk & MT_UPPER) | (xk1 & MT_LOWER);
  return xkm ^ (y >> 1) ^ ((xk1 & 1) ? MT_A : 0);
}

__host__ __device__ inline uint64_t mt_temper(uint64_t z) {
  z ^= (z >> 29) & 0x5555555555555555ull;
  z ^= (z << 17) & 0x71D67FFFEDA60000ull;
  z ^= (z << 37) & 0xFFF7EEE000000000ull;
  z ^= z >> 43;
  return z;
}

// libstdc++ generate_canonical<T, digits>() for a 64-bit engine: one draw,
// T(u) / 2^64 (the conversion rounds to nearest), then the largest T below 1
// if that rounded up to 1.
__host__ __device__ inline float canonical(uint64_t u, float) {
  const float r = float(u) * 0x1p-64f;
  return r >= 1.0f ? 0x1.fffffep-1f : r;
}
__host__ __device__ inline double canonical(uint64_t u, double) {
  const double r = double(u) * 0x1p-64;
  return r >= 1.0 ? 0x1.fffffffffffffp-1 : r;
}

// One draw of uniform_real_distribution<T>(a, b) from raw word x:
// (canonical * (b - a)) + a, span = b - a already rounded to T.
template <class T>
__host__ __device__ inline T uniform_of(uint64_t x, T lo, T span) {
  return canonical(mt_temper(x), T{}) * span + lo;
}

void mt_seed(uint64_t *x, uint64_t s) {
  x[0] = s;
  for (int i = 1; i < MT_N; ++i)
    x[i] = MT_F * (x[i - 1] ^ (x[i - 1] >> 62)) + uint64_t(i);
}

// Replaces the block x_k .. x_{k+311} by x_{k+312} .. x_{k+623}, in place:
// a word past the middle reads the new words of its own block.
void mt_twist(uint64_t *x) {
  for (int k = 0; k < MT_N; ++k)
    x[k] = mt_next(x[k], x[(k + 1) % MT_N], x[(k + MT_M) % MT_N]);
}

// ------------------------------------------------------ device geometry

constexpr int64_t SUB_WORDS = int64_t(MT_N) * 512; // raw words per substream
constexpr int MAX_SUBSTREAMS = 512;                 // per launch round
constexpr int POLY_WORDS = MT_N;                    // 19968 bits >= degree
constexpr int JUMP_CHUNKS = 8;                      // bit ranges per jump
constexpr int CHUNK_WORDS = POLY_WORDS / JUMP_CHUNKS; // 39
constexpr int CHUNK_BITS = CHUNK_WORDS * 64;          // 2496
constexpr int JUMP_SPAN = CHUNK_BITS + MT_N;          // raw words per chunk
constexpr int JUMP_RUN = 6;                           // window words per lane
constexpr int JUMP_LANES = MT_N / JUMP_RUN;           // 52
#ifndef NT_RNG_JUMP_WAVES
#define NT_RNG_JUMP_WAVES 4
#endif
constexpr int JUMP_WAVES = NT_RNG_JUMP_WAVES;         // substreams per group
constexpr int RAW_HALVES = 130;                       // half-blocks of raw
constexpr int RAW_WORDS = RAW_HALVES * MT_M;          // 20280
#ifndef NT_RNG_GEN_BATCH
#define NT_RNG_GEN_BATCH 16
#endif
#ifndef NT_RNG_GEN_THREADS
#define NT_RNG_GEN_THREADS 512
#endif
constexpr int GEN_BATCH = NT_RNG_GEN_BATCH; // half-blocks handed over per barrier
constexpr int GEN_THREADS = NT_RNG_GEN_THREADS; // one producer wave + consumers
static_assert(CHUNK_WORDS * JUMP_CHUNKS == POLY_WORDS, "chunking");
static_assert((JUMP_CHUNKS - 1) * CHUNK_BITS + JUMP_SPAN <= RAW_WORDS,
              "a jump chunk reads past the raw sequence");
static_assert(JUMP_LANES * JUMP_RUN == MT_N && JUMP_LANES <= 64, "lanes");
static_assert(CHUNK_BITS - 1 + JUMP_RUN + (JUMP_LANES - 1) * JUMP_RUN <
                  JUMP_SPAN,
              "a lane's register window stays inside the chunk's raw words");
static_assert(SUB_WORDS % MT_N == 0, "substreams hold whole blocks");
static_assert((GEN_BATCH * MT_M) % 2 == 0, "consumers read word pairs");

// ------------------------------------------------------------- kernels

// x_{k+312} from x_k, the low 32 bits of x_{k+1} (only its low 31 bits and
// bit 0 enter) and x_{k+156}.
__device__ inline uint64_t mt_next_lo(uint64_t xk, uint32_t xk1_lo,
                                      uint64_t xkm) {
  const uint64_t y = (xk & MT_UPPER) | (xk1_lo & MT_LOWER);
  return xkm ^ (y >> 1) ^ ((xk1_lo & 1) ? MT_A : 0);
}

// Lane l receives v of lane (l + 1) mod 64: a DPP wavefront rotate.
__device__ inline uint32_t from_next_lane(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x134 /*wave_rol:1*/,
                                              0xf, 0xf, false));
}

constexpr int HB_LANES = MT_M / 3; // 52 lanes hold a half-block

// A wave holding two consecutive half-blocks of the raw sequence: lane
// l < 52 has words 3l, 3l+1, 3l+2 of each; lanes 52-63 hold zeros (and
// stay zero: the recurrence maps zeros to zero).
struct HalfBlocks {
  uint64_t a[3], b[3]; // half-blocks t-2 and t-1
  uint32_t nx;         // low half of word 3l+3 of a

  __device__ void load(const uint64_t *win, int l) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      a[j] = l < HB_LANES ? win[3 * l + j] : 0;
      b[j] = l < HB_LANES ? win[MT_M + 3 * l + j] : 0;
    }
    set_nx(l, from_next_lane(uint32_t(a[0])), b[0]);
  }

  // Word 3l+3 of a is the next lane's first word; for l = 51 it is word
  // 156, b's first word, held by lane 0.
  __device__ void set_nx(int l, uint32_t next_first, uint64_t b0) {
    const uint32_t z = __builtin_amdgcn_readfirstlane(int(uint32_t(b0)));
    nx = l == HB_LANES - 1 ? z : (l < HB_LANES - 1 ? next_first : 0u);
  }

  // Half-block t into c; then (a, b) = (b, c).  The lane exchange for the
  // next step reads b, known before c.
  __device__ void step(int l, uint64_t (&c)[3]) {
    const uint32_t next_first = from_next_lane(uint32_t(b[0]));
    c[0] = mt_next_lo(a[0], uint32_t(a[1]), b[0]);
    c[1] = mt_next_lo(a[1], uint32_t(a[2]), b[1]);
    c[2] = mt_next_lo(a[2], nx, b[2]);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      a[j] = b[j];
      b[j] = c[j];
    }
    set_nx(l, next_first, b[0]);
  }
};

// Draws 0 .. first-1 come from the current block (words p .. p+first-1);
// next_block, when given, receives the following block (one twist).
template <class T>
__global__ __launch_bounds__(320) void rng_head_kernel(
    const uint64_t *words, int p, int first, T *out, T lo, T span,
    uint64_t *next_block) {
  __shared__ uint64_t nb[MT_N];
  const int t = threadIdx.x;
  if (t < first)
    out[t] = uniform_of<T>(words[p + t], lo, span);
  if (next_block == nullptr)
    return;
  if (t < MT_M)
    nb[t] = mt_next(words[t], words[t + 1], words[t + MT_M]);
  __syncthreads();
  if (t >= MT_M && t < MT_N)
    nb[t] = mt_next(words[t], t + 1 < MT_N ? words[t + 1] : nb[0],
                    nb[t - MT_M]);
  __syncthreads();
  if (t < MT_N)
    next_block[t] = nb[t];
}

// raw[0 .. RAW_WORDS) = the raw words from the base window on: one wave
// stepping half-blocks in registers.
__global__ __launch_bounds__(64) void rng_raw_kernel(const uint64_t *base,
                                                     uint64_t *raw) {
  const int l = threadIdx.x;
  HalfBlocks hb;
  hb.load(base, l);
  if (l < HB_LANES)
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      raw[3 * l + j] = hb.a[j];
      raw[MT_M + 3 * l + j] = hb.b[j];
    }
  for (int t = 2; t < RAW_HALVES; ++t) {
    uint64_t c[3];
    hb.step(l, c);
    if (l < HB_LANES)
#pragma unroll
      for (int j = 0; j < 3; ++j)
        raw[int64_t(t) * MT_M + 3 * l + j] = c[j];
  }
}

// partial[(w-1, c)][m] = XOR over the set bits i of g_w in chunk c of
// raw[i + m]: chunk c's share of the start window of substream w.  A
// workgroup loads chunk c's raw words into LDS once for JUMP_WAVES
// substreams, one wave each; lane l owns m = 6l .. 6l+5.  Per 32 bits of g
// the lane loads the 38 words its six m's meet into registers, then each
// set (wave-uniform) bit b costs six 64-bit XORs of registers b .. b+5.
__global__ __launch_bounds__(64 * JUMP_WAVES) void rng_jump_kernel(
    const uint64_t *raw, const uint64_t *polys, uint64_t *partial,
    int jumps) {
  __shared__ uint64_t win[JUMP_SPAN];
  const int c = blockIdx.x;
  const int l = threadIdx.x & 63;
  const int w1 = blockIdx.y * JUMP_WAVES + (threadIdx.x >> 6); // w = w1 + 1
  const int64_t i0 = int64_t(c) * CHUNK_BITS;
  for (int k = threadIdx.x; k < JUMP_SPAN; k += 64 * JUMP_WAVES)
    win[k] = raw[i0 + k];
  __syncthreads();
  if (w1 >= jumps)
    return;
  const int m0 = l < JUMP_LANES ? l * JUMP_RUN : 0;
  const uint32_t *g = reinterpret_cast<const uint32_t *>(
      polys + int64_t(w1) * POLY_WORDS + c * CHUNK_WORDS);
  uint64_t acc[JUMP_RUN], w[32 + JUMP_RUN];
#pragma unroll
  for (int r = 0; r < JUMP_RUN; ++r) {
    acc[r] = 0;
    w[r] = win[m0 + r];
  }
  for (int k = 0; k < 2 * CHUNK_WORDS; ++k) {
    // w[r] = word 32k + m0 + r; the last index read is
    // 32 * 77 + 6 + 306 + 31 = JUMP_SPAN - 1
#pragma unroll
    for (int t = 0; t < 32; ++t)
      w[JUMP_RUN + t] = win[k * 32 + JUMP_RUN + m0 + t];
    const uint32_t bits = g[k]; // little-endian: bits 32k .. 32k+31
#pragma unroll
    for (int b = 0; b < 32; ++b)
      if ((bits >> b) & 1) {
#pragma unroll
        for (int r = 0; r < JUMP_RUN; ++r)
          acc[r] ^= w[b + r];
      }
#pragma unroll
    for (int r = 0; r < JUMP_RUN; ++r)
      w[r] = w[32 + r];
  }
  if (l < JUMP_LANES) {
    uint64_t *dst = partial + (int64_t(w1) * JUMP_CHUNKS + c) * MT_N + m0;
#pragma unroll
    for (int r = 0; r < JUMP_RUN; ++r)
      dst[r] = acc[r];
  }
}

// One workgroup per substream of one round.  Substream w covers raw words
// [w SUB_WORDS, w SUB_WORDS + count) of the round (count = min(SUB_WORDS,
// round_words - w SUB_WORDS)) and writes their draws to out + w SUB_WORDS.
// Wave 0 runs the recurrence in registers and hands GEN_BATCH half-blocks
// per barrier to the other waves through a double buffer in LDS; they temper,
// convert and store.  The last workgroup's producer also writes the block
// starting at local word final_lo to final_words (the generator's new
// state), or, when next_base is given, the window right after its range
// (the next round's base).
template <class T>
__global__ __launch_bounds__(GEN_THREADS) void rng_gen_kernel(
    const uint64_t *base, const uint64_t *partial, int64_t round_words,
    T *out, T lo, T span, uint64_t *final_words, int64_t final_lo,
    uint64_t *next_base) {
  __shared__ __align__(16) uint64_t ring[2][GEN_BATCH * MT_M];
  const int w = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int l = threadIdx.x & 63;
  const bool last = w == int(gridDim.x) - 1;
  const int64_t count =
      round_words - int64_t(w) * SUB_WORDS < SUB_WORDS
          ? round_words - int64_t(w) * SUB_WORDS
          : SUB_WORDS;
  int64_t end = count; // raw words to generate, from the window on
  if (last && final_words)
    end = final_lo + MT_N > end ? final_lo + MT_N : end;
  if (last && next_base)
    end = SUB_WORDS + MT_N;
  const int64_t halves = (end + MT_M - 1) / MT_M;
  const int64_t batches = (halves + GEN_BATCH - 1) / GEN_BATCH;
  uint64_t *keep = last ? (final_words ? final_words : next_base) : nullptr;
  const int64_t keep_lo = final_words ? final_lo : SUB_WORDS;
  T *o = out + int64_t(w) * SUB_WORDS;

  HalfBlocks hb;
  if (wave == 0) {
    if (w == 0) {
      hb.load(base, l);
    } else {
      const uint64_t *pp = partial + int64_t(w - 1) * JUMP_CHUNKS * MT_N;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        hb.a[j] = hb.b[j] = 0;
        if (l < HB_LANES)
          for (int c = 0; c < JUMP_CHUNKS; ++c) {
            hb.a[j] ^= pp[c * MT_N + 3 * l + j];
            hb.b[j] ^= pp[c * MT_N + MT_M + 3 * l + j];
          }
      }
      hb.set_nx(l, from_next_lane(uint32_t(hb.a[0])), hb.b[0]);
    }
  }

  for (int64_t q = 0; q <= batches; ++q) {
    if (wave == 0) {
      if (q < batches) {
        uint64_t *dst = ring[q & 1];
#pragma unroll
        for (int k = 0; k < GEN_BATCH; ++k) {
          const int64_t t = q * GEN_BATCH + k;
          uint64_t c[3];
          if (t == 0) {
#pragma unroll
            for (int j = 0; j < 3; ++j)
              c[j] = hb.a[j];
          } else if (t == 1) {
#pragma unroll
            for (int j = 0; j < 3; ++j)
              c[j] = hb.b[j];
          } else {
            hb.step(l, c);
          }
          if (l < HB_LANES)
#pragma unroll
            for (int j = 0; j < 3; ++j)
              dst[k * MT_M + 3 * l + j] = c[j];
          if (keep && t * MT_M + MT_M > keep_lo && t * MT_M < keep_lo + MT_N &&
              l < HB_LANES)
#pragma unroll
            for (int j = 0; j < 3; ++j) {
              const int64_t at = t * MT_M + 3 * l + j - keep_lo;
              if (at >= 0 && at < MT_N)
                keep[at] = c[j];
            }
        }
      }
    } else if (q > 0) {
      // two words per thread and pass (one 16-byte LDS read)
      const ulonglong2 *src =
          reinterpret_cast<const ulonglong2 *>(ring[(q - 1) & 1]);
      const int64_t p0 = (q - 1) * GEN_BATCH * MT_M;
      for (int j = threadIdx.x - 64; j < GEN_BATCH * MT_M / 2;
           j += GEN_THREADS - 64) {
        const ulonglong2 v = src[j];
        const int64_t pos = p0 + 2 * j;
        if (pos + 1 < count) {
          o[pos] = uniform_of<T>(v.x, lo, span);
          o[pos + 1] = uniform_of<T>(v.y, lo, span);
        } else if (pos < count) {
          o[pos] = uniform_of<T>(v.x, lo, span);
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------- host state

struct Generator {
  std::mutex mu;
  uint64_t x[MT_N];
  int p = MT_N;            // next word of x; MT_N: twist before the next draw
  bool seeded = false;
  bool words_on_device = false; // x lives in dev.words (p stays here)
};

struct DeviceBuffers {
  uint64_t *words = nullptr; // the current block while words_on_device
  uint64_t *base[2] = {nullptr, nullptr};
  uint64_t *raw = nullptr;
  uint64_t *partial = nullptr;
  uint64_t *polys = nullptr;
  int polys_on_device = 0;
};

struct JumpTables {
  bool ready = false;
  std::unique_ptr<gf2::Modulus> mod;
  gf2::Poly step; // x^SUB_WORDS mod P
  std::vector<uint64_t> table; // g_1, g_2, ... POLY_WORDS words each
  int count = 0;
};

Generator &generator() {
  static Generator g;
  return g;
}

void ensure_seeded(Generator &g) {
  if (!g.seeded) {
    mt_seed(g.x, std::random_device{}());
    g.p = MT_N;
    g.seeded = true;
  }
}

DeviceBuffers &device_buffers() {
  static DeviceBuffers d;
  if (!d.words) {
    const size_t n = size_t(MT_N) * 3 + RAW_WORDS +
                     size_t(MAX_SUBSTREAMS - 1) * JUMP_CHUNKS * MT_N +
                     size_t(MAX_SUBSTREAMS - 1) * POLY_WORDS;
    // Held for the life of the process, like the generator itself.
    auto *p = static_cast<uint64_t *>(device_alloc(n * sizeof(uint64_t)));
    d.words = p;
    d.base[0] = p + MT_N;
    d.base[1] = p + 2 * MT_N;
    d.raw = p + 3 * MT_N;
    d.partial = d.raw + RAW_WORDS;
    d.polys = d.partial + size_t(MAX_SUBSTREAMS - 1) * JUMP_CHUNKS * MT_N;
  }
  return d;
}

// XOR over the set bits i of g of seq[i + m], m < MT_N: the window a jump
// by g lands on (host form of rng_jump_kernel, for the table self-check).
void host_jump(const uint64_t *seq, const gf2::Poly &g, uint64_t *win) {
  for (int m = 0; m < MT_N; ++m)
    win[m] = 0;
  for (size_t k = 0; k < g.size(); ++k)
    for (uint64_t bits = g[k]; bits; bits &= bits - 1) {
      const size_t i = k * 64 + size_t(__builtin_ctzll(bits));
      for (int m = 0; m < MT_N; ++m)
        win[m] ^= seq[i + size_t(m)];
    }
}

// The characteristic polynomial from one output bit, and x^SUB_WORDS mod
// it, checked once against stepping the generator SUB_WORDS words.
void build_jump_base(JumpTables &jt) {
  const int64_t nbits = 2 * int64_t(MT_DEGREE) + 64;
  const int64_t nseq = std::max<int64_t>(nbits, SUB_WORDS + RAW_WORDS);
  std::vector<uint64_t> seq(size_t(nseq) + MT_N);
  uint64_t x[MT_N];
  mt_seed(x, 5489u);
  for (int64_t k = 0; k < nseq + MT_N; k += MT_N) {
    mt_twist(x); // every window used below is past one step
    for (int i = 0; i < MT_N && k + i < nseq + MT_N; ++i)
      seq[size_t(k + i)] = x[i];
  }
  std::vector<uint8_t> bits(static_cast<size_t>(nbits), 0);
  for (int64_t k = 0; k < nbits; ++k)
    bits[size_t(k)] = uint8_t(seq[size_t(k)] & 1);
  int deg = 0;
  const gf2::Poly P = gf2::minimal_polynomial(bits, &deg);
  if (deg != MT_DEGREE)
    fail(NT_ERR_RUNTIME, "rng: generator polynomial has degree " +
                             std::to_string(deg));
  jt.mod = std::make_unique<gf2::Modulus>(P, deg);
  jt.step = jt.mod->xpow(uint64_t(SUB_WORDS));
  jt.step.resize(POLY_WORDS, 0);
  uint64_t win[MT_N];
  host_jump(seq.data(), jt.step, win);
  for (int m = 0; m < MT_N; ++m)
    if (win[m] != seq[size_t(SUB_WORDS + m)])
      fail(NT_ERR_RUNTIME, "rng: jump table self-check failed");
  jt.ready = true;
}

JumpTables &jump_tables() {
  static JumpTables jt;
  return jt;
}

// Host tables g_1 .. g_count (no device work).
const JumpTables &host_polys(int count) {
  JumpTables &jt = jump_tables();
  if (!jt.ready)
    build_jump_base(jt);
  while (jt.count < count) {
    gf2::Poly g = jt.count == 0
                      ? jt.step
                      : jt.mod->mul(
                            gf2::Poly(jt.table.end() - POLY_WORDS,
                                      jt.table.end()),
                            jt.step);
    g.resize(POLY_WORDS, 0);
    jt.table.insert(jt.table.end(), g.begin(), g.end());
    ++jt.count;
  }
  return jt;
}

// Makes g_1 .. g_count available on the device.
void ensure_polys(DeviceBuffers &d, int count) {
  if (count <= d.polys_on_device)
    return;
  const JumpTables &jt = host_polys(count);
  const int from = d.polys_on_device;
  NT_HIP_CHECK(hipMemcpy(d.polys + size_t(from) * POLY_WORDS,
                         jt.table.data() + size_t(from) * POLY_WORDS,
                         size_t(count - from) * POLY_WORDS * sizeof(uint64_t),
                         hipMemcpyHostToDevice));
  d.polys_on_device = count;
}

// Brings the generator's words back to the host after device draws.
void words_to_host(Generator &g) {
  if (!g.words_on_device)
    return;
  NT_HIP_CHECK(hipStreamSynchronize(stream()));
  NT_HIP_CHECK(hipMemcpy(g.x, device_buffers().words, sizeof g.x,
                         hipMemcpyDeviceToHost));
  g.words_on_device = false;
}

template <class T>
void host_draws(Generator &g, T *o, int64_t n, T lo, T span) {
  for (int64_t i = 0; i < n; ++i) {
    if (g.p >= MT_N) {
      mt_twist(g.x);
      g.p = 0;
    }
    o[i] = uniform_of<T>(g.x[g.p++], lo, span);
  }
}

template <class T>
void device_draws(Generator &g, T *out, int64_t n, T lo, T span) {
  DeviceBuffers &d = device_buffers();
  hipStream_t s = stream();
  if (!g.words_on_device) {
    NT_HIP_CHECK(hipStreamSynchronize(s));
    NT_HIP_CHECK(
        hipMemcpy(d.words, g.x, sizeof g.x, hipMemcpyHostToDevice));
    g.words_on_device = true;
  }
  const int first = int(std::min<int64_t>(n, MT_N - g.p));
  const int64_t rest = n - first;
  rng_head_kernel<T><<<1, 320, 0, s>>>(d.words, g.p, first, out, lo, span,
                                       rest > 0 ? d.base[0] : nullptr);
  NT_LAUNCH_CHECK();
  if (rest == 0) {
    g.p += first;
    return;
  }
  const int64_t per_round = int64_t(MAX_SUBSTREAMS) * SUB_WORDS;
  const int64_t e = (rest - 1) % SUB_WORDS; // last word, in its substream
  const int64_t final_lo = e / MT_N * MT_N;
  int64_t done = 0;
  for (int r = 0; done < rest; ++r) {
    const int64_t words = std::min(rest - done, per_round);
    const int subs = int((words + SUB_WORDS - 1) / SUB_WORDS);
    const bool last = done + words == rest;
    uint64_t *base = d.base[r & 1];
    if (subs > 1) {
      ensure_polys(d, subs - 1);
      rng_raw_kernel<<<1, 64, 0, s>>>(base, d.raw);
      NT_LAUNCH_CHECK();
      const unsigned groups = unsigned((subs - 1 + JUMP_WAVES - 1) / JUMP_WAVES);
      rng_jump_kernel<<<dim3(JUMP_CHUNKS, groups), 64 * JUMP_WAVES, 0, s>>>(
          d.raw, d.polys, d.partial, subs - 1);
      NT_LAUNCH_CHECK();
    }
    rng_gen_kernel<T><<<unsigned(subs), GEN_THREADS, 0, s>>>(
        base, d.partial, words, out + first + done, lo, span,
        last ? d.words : nullptr, final_lo,
        last ? nullptr : d.base[(r + 1) & 1]);
    NT_LAUNCH_CHECK();
    done += words;
  }
  g.p = int(e - final_lo) + 1;
}

} // namespace
} // namespace nt

using namespace nt;

extern "C" {

int nt_manual_seed(uint64_t seed) {
  try {
    Generator &g = generator();
    std::lock_guard<std::mutex> lock(g.mu);
    mt_seed(g.x, seed);
    g.p = MT_N;
    g.seeded = true;
    g.words_on_device = false; // queued device draws no longer matter
  } catch (...) {
    return NT_ERR_RUNTIME;
  }
  return NT_OK;
}

int nt_host_uniform(void *host_out, int32_t dtype, int64_t n, double low,
                    double high) {
  // Needs no device unless earlier draws ran there.
  try {
    if (dtype != NT_FLOAT32 && dtype != NT_FLOAT64) {
      set_last_error("nt_host_uniform: float dtype required");
      return NT_ERR_VALUE;
    }
    if (n < 0 || (n > 0 && host_out == nullptr)) {
      set_last_error("nt_host_uniform: bad output buffer");
      return NT_ERR_VALUE;
    }
    Generator &g = generator();
    std::lock_guard<std::mutex> lock(g.mu);
    ensure_seeded(g);
    words_to_host(g);
    if (dtype == NT_FLOAT32) {
      const float lo = float(low), span = float(high) - float(low);
      host_draws(g, static_cast<float *>(host_out), n, lo, span);
    } else {
      host_draws(g, static_cast<double *>(host_out), n, low, high - low);
    }
  } catch (const Error &e) {
    set_last_error(e.msg);
    return e.code;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return NT_ERR_RUNTIME;
  }
  return NT_OK;
}

int nt_rng_prepare(void) {
  // Host only: the generator's polynomial, jump tables and their check.
  try {
    Generator &g = generator();
    std::lock_guard<std::mutex> lock(g.mu);
    host_polys(MAX_SUBSTREAMS - 1);
  } catch (const Error &e) {
    set_last_error(e.msg);
    return e.code;
  } catch (const std::exception &e) {
    set_last_error(e.what());
    return NT_ERR_RUNTIME;
  }
  return NT_OK;
}

int nt_device_uniform(void *out, int32_t dtype, int64_t n, double low,
                      double high) {
  return guard([&] {
    if (dtype != NT_FLOAT32 && dtype != NT_FLOAT64)
      fail(NT_ERR_VALUE, "nt_device_uniform: float dtype required");
    if (n < 0 || (n > 0 && out == nullptr))
      fail(NT_ERR_VALUE, "nt_device_uniform: bad output buffer");
    if (n == 0)
      return;
    Generator &g = generator();
    std::lock_guard<std::mutex> lock(g.mu);
    ensure_seeded(g);
    if (dtype == NT_FLOAT32) {
      const float lo = float(low), span = float(high) - float(low);
      device_draws(g, static_cast<float *>(out), n, lo, span);
    } else {
      device_draws(g, static_cast<double *>(out), n, low, high - low);
    }
  });
}

} // extern "C"
