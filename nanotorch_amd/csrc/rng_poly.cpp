// GF(2)[x] arithmetic for the generator jump tables (host only).
#include "rng_poly.h"

#include <immintrin.h>

#include <algorithm>
#include <stdexcept>

namespace nt::gf2 {
namespace {

bool get_bit(const Poly &a, int64_t i) {
  return size_t(i >> 6) < a.size() && ((a[size_t(i >> 6)] >> (i & 63)) & 1);
}

// 64 bits of a starting at bit offset off (bits past the end read as 0).
uint64_t bits_at(const Poly &a, int64_t off) {
  const size_t w = size_t(off >> 6);
  const int s = int(off & 63);
  const uint64_t lo = w < a.size() ? a[w] : 0;
  if (s == 0)
    return lo;
  const uint64_t hi = w + 1 < a.size() ? a[w + 1] : 0;
  return (lo >> s) | (hi << (64 - s));
}

// acc ^= src * x^shift, over the first nsrc words of src.
void xor_shifted(Poly &acc, const Poly &src, size_t nsrc, int64_t shift) {
  const size_t ws = size_t(shift >> 6);
  const int s = int(shift & 63);
  for (size_t k = 0; k < nsrc && k < src.size(); ++k) {
    const uint64_t v = src[k];
    if (!v)
      continue;
    if (ws + k < acc.size())
      acc[ws + k] ^= v << s;
    if (s && ws + k + 1 < acc.size())
      acc[ws + k + 1] ^= v >> (64 - s);
  }
}

// Carry-less 64 x 64 -> 128 product, portable form.
inline void clmul64_soft(uint64_t a, uint64_t b, uint64_t &lo, uint64_t &hi) {
  lo = hi = 0;
  for (int i = 0; i < 64; ++i)
    if ((b >> i) & 1) {
      lo ^= a << i;
      if (i)
        hi ^= a >> (64 - i);
    }
}

void mul_soft(const uint64_t *a, size_t na, const uint64_t *b, size_t nb,
              uint64_t *r, size_t nr) {
  std::fill(r, r + nr, 0);
  for (size_t i = 0; i < na; ++i) {
    if (!a[i])
      continue;
    for (size_t j = 0; j < nb && i + j < nr; ++j) {
      uint64_t lo, hi;
      clmul64_soft(a[i], b[j], lo, hi);
      r[i + j] ^= lo;
      if (i + j + 1 < nr)
        r[i + j + 1] ^= hi;
    }
  }
}

__attribute__((target("pclmul,sse2"))) void
mul_pclmul(const uint64_t *a, size_t na, const uint64_t *b, size_t nb,
           uint64_t *r, size_t nr) {
  std::fill(r, r + nr, 0);
  for (size_t i = 0; i < na; ++i) {
    if (!a[i])
      continue;
    const __m128i ai = _mm_cvtsi64_si128(int64_t(a[i]));
    for (size_t j = 0; j < nb && i + j < nr; ++j) {
      const __m128i p =
          _mm_clmulepi64_si128(ai, _mm_cvtsi64_si128(int64_t(b[j])), 0x00);
      r[i + j] ^= uint64_t(_mm_cvtsi128_si64(p));
      if (i + j + 1 < nr)
        r[i + j + 1] ^= uint64_t(_mm_cvtsi128_si64(_mm_unpackhi_epi64(p, p)));
    }
  }
}

// r (nr words: the product truncated to nr words) = a * b.
void mul_words(const uint64_t *a, size_t na, const uint64_t *b, size_t nb,
               uint64_t *r, size_t nr) {
  static const bool has_pclmul = __builtin_cpu_supports("pclmul");
  if (has_pclmul)
    mul_pclmul(a, na, b, nb, r, nr);
  else
    mul_soft(a, na, b, nb, r, nr);
}

// The bits [from, from + nbits) of a, as a polynomial.
Poly extract(const Poly &a, int64_t from, int64_t nbits, size_t nwords) {
  Poly r(nwords, 0);
  for (size_t k = 0; k < nwords && int64_t(k) * 64 < nbits; ++k)
    r[k] = bits_at(a, from + int64_t(k) * 64);
  const int64_t tail = nbits - int64_t(nwords - 1) * 64;
  if (tail > 0 && tail < 64)
    r[nwords - 1] &= (uint64_t(1) << tail) - 1;
  return r;
}

} // namespace

Poly minimal_polynomial(const std::vector<uint8_t> &s, int *degree) {
  // Berlekamp-Massey: C(x) = 1 + c_1 x + ... + c_L x^L is the shortest
  // connection polynomial with s_k = sum_{i=1..L} c_i s_{k-i}.
  const int64_t n = int64_t(s.size());
  const size_t cw = size_t(n / 64 + 2);
  // rev bit j = s[n - 1 - j]: the terms s_k, s_{k-1}, ... of the
  // discrepancy sum are then consecutive bits from offset n - 1 - k.
  Poly rev(size_t((2 * n) / 64 + 4), 0);
  for (int64_t j = 0; j < n; ++j)
    if (s[size_t(n - 1 - j)])
      rev[size_t(j >> 6)] |= uint64_t(1) << (j & 63);
  Poly C(cw, 0), B(cw, 0), T;
  C[0] = B[0] = 1;
  int64_t L = 0, m = 1;
  for (int64_t k = 0; k < n; ++k) {
    uint64_t acc = 0;
    const size_t nw = size_t(L / 64 + 1);
    for (size_t w = 0; w < nw; ++w) {
      uint64_t c = C[w];
      if (w + 1 == nw && (L & 63) != 63)
        c &= (uint64_t(2) << (L & 63)) - 1; // terms c_0 .. c_L only
      acc ^= c & bits_at(rev, n - 1 - k + int64_t(w) * 64);
    }
    if (!(__builtin_popcountll(acc) & 1)) {
      ++m;
      continue;
    }
    if (2 * L <= k) {
      T = C;
      xor_shifted(C, B, cw, m);
      L = k + 1 - L;
      B = T;
      m = 1;
    } else {
      xor_shifted(C, B, cw, m);
      ++m;
    }
  }
  // P(x) = x^L C(1/x): the coefficient of x^(L-i) is c_i.
  Poly P(size_t(L / 64 + 1), 0);
  for (int64_t i = 0; i <= L; ++i)
    if (get_bit(C, i))
      P[size_t((L - i) >> 6)] |= uint64_t(1) << ((L - i) & 63);
  *degree = int(L);
  return P;
}

Modulus::Modulus(const Poly &p, int degree)
    : p_(p), d_(degree), nw_(degree / 64 + 1) {
  if (degree < 1 || !get_bit(p, degree))
    throw std::runtime_error("gf2::Modulus: polynomial degree mismatch");
  p_.resize(size_t(nw_), 0);
  // mu = floor(x^(2d) / P) by long division.
  const int64_t top = 2 * int64_t(d_);
  Poly rem(size_t(top / 64 + 2), 0);
  rem[size_t(top >> 6)] |= uint64_t(1) << (top & 63);
  mu_.assign(size_t(nw_), 0);
  for (int64_t k = top; k >= d_; --k) {
    if (!get_bit(rem, k))
      continue;
    xor_shifted(rem, p_, size_t(nw_), k - d_);
    mu_[size_t((k - d_) >> 6)] |= uint64_t(1) << ((k - d_) & 63);
  }
}

Poly Modulus::mul(const Poly &a, const Poly &b) const {
  const size_t n = size_t(nw_);
  Poly prod(2 * n, 0);
  mul_words(a.data(), std::min(a.size(), n), b.data(), std::min(b.size(), n),
            prod.data(), 2 * n);
  // A = hi x^d + lo with deg hi <= d - 2; the quotient is
  // floor(hi * mu / x^d), and A - q P has degree < d.
  const Poly hi = extract(prod, d_, int64_t(d_), n);
  Poly hm(2 * n, 0);
  mul_words(hi.data(), n, mu_.data(), n, hm.data(), 2 * n);
  const Poly q = extract(hm, d_, int64_t(d_), n);
  Poly qp(n, 0);
  mul_words(q.data(), n, p_.data(), n, qp.data(), n);
  Poly r(n, 0);
  for (size_t k = 0; k < n; ++k)
    r[k] = prod[k] ^ qp[k];
  const int tail = d_ - int(n - 1) * 64;
  r[n - 1] &= tail >= 64 ? ~uint64_t(0) : (uint64_t(1) << tail) - 1;
  return r;
}

Poly Modulus::xpow(uint64_t e) const {
  Poly r(size_t(nw_), 0);
  r[0] = 1;
  for (int b = 63; b >= 0; --b) {
    r = mul(r, r);
    if ((e >> b) & 1) {
      // r *= x
      uint64_t carry = 0;
      for (auto &w : r) {
        const uint64_t next = w >> 63;
        w = (w << 1) | carry;
        carry = next;
      }
      if (get_bit(r, d_))
        for (size_t k = 0; k < r.size(); ++k)
          r[k] ^= p_[k];
    }
  }
  return r;
}

} // namespace nt::gf2
