// Polynomial arithmetic over GF(2), host only: what jumping a linear
// generator ahead needs (a minimal polynomial from its output bits, and
// x^e modulo that polynomial).  A polynomial is a word vector: bit i of word
// i / 64 is the coefficient of x^i.
#pragma once

#include <cstdint>
#include <vector>

namespace nt::gf2 {

using Poly = std::vector<uint64_t>;

// Minimal polynomial of the bit sequence s (monic, returned with its
// degree), by Berlekamp-Massey (Massey 1969).  s needs at least twice the
// degree bits.
Poly minimal_polynomial(const std::vector<uint8_t> &s, int *degree);

// Arithmetic modulo a fixed polynomial P of degree d: Barrett reduction
// with mu = floor(x^(2d) / P), which over GF(2) gives the exact quotient of
// any product of two residues.  Products use PCLMULQDQ when the CPU has it.
class Modulus {
public:
  Modulus(const Poly &p, int degree);
  int degree() const { return d_; }
  int words() const { return nw_; } // words of a residue (degree < d)
  Poly mul(const Poly &a, const Poly &b) const;
  Poly xpow(uint64_t e) const; // x^e mod P

private:
  Poly p_, mu_;
  int d_, nw_;
};

} // namespace nt::gf2
