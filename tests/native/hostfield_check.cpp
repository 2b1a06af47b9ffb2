// Driver for tests/test_hostfield.py: reads a command and QM31 data (decimal words) on stdin,
// runs the host-side AVX2 routines of stwo-ml_amd/csrc/hostfield.h, prints the results.
#include <cstdio>
#include <string>
#include <vector>

#include "../../stwo-ml_amd/csrc/hostfield.h"

static std::vector<uint32_t> read_q(size_t n) {
  std::vector<uint32_t> v(4 * n);
  for (auto& x : v)
    if (scanf("%u", &x) != 1) x = 0;
  return v;
}
static void print_q(const uint32_t* q, size_t n) {
  for (size_t i = 0; i < 4 * n; i++) printf("%u%c", q[i], i + 1 == 4 * n ? '\n' : ' ');
}

int main() {
  char op[32];
  size_t n;
  while (scanf("%31s %zu", op, &n) == 2) {
    const std::string s(op);
    if (s == "mul") {  // n pairs -> n products (4 at a time, then the scalar rest)
      std::vector<uint32_t> x = read_q(n), y = read_q(n), out(4 * n);
      size_t i = 0;
      for (; i + 4 <= n; i += 4)
        hostfield::q4_st(out.data() + 4 * i,
                         hostfield::q4_mul(hostfield::q4_ld(x.data() + 4 * i), hostfield::q4_ld(y.data() + 4 * i)));
      for (; i < n; i++)
        hostfield::q_st(out.data() + 4 * i, hostfield::q_mul(hostfield::q_ld(x.data() + 4 * i),
                                                             hostfield::q_ld(y.data() + 4 * i)));
      print_q(out.data(), n);
    } else if (s == "addsub") {  // sum and difference, 4 at a time
      std::vector<uint32_t> x = read_q(n), y = read_q(n), a(4 * n), d(4 * n);
      for (size_t i = 0; i + 4 <= n; i += 4) {
        const auto X = hostfield::q4_ld(x.data() + 4 * i), Y = hostfield::q4_ld(y.data() + 4 * i);
        hostfield::q4_st(a.data() + 4 * i, hostfield::q4_add(X, Y));
        hostfield::q4_st(d.data() + 4 * i, hostfield::q4_sub(X, Y));
      }
      print_q(a.data(), n);
      print_q(d.data(), n);
    } else if (s == "product") {  // A, B of 2n values -> 3 sums
      std::vector<uint32_t> a = read_q(2 * n), b = read_q(2 * n);
      uint32_t out[3][4];
      hostfield::product_round(a.data(), b.data(), n, out);
      print_q(&out[0][0], 3);
    } else if (s == "eq3") {
      std::vector<uint32_t> e = read_q(2 * n), w = read_q(2 * n), d = read_q(2 * n);
      uint32_t out[4][4];
      hostfield::eq3_round(e.data(), w.data(), d.data(), n, out);
      print_q(&out[0][0], 4);
    } else if (s == "halves") {
      std::vector<uint32_t> v = read_q(2 * n);
      uint32_t out[2][4];
      hostfield::halves_sum(v.data(), n, out);
      print_q(&out[0][0], 2);
    } else if (s == "fold") {  // V of 2n values and r -> n folded values
      std::vector<uint32_t> v = read_q(2 * n), r = read_q(1);
      hostfield::fold(v.data(), n, r.data());
      print_q(v.data(), n);
    }
    fflush(stdout);
  }
  return 0;
}
