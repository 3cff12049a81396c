// Evaluates two SUF gates with the reference's own eval_suf_ref
// (include/suf/ref_eval.hpp:58-78) at fixed points, for the fixture
// tests/golden/suf_ref_eval.json (tests/golden/make_suf_ref.py runs it).
// The gates are the two specs of tests/golden/make_suf_ref.py (MIXED and
// DRELU), written here with the reference's SUF types.  Built by
// oracle/build_ref.sh.  TEST INFRASTRUCTURE ONLY.
#include <cstdint>
#include <cstdio>
#include <memory>
#include <stdexcept>  // ref_eval.hpp throws std::runtime_error without including it
#include <random>
#include <vector>

#include "suf/ref_eval.hpp"

using suf::BoolExpr;

static BoolExpr C(bool v) { return BoolExpr{suf::BConst{v}}; }
static BoolExpr V(int i) { return BoolExpr{suf::BVar{i}}; }
static BoolExpr Not(BoolExpr a) { return BoolExpr{suf::BNot{std::make_unique<BoolExpr>(std::move(a))}}; }
static BoolExpr Xor(BoolExpr a, BoolExpr b) {
  return BoolExpr{suf::BXor{std::make_unique<BoolExpr>(std::move(a)), std::make_unique<BoolExpr>(std::move(b))}};
}
static BoolExpr And(BoolExpr a, BoolExpr b) {
  return BoolExpr{suf::BAnd{std::make_unique<BoolExpr>(std::move(a)), std::make_unique<BoolExpr>(std::move(b))}};
}
static BoolExpr Or(BoolExpr a, BoolExpr b) {
  return BoolExpr{suf::BOr{std::make_unique<BoolExpr>(std::move(a)), std::make_unique<BoolExpr>(std::move(b))}};
}

static suf::SufPiece<uint64_t> piece(uint64_t w, std::vector<BoolExpr> bools) {
  suf::SufPiece<uint64_t> p;
  suf::Poly<uint64_t> poly;
  poly.coeffs = {w};
  p.polys.push_back(poly);
  p.bool_outs = std::move(bools);
  return p;
}

static std::vector<BoolExpr> two(BoolExpr a, BoolExpr b) {
  std::vector<BoolExpr> v;
  v.push_back(std::move(a));
  v.push_back(std::move(b));
  return v;
}

static std::vector<BoolExpr> one(BoolExpr a) {
  std::vector<BoolExpr> v;
  v.push_back(std::move(a));
  return v;
}

static void dump(const char* name, const suf::SUF<uint64_t>& F, const std::vector<uint64_t>& xs,
                 bool comma) {
  std::printf("\"%s\": [", name);
  for (size_t i = 0; i < xs.size(); ++i) {
    auto r = suf::eval_suf_ref(F, xs[i]);
    std::printf("%s{\"x\": \"%llu\", \"piece\": %d, \"arith\": \"%llu\", \"bools\": [", i ? ", " : "",
                static_cast<unsigned long long>(xs[i]), r.piece_idx,
                static_cast<unsigned long long>(r.arith[0]));
    for (size_t j = 0; j < r.bools.size(); ++j) std::printf("%s%d", j ? ", " : "", r.bools[j] ? 1 : 0);
    std::printf("]}");
  }
  std::printf("]%s\n", comma ? "," : "");
}

int main() {
  const uint64_t T62 = uint64_t(1) << 62, T63 = uint64_t(1) << 63;
  suf::SUF<uint64_t> A;
  A.n_bits = 64;
  A.r_out = 1;
  A.l_out = 2;
  A.degree = 0;
  A.alpha = {0, T62, T63, T63 + T62, ~uint64_t(0)};
  A.primitive_preds = {suf::Pred_X_lt_const{1000}, suf::Pred_X_mod2f_lt{12, 2048},
                       suf::Pred_MSB_x{}, suf::Pred_MSB_x_plus{5000}};
  A.pieces.push_back(piece(7, two(And(V(0), Not(V(1))), Or(V(2), V(3)))));
  A.pieces.push_back(piece(11, two(Xor(V(1), V(3)), C(true))));
  A.pieces.push_back(piece(13, two(Not(V(0)), And(Or(V(1), V(2)), V(3)))));
  A.pieces.push_back(piece(17, two(C(false), V(2))));
  suf::SUF<uint64_t> D;  // the ReLU gate's sign output (include/gates/relu_gate.hpp:9-44)
  D.n_bits = 64;
  D.r_out = 1;
  D.l_out = 1;
  D.degree = 0;
  D.alpha = {0, T63, ~uint64_t(0)};
  D.pieces.push_back(piece(1, one(C(true))));
  D.pieces.push_back(piece(0, one(C(false))));
  std::vector<uint64_t> xs;
  for (uint64_t b : {uint64_t(0), uint64_t(1000), uint64_t(2048), uint64_t(4096), T62, T63, T63 + T62,
                     T63 - 5000, ~uint64_t(0)}) {
    xs.push_back(b - 1);
    xs.push_back(b);
    xs.push_back(b + 1);
  }
  std::mt19937_64 g(77);
  for (int i = 0; i < 200; ++i) xs.push_back(g());
  for (int i = 0; i < 100; ++i) xs.push_back(g() % 8192 - 4096);
  std::printf("{\n");
  dump("mixed", A, xs, true);
  dump("drelu", D, xs, false);
  std::printf("}\n");
  return 0;
}
