// Dumps the dealer-side gate tables as the reference builds them, for the
// fixture tests/golden/tables_f12.json (tests/golden/make_tables.py runs it).
// Built by oracle/build_ref.sh from the reference's own headers, in place:
//   GeLU   gates::make_gelu_spline_spec      (include/gates/tables/gelu_spline_table.hpp:57-92)
//   nExp   gates::make_nexp_piecewise_spec   (include/gates/tables/nexp_piecewise_table.hpp:40-81)
//   Recip  gates::make_recip_affine_init_spec (include/gates/tables/recip_piecewise_affine_init.hpp)
//   each through suf::build_silu_suf_from_piecewise (include/suf/suf_silu_builders.hpp:79-186);
//   Rsqrt  gates::make_rsqrt_affine_init_spec (include/gates/tables/rsqrt_piecewise_affine_init.hpp)
//   as its raw intervals (start, end, offset, coefficients).
// Output: one JSON object on stdout.  TEST INFRASTRUCTURE ONLY.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "gates/tables/gelu_spline_table.hpp"
#include "gates/tables/nexp_piecewise_table.hpp"
#include "gates/tables/recip_piecewise_affine_init.hpp"
#include "gates/tables/rsqrt_piecewise_affine_init.hpp"
#include "suf/suf_silu_builders.hpp"

static void dump_suf(const char* name, const suf::SUF<uint64_t>& F, bool comma) {
  std::printf("\"%s\": {\"alpha\": [", name);
  for (size_t i = 0; i < F.alpha.size(); ++i)
    std::printf("%s\"%llu\"", i ? ", " : "", static_cast<unsigned long long>(F.alpha[i]));
  std::printf("], \"coeffs\": [");
  for (size_t p = 0; p < F.pieces.size(); ++p) {
    std::printf("%s[", p ? ", " : "");
    for (size_t w = 0; w < F.pieces[p].polys.size(); ++w) {
      const auto& c = F.pieces[p].polys[w].coeffs;
      std::printf("%s\"%lld\"", w ? ", " : "",
                  static_cast<long long>(static_cast<int64_t>(c.empty() ? 0 : c[0])));
    }
    std::printf("]");
  }
  std::printf("]}%s\n", comma ? "," : "");
}

static void dump_spec(const char* name, const gates::PiecewisePolySpec& s, bool comma) {
  std::printf("\"%s\": {\"frac_bits_in\": %d, \"intervals\": [", name, s.frac_bits_in);
  for (size_t i = 0; i < s.intervals.size(); ++i) {
    const auto& iv = s.intervals[i];
    std::printf("%s{\"start\": \"%llu\", \"end\": \"%llu\", \"offset\": \"%lld\", \"coeffs\": [",
                i ? ", " : "", static_cast<unsigned long long>(iv.start),
                static_cast<unsigned long long>(iv.end), static_cast<long long>(iv.pack.offset));
    for (size_t j = 0; j < iv.pack.coeffs.size(); ++j)
      std::printf("%s\"%lld\"", j ? ", " : "", static_cast<long long>(iv.pack.coeffs[j]));
    std::printf("]}");
  }
  std::printf("]}%s\n", comma ? "," : "");
}

int main() {
  const int f = 12;
  std::printf("{\"frac_bits\": %d,\n", f);
  dump_suf("gelu", suf::build_silu_suf_from_piecewise(gates::make_gelu_spline_spec(f, 16)), true);
  dump_suf("nexp", suf::build_silu_suf_from_piecewise(gates::make_nexp_piecewise_spec(f, 16)), true);
  dump_suf("recip", suf::build_silu_suf_from_piecewise(gates::make_recip_affine_init_spec(f, 1024.0)),
           true);
  dump_spec("rsqrt_spec", gates::make_rsqrt_affine_init_spec(f, 1.0 / 1024.0, 16.0), false);
  std::printf("}\n");
  return 0;
}
