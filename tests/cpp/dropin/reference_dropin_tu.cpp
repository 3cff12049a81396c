// Compiled (not run) against the SUF tree by tests/test_dropin_compile.py:
// the reference's launcher header and this repository's replacement declare
// the same extern "C" prototypes (a differing one fails to compile), every
// launcher is called with the reference's argument types, and the factory
// replacement hands out the MI355X backend for SUF_PFSS_BACKEND=hip through
// SUF's own interfaces.
#include "runtime/cuda_primitives.hpp"
#include "suf_hip/cuda_primitives.hpp"
#include "suf_hip/backend_factory.hpp"

#include <memory>
#include <vector>

void call_every_launcher(void* stream) {
  std::vector<uint64_t> v(64);
  uint64_t* p = v.data();
  const uint64_t* c = v.data();
  int lens[4] = {1, 2, 3, 4};
  launch_beaver_mul_kernel(0, c, c, c, c, c, c, c, p, 8, stream);
  launch_beaver_mul_aos_kernel(1, static_cast<const void*>(c), c, c, p, 8, stream);
  launch_trunc_shift_kernel(c, p, 12, 8, stream);
  launch_trunc_postproc_kernel(0, 1, 12, 0u, 0u, c, c, 1, 0, c, 3, 0, 1, 2, p, 8, stream);
  launch_horner_cubic_kernel(c, c, c, c, c, p, 8, stream);
  launch_add_rout_aos_kernel(p, 2, 4, c, 4, stream);
  launch_row_broadcast_mul_kernel(0, c, c, c, c, c, 4, 4, lens, p, 16, stream);
  launch_row_sum_kernel(c, 4, 4, lens, p, stream);
  launch_row_sum_ragged_kernel(c, lens, 3, p, stream);
  launch_beaver_matmul2d_kernel(0, c, c, c, c, c, 2, 2, 2, 0, 1, int64_t(5), 3, p, stream);
  launch_beaver_matmul2d_batched_kernel(1, c, c, c, c, c, 2, 2, 2, 2, 1, 0, 0, 0, p, stream);
  launch_row_mean_kernel(c, 4, 4, nullptr, p, stream);
  launch_row_variance_kernel(c, c, 4, 4, lens, p, stream);
  launch_unpack_eff_bits_kernel(c, 13, p, 8, stream);
  launch_pack_eff_bits_kernel(c, 13, p, 8, stream);
  launch_open_add_to_signed_kernel(c, c, p, 8, 50, (uint64_t(1) << 50) - 1, stream);
  launch_unpack_add_to_signed_kernel(c, c, 13, p, 8, 50, (uint64_t(1) << 50) - 1, stream);
  launch_unpack_add_mod_kernel(c, c, 13, p, 8, 50, (uint64_t(1) << 50) - 1, stream);
}

std::unique_ptr<proto::PfssBackendBatch> make_hip_backend_like_suf() {
  proto::PfssBackendOptions opts;
  opts.kind = proto::parse_backend_kind("hip");
  std::unique_ptr<proto::PfssBackendBatch> b = proto::make_pfss_backend(opts);
  // SUF discovers the device paths and the LUT extension by dynamic_cast.
  auto* staged = dynamic_cast<proto::PfssGpuStagedEval*>(b.get());
  auto* lut = dynamic_cast<proto::PfssIntervalLutExt*>(b.get());
  auto* packed = dynamic_cast<proto::PackedLtBackend*>(b.get());
  (void)staged;
  (void)lut;
  (void)packed;
  return b;
}
