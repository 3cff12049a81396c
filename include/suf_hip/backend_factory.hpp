// Replacement for SUF's include/proto/backend_factory.hpp (reference lines
// 1-89) with a `hip` kind: SUF_PFSS_BACKEND=hip (or PfssBackendKind::Hip)
// makes suf_hip::HipPfssBackend, the MI355X backend.  Every other kind keeps
// the reference factory's behaviour (unset: Grotto with libdpf, else
// SigmaFast; grotto likewise; the CUDA backend under SUF_HAVE_CUDA, else the
// clear backend; cpu -> ClearBackend).  The names, enumerators, option fields and
// functions are the reference's so that callers (LayerContext::
// select_backend_from_env, include/nn/layer_context.hpp:89-97, the tests and
// benches) compile unchanged.  Used inside the SUF tree only: it needs SUF's
// proto headers, so it requires SUF_HIP_USE_REFERENCE_PROTO.
#pragma once

#ifndef SUF_HIP_USE_REFERENCE_PROTO
#error "suf_hip/backend_factory.hpp replaces SUF's proto/backend_factory.hpp: build inside the SUF tree with SUF_HIP_USE_REFERENCE_PROTO"
#endif

#include <cctype>
#include <cstdlib>
#include <memory>
#include <stdexcept>
#include <string>

#include "proto/backend_clear.hpp"
#include "proto/backend_gpu.hpp"
#include "proto/sigma_fast_backend_ext.hpp"
#ifdef SUF_HAVE_LIBDPF
#include "proto/grotto_backend.hpp"
#endif
#include "suf_hip/hip_pfss_backend.hpp"

namespace proto {

enum class PfssBackendKind { Auto, Cpu, Gpu, SigmaFast, Grotto, Hip };

struct PfssBackendOptions {
  PfssBackendKind kind = PfssBackendKind::Auto;
  bool allow_gpu_stub = true;  // no CUDA build: the Gpu kind falls back to the CPU backend
};

inline PfssBackendKind parse_backend_kind(const char* env) {
  if (env == nullptr) return PfssBackendKind::Auto;
  std::string v;
  for (const char* p = env; *p; ++p) v.push_back(static_cast<char>(std::tolower(static_cast<unsigned char>(*p))));
  if (v == "hip") return PfssBackendKind::Hip;
  if (v == "gpu") return PfssBackendKind::Gpu;
  if (v == "cpu") return PfssBackendKind::Cpu;
  if (v == "sigma" || v == "sigmafast" || v == "sigma_fast") return PfssBackendKind::SigmaFast;
  if (v == "grotto") return PfssBackendKind::Grotto;
  return PfssBackendKind::Auto;
}

inline std::unique_ptr<PfssBackendBatch> make_pfss_backend(const PfssBackendOptions& opts = {}) {
  PfssBackendKind kind = opts.kind;
  if (kind == PfssBackendKind::Auto) kind = parse_backend_kind(std::getenv("SUF_PFSS_BACKEND"));
  switch (kind) {
    case PfssBackendKind::Hip:
      // One instance per party, like every other kind; a GPU that is absent
      // or not gfx950 throws here instead of falling back.
      return std::make_unique<suf_hip::HipPfssBackend>();
    case PfssBackendKind::SigmaFast:
      return std::make_unique<SigmaFastBackend>();
    case PfssBackendKind::Auto:
    case PfssBackendKind::Grotto:
#ifdef SUF_HAVE_LIBDPF
      return std::make_unique<GrottoBackend>();
#else
      return std::make_unique<SigmaFastBackend>();
#endif
    case PfssBackendKind::Gpu:
#ifdef SUF_HAVE_CUDA
    {
      auto gpu = make_real_gpu_backend();
      if (!gpu) throw std::runtime_error("GPU backend unavailable");
      return gpu;
    }
#else
      if (!opts.allow_gpu_stub)
        throw std::runtime_error("GPU backend requested but SUF_HAVE_CUDA is not enabled");
      return ClearBackend::make();
#endif
    case PfssBackendKind::Cpu:
    default:
      return ClearBackend::make();
  }
}

inline std::unique_ptr<PfssBackendBatch> make_pfss_backend_from_env(
    const PfssBackendOptions& defaults = {}) {
  PfssBackendOptions opts = defaults;
  if (const char* env = std::getenv("SUF_PFSS_BACKEND")) opts.kind = parse_backend_kind(env);
  return make_pfss_backend(opts);
}

}  // namespace proto
