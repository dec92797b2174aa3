// Checker only (tests/ load it; nothing else does): the reference's own generator --
// RandomState, splitmix64, the 53-bit open uniform, the Marsaglia polar pair with its spare,
// and the contiguous normal/uniform fills of cpp/mtorch/python/module.cpp:47-183 -- compiled
// from the reference tree where it lies (this file includes it; nothing is copied), behind a C
// ABI, so that tests/test_oracle_rng.py can pin the oracle's restatement (oracle.c orc_rng_*)
// bit for bit.  `make -C oracle ref` builds it into oracle/_ref/ when /root/reference is
// present; the version script exports only these entry points and --gc-sections discards
// every part of module.cpp they do not reach (the Python bindings and their calls into
// tensor.cpp), so nothing else of the reference is linked.
#include "mtorch/python/module.cpp"

namespace {
RandomState& state_of(void* p) { return *static_cast<RandomState*>(p); }
}  // namespace

extern "C" {
void* ref_rng_new(uint64_t seed) {
  auto* r = new RandomState();
  seed_random_state(*r, seed);
  return r;
}
void ref_rng_free(void* p) { delete static_cast<RandomState*>(p); }
uint64_t ref_rng_next_u64(void* p) { return next_random_u64(state_of(p)); }
double ref_rng_next_uniform(void* p) { return next_uniform_open(state_of(p)); }
double ref_rng_next_normal(void* p) { return next_standard_normal(state_of(p)); }
void ref_rng_fill_normal_f32(void* p, float* out, int64_t n, double mean, double std) {
  fill_random_normal_contiguous<float>(out, n, mean, std, state_of(p));
}
void ref_rng_fill_normal_f64(void* p, double* out, int64_t n, double mean, double std) {
  fill_random_normal_contiguous<double>(out, n, mean, std, state_of(p));
}
void ref_rng_fill_uniform_f32(void* p, float* out, int64_t n, double from, double to) {
  fill_random_uniform_contiguous<float>(out, n, from, to, state_of(p));
}
}
