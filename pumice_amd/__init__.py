"""MI355X (gfx950) token sampler: logits -> token with repetition / presence
penalty, temperature, top-k, top-p, min-p and a seeded draw, behind the C ABI
of include/pumice_sampler.h.  `pumice_amd.sampler` is the ctypes mirror of that
ABI; `pumice_amd.hip` is HIP runtime plumbing for tests and benchmarks."""
