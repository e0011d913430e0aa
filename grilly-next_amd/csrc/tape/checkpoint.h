// checkpoint.h — the GRLY v3 hypernetwork checkpoint (bindings.cpp:2965-3039) and an
// optional optimizer-state section after it.
//
// File layout (little-endian):
//   u32 header[6] = {0x47524C59 "GRLY", d_model, vsa_dim, K, num_params = 10, router_hidden}
//   num_params x { u32 count; f32 data[count] }   in the order W_proj, b_proj, W1, b1, W2, b2,
//                                                 W_r1, b_r1, W_r2, b_r2
// Optimizer section (this build's addition; the reference saves no optimizer state and its
// loader stops after num_params tensors, so it still reads such a file):
//   u32 magic 0x54504F47 "GOPT", u32 version = 1, u32 kind (0 surprise momentum, 1 AdamW),
//   u32 n_states (tensors per parameter), u64 step, u32 n_hyper, f32 hyper[n_hyper],
//   num_params x n_states x { u32 count; f32 data[count] }   (parameter-major)
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace grilly {
namespace ckpt {

constexpr uint32_t kGrlyMagic = 0x47524C59u;  // "GRLY"
constexpr uint32_t kOptMagic = 0x54504F47u;   // "GOPT"
constexpr uint32_t kOptVersion = 1;
constexpr uint32_t kHyperParams = 10;

struct HyperDims {
    uint32_t d_model = 0, vsa_dim = 0, K = 0, router_hidden = 32;
};

// Element counts of the ten tensors (bindings.cpp:2973-2984); throws std::invalid_argument
// when one does not fit the format's 32-bit count.
std::vector<uint64_t> hyper_sizes(const HyperDims& d);

struct OptHeader {
    uint32_t kind = 0;
    uint32_t n_states = 0;
    uint64_t step = 0;
    std::vector<float> hyper;
};

// Host layer: fp32 host arrays, one per tensor (weights: 10; states: 10 x n_states,
// parameter-major).  write_* throws std::runtime_error on I/O failure; read_* checks the
// magic ("Invalid checkpoint magic"), the dimensions ("Model dimension mismatch"), the
// parameter count and every tensor's count against the model, and truncation — the
// reference reads the stored count into a buffer sized by the model, unchecked.
void write_hyper(const std::string& path, const HyperDims& d, const std::vector<const float*>& w,
                 const OptHeader* opt, const std::vector<const float*>& states);
// Reads the weights; when `opt` is given, also the optimizer section (an error if absent).
// `states` must then hold opt_expected_states pointers, filled parameter-major.
void read_hyper(const std::string& path, const HyperDims& d, const std::vector<float*>& w,
                OptHeader* opt, const std::vector<float*>& states, uint32_t opt_expected_states);
// Header only: dims, and whether an optimizer section follows (kind, n_states, step, hyper).
bool probe_hyper(const std::string& path, HyperDims* d, OptHeader* opt);

// Device layer: tensors in device memory, fp32 (dtype 0) or bf16 (dtype 4).  Waits for the
// device to be idle, stages through host memory; bf16 widens exactly on save and rounds to
// nearest-even on load.
struct DevTensor {
    uint64_t ptr;
    uint64_t numel;
    int dtype;
};
void save_hyper_device(const std::string& path, const HyperDims& d, const std::vector<DevTensor>& w,
                       const OptHeader* opt, const std::vector<DevTensor>& states);
void load_hyper_device(const std::string& path, const HyperDims& d, const std::vector<DevTensor>& w,
                       OptHeader* opt, const std::vector<DevTensor>& states);

}  // namespace ckpt
}  // namespace grilly
