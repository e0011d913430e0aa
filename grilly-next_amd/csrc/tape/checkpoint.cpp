// checkpoint.cpp — GRLY v3 hypernetwork checkpoint and optimizer section (see checkpoint.h).
#include "checkpoint.h"

#include <cstdio>
#include <cstring>
#include <stdexcept>

#include "device.h"

namespace grilly {
namespace ckpt {
namespace {

struct File {
    FILE* f = nullptr;
    std::string path;
    File(const std::string& p, const char* mode) : f(std::fopen(p.c_str(), mode)), path(p) {
        if (!f) throw std::runtime_error("Cannot open " + p);
    }
    ~File() {
        if (f) std::fclose(f);
    }
    void put(const void* p, size_t bytes) {
        if (bytes && std::fwrite(p, 1, bytes, f) != bytes)
            throw std::runtime_error("write failed: " + path);
    }
    void get(void* p, size_t bytes, const char* what) {
        if (bytes && std::fread(p, 1, bytes, f) != bytes)
            throw std::runtime_error(std::string("truncated checkpoint (") + what + "): " + path);
    }
    bool try_get(void* p, size_t bytes) { return std::fread(p, 1, bytes, f) == bytes; }
    void skip(uint64_t bytes, const char* what) {
        if (std::fseek(f, (long)bytes, SEEK_CUR) != 0)
            throw std::runtime_error(std::string("truncated checkpoint (") + what + "): " + path);
    }
    void close() {
        if (std::fflush(f) != 0 || std::ferror(f)) throw std::runtime_error("write failed: " + path);
        const int rc = std::fclose(f);
        f = nullptr;
        if (rc != 0) throw std::runtime_error("write failed: " + path);
    }
};

void put_tensor(File& f, const float* p, uint64_t n) {
    const uint32_t c = (uint32_t)n;
    f.put(&c, 4);
    f.put(p, n * sizeof(float));
}

void get_tensor(File& f, float* p, uint64_t n, const char* name) {
    uint32_t c = 0;
    f.get(&c, 4, name);
    if (c != n)
        throw std::runtime_error(std::string("checkpoint tensor ") + name + " holds " +
                                 std::to_string(c) + " values, the model needs " + std::to_string(n));
    f.get(p, n * sizeof(float), name);
}

const char* kNames[kHyperParams] = {"W_proj", "b_proj", "W1", "b1", "W2", "b2",
                                    "W_r1", "b_r1", "W_r2", "b_r2"};

void read_header(File& f, const HyperDims& d) {
    uint32_t h[6] = {};
    f.get(h, sizeof(h), "header");
    if (h[0] != kGrlyMagic) throw std::runtime_error("Invalid checkpoint magic");
    if (h[1] != d.d_model || h[2] != d.vsa_dim || h[3] != d.K)
        throw std::runtime_error("Model dimension mismatch");
    if (h[4] != kHyperParams)
        throw std::runtime_error("checkpoint holds " + std::to_string(h[4]) + " tensors, the model " +
                                 std::to_string(kHyperParams));
    if (h[5] != d.router_hidden)
        throw std::runtime_error("checkpoint router_hidden " + std::to_string(h[5]) +
                                 " != model " + std::to_string(d.router_hidden));
}

// bf16 <-> fp32 on the host: widening is exact; narrowing rounds to nearest-even, NaN stays
// a quiet NaN.
inline float bf2f_host(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
inline uint16_t f2bf_host(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

std::vector<float> download(const DevTensor& t) {
    std::vector<float> h(t.numel);
    if (t.numel == 0) return h;
    if (t.dtype == 0) {
        hip_check(hipMemcpy(h.data(), reinterpret_cast<const void*>(t.ptr), t.numel * 4,
                            hipMemcpyDeviceToHost), "checkpoint download");
    } else {
        std::vector<uint16_t> b(t.numel);
        hip_check(hipMemcpy(b.data(), reinterpret_cast<const void*>(t.ptr), t.numel * 2,
                            hipMemcpyDeviceToHost), "checkpoint download");
        for (uint64_t i = 0; i < t.numel; ++i) h[i] = bf2f_host(b[i]);
    }
    return h;
}

void upload(const DevTensor& t, const std::vector<float>& h) {
    if (t.numel == 0) return;
    if (t.dtype == 0) {
        hip_check(hipMemcpy(reinterpret_cast<void*>(t.ptr), h.data(), t.numel * 4, hipMemcpyHostToDevice),
                  "checkpoint upload");
    } else {
        std::vector<uint16_t> b(t.numel);
        for (uint64_t i = 0; i < t.numel; ++i) b[i] = f2bf_host(h[i]);
        hip_check(hipMemcpy(reinterpret_cast<void*>(t.ptr), b.data(), t.numel * 2, hipMemcpyHostToDevice),
                  "checkpoint upload");
    }
}

void check_dev(const std::vector<DevTensor>& ts, const std::vector<uint64_t>& sizes, size_t per,
               const char* what) {
    if (ts.size() != sizes.size() * per)
        throw std::invalid_argument(std::string(what) + ": expected " + std::to_string(sizes.size() * per) +
                                    " tensors, got " + std::to_string(ts.size()));
    for (size_t i = 0; i < ts.size(); ++i) {
        const uint64_t need = sizes[i / per];
        if (ts[i].numel != need)
            throw std::invalid_argument(std::string(what) + ": tensor " + kNames[i / per] + " has " +
                                        std::to_string(ts[i].numel) + " elements, the model needs " +
                                        std::to_string(need));
        if (ts[i].dtype != 0 && ts[i].dtype != 4)
            throw std::invalid_argument(std::string(what) + ": dtype must be f32 (0) or bf16 (4)");
        if (need && !ts[i].ptr) throw std::invalid_argument(std::string(what) + ": null tensor");
    }
}

}  // namespace

std::vector<uint64_t> hyper_sizes(const HyperDims& d) {
    const uint64_t dm = d.d_model, v = d.vsa_dim, K = d.K, rh = d.router_hidden, h = 2 * dm;
    std::vector<uint64_t> s = {dm * v, dm, h * dm, h, K * v * h, K * v, rh * dm, rh, K * rh, K};
    for (uint64_t x : s)
        if (x > 0xffffffffull)
            throw std::invalid_argument("hypernetwork tensor of " + std::to_string(x) +
                                        " values exceeds the checkpoint's 32-bit count");
    return s;
}

void write_hyper(const std::string& path, const HyperDims& d, const std::vector<const float*>& w,
                 const OptHeader* opt, const std::vector<const float*>& states) {
    const auto sizes = hyper_sizes(d);
    if (w.size() != kHyperParams) throw std::invalid_argument("write_hyper: 10 weight tensors expected");
    if (opt && states.size() != (size_t)kHyperParams * opt->n_states)
        throw std::invalid_argument("write_hyper: 10 x n_states state tensors expected");
    File f(path, "wb");
    const uint32_t header[6] = {kGrlyMagic, d.d_model, d.vsa_dim, d.K, kHyperParams, d.router_hidden};
    f.put(header, sizeof(header));
    for (uint32_t i = 0; i < kHyperParams; ++i) put_tensor(f, w[i], sizes[i]);
    if (opt) {
        const uint32_t h4[4] = {kOptMagic, kOptVersion, opt->kind, opt->n_states};
        f.put(h4, sizeof(h4));
        f.put(&opt->step, 8);
        const uint32_t nh = (uint32_t)opt->hyper.size();
        f.put(&nh, 4);
        f.put(opt->hyper.data(), nh * sizeof(float));
        for (size_t i = 0; i < states.size(); ++i) put_tensor(f, states[i], sizes[i / opt->n_states]);
    }
    f.close();
}

void read_hyper(const std::string& path, const HyperDims& d, const std::vector<float*>& w,
                OptHeader* opt, const std::vector<float*>& states, uint32_t opt_expected_states) {
    const auto sizes = hyper_sizes(d);
    if (w.size() != kHyperParams) throw std::invalid_argument("read_hyper: 10 weight tensors expected");
    File f(path, "rb");
    read_header(f, d);
    for (uint32_t i = 0; i < kHyperParams; ++i) get_tensor(f, w[i], sizes[i], kNames[i]);
    if (!opt) return;
    uint32_t h4[4] = {};
    if (!f.try_get(h4, sizeof(h4)) || h4[0] != kOptMagic)
        throw std::runtime_error("checkpoint has no optimizer section: " + path);
    if (h4[1] != kOptVersion)
        throw std::runtime_error("optimizer section version " + std::to_string(h4[1]) + " not supported");
    if (h4[3] != opt_expected_states)
        throw std::runtime_error("optimizer section holds " + std::to_string(h4[3]) +
                                 " state tensors per parameter, expected " +
                                 std::to_string(opt_expected_states));
    if (states.size() != (size_t)kHyperParams * h4[3])
        throw std::invalid_argument("read_hyper: 10 x n_states state tensors expected");
    opt->kind = h4[2];
    opt->n_states = h4[3];
    f.get(&opt->step, 8, "optimizer step");
    uint32_t nh = 0;
    f.get(&nh, 4, "optimizer hyper-parameters");
    if (nh > 64) throw std::runtime_error("optimizer section: implausible hyper-parameter count");
    opt->hyper.resize(nh);
    f.get(opt->hyper.data(), nh * sizeof(float), "optimizer hyper-parameters");
    for (size_t i = 0; i < states.size(); ++i) get_tensor(f, states[i], sizes[i / h4[3]], "optimizer state");
}

bool probe_hyper(const std::string& path, HyperDims* d, OptHeader* opt) {
    File f(path, "rb");
    uint32_t h[6] = {};
    f.get(h, sizeof(h), "header");
    if (h[0] != kGrlyMagic) throw std::runtime_error("Invalid checkpoint magic");
    d->d_model = h[1];
    d->vsa_dim = h[2];
    d->K = h[3];
    d->router_hidden = h[5];
    for (uint32_t i = 0; i < h[4]; ++i) {
        uint32_t c = 0;
        f.get(&c, 4, "tensor count");
        f.skip((uint64_t)c * 4, "tensor data");
    }
    uint32_t h4[4] = {};
    if (!f.try_get(h4, sizeof(h4)) || h4[0] != kOptMagic) return false;
    if (opt) {
        opt->kind = h4[2];
        opt->n_states = h4[3];
        f.get(&opt->step, 8, "optimizer step");
        uint32_t nh = 0;
        f.get(&nh, 4, "optimizer hyper-parameters");
        if (nh > 64) throw std::runtime_error("optimizer section: implausible hyper-parameter count");
        opt->hyper.resize(nh);
        f.get(opt->hyper.data(), nh * sizeof(float), "optimizer hyper-parameters");
    }
    return true;
}

void save_hyper_device(const std::string& path, const HyperDims& d, const std::vector<DevTensor>& w,
                       const OptHeader* opt, const std::vector<DevTensor>& states) {
    const auto sizes = hyper_sizes(d);
    check_dev(w, sizes, 1, "save_hypernetwork_weights");
    if (opt) check_dev(states, sizes, opt->n_states, "save_hypernetwork_weights (optimizer)");
    hip_check(hipDeviceSynchronize(), "checkpoint: device synchronize");
    std::vector<std::vector<float>> hw, hs;
    std::vector<const float*> pw, ps;
    for (const auto& t : w) hw.push_back(download(t));
    for (const auto& h : hw) pw.push_back(h.data());
    if (opt) {
        for (const auto& t : states) hs.push_back(download(t));
        for (const auto& h : hs) ps.push_back(h.data());
    }
    write_hyper(path, d, pw, opt, ps);
}

void load_hyper_device(const std::string& path, const HyperDims& d, const std::vector<DevTensor>& w,
                       OptHeader* opt, const std::vector<DevTensor>& states) {
    const auto sizes = hyper_sizes(d);
    check_dev(w, sizes, 1, "load_hypernetwork_weights");
    const uint32_t per = opt ? (uint32_t)(states.size() / kHyperParams) : 0;
    if (opt) check_dev(states, sizes, per, "load_hypernetwork_weights (optimizer)");
    std::vector<std::vector<float>> hw, hs;
    std::vector<float*> pw, ps;
    for (uint32_t i = 0; i < kHyperParams; ++i) hw.emplace_back(sizes[i]);
    for (auto& h : hw) pw.push_back(h.data());
    if (opt) {
        for (size_t i = 0; i < states.size(); ++i) hs.emplace_back(sizes[i / per]);
        for (auto& h : hs) ps.push_back(h.data());
    }
    read_hyper(path, d, pw, opt, ps, per);  // the whole file is checked before any upload
    hip_check(hipDeviceSynchronize(), "checkpoint: device synchronize");
    for (uint32_t i = 0; i < kHyperParams; ++i) upload(w[i], hw[i]);
    for (size_t i = 0; i < hs.size(); ++i) upload(states[i], hs[i]);
}

}  // namespace ckpt
}  // namespace grilly
