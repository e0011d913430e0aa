// bindings.cpp — pybind11 module `_grilly_core` (imported as grilly_core through
// grilly_core.py): the reference's autograd API surface
// (cpp/python/bindings.cpp:2688-2880) on the MI355X tape engine, plus a Device with
// explicit buffer upload/download (the reference gives Python no way to create a buffer
// id for its own data, bindings.cpp:2725).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include "autograd.h"
#include "checkpoint.h"
#include "device.h"
#include "gn_bwd.h"
#include "hypernet.h"
#include "op_graph.h"

namespace py = pybind11;
using namespace grilly;
using namespace grilly::autograd;

namespace {

py::dict stats_dict(const BackwardEngine::Stats& s) {
    py::dict d;
    d["nodes_visited"] = s.nodes_visited;
    d["nodes_with_grad"] = s.nodes_with_grad;
    d["shaders_dispatched"] = s.shaders_dispatched;
    d["cpu_fallbacks"] = s.cpu_fallbacks;
    d["fanout_accumulations"] = s.fanout_accumulations;
    return d;
}

}  // namespace

PYBIND11_MODULE(_grilly_core, m) {
    m.doc() = "grilly-next tape autograd on MI355X (HIP kernels through libgn_bwd's C ABI)";
    m.attr("__backend__") = "hip-gfx950";
    m.def("kernel_library_version", []() { return std::string(gn_version()); });

    py::class_<Device>(m, "Device")
        .def(py::init<int>(), py::arg("index") = 0)
        .def_property_readonly("name", &Device::name)
        .def_property_readonly("index", &Device::index)
        .def("use_stream", &Device::use_stream, py::arg("stream_handle"),
             "Launch on a caller-owned HIP stream (e.g. torch.cuda.current_stream().cuda_stream); "
             "0 = the null (default) stream")
        .def("use_own_stream", &Device::use_own_stream, "Launch on the device's own stream again")
        .def("stream_handle", [](const Device& d) { return reinterpret_cast<uint64_t>(d.stream()); })
        .def("alloc", &Device::acquire, py::arg("nbytes"))
        .def("free", &Device::release, py::arg("buffer_id"))
        .def("buffer_bytes", &Device::buffer_bytes, py::arg("buffer_id"))
        .def("upload",
             [](Device& d, py::array arr) {
                 py::buffer_info bi = py::array::ensure(arr, py::array::c_style).request();
                 const size_t bytes = (size_t)bi.size * bi.itemsize;
                 uint64_t id = d.acquire(bytes);
                 d.upload(id, bi.ptr, bytes);
                 return id;
             },
             py::arg("array"), "Allocate a pool buffer holding a copy of `array`; returns its id")
        .def("upload_to",
             [](Device& d, uint64_t id, py::array arr, size_t offset) {
                 py::buffer_info bi = py::array::ensure(arr, py::array::c_style).request();
                 d.upload(id, bi.ptr, (size_t)bi.size * bi.itemsize, offset);
             },
             py::arg("buffer_id"), py::arg("array"), py::arg("offset") = 0)
        .def("download",
             [](Device& d, uint64_t id, std::vector<ssize_t> shape, py::dtype dtype) {
                 py::array out(dtype, shape);
                 d.download(id, out.mutable_data(), (size_t)out.nbytes());
                 return out;
             },
             py::arg("buffer_id"), py::arg("shape"), py::arg("dtype"))
        .def("zero", &Device::zero, py::arg("buffer_id"), py::arg("nbytes"))
        .def("synchronize", &Device::synchronize)
        .def("trim", &Device::trim)
        .def("pool_stats", [](const Device& d) {
            auto s = d.stats();
            py::dict r;
            r["bytes_live"] = s.bytes_live;
            r["bytes_cached"] = s.bytes_cached;
            r["allocs"] = s.allocs;
            r["reuses"] = s.reuses;
            return r;
        });

    py::enum_<OpType>(m, "OpType")
        .value("Add", OpType::Add).value("Sub", OpType::Sub).value("Mul", OpType::Mul)
        .value("Div", OpType::Div).value("Neg", OpType::Neg).value("Pow", OpType::Pow)
        .value("MatMul", OpType::MatMul).value("Linear", OpType::Linear)
        .value("ReLU", OpType::ReLU).value("GELU", OpType::GELU).value("SiLU", OpType::SiLU)
        .value("Tanh", OpType::Tanh).value("Sigmoid", OpType::Sigmoid)
        .value("Softmax", OpType::Softmax).value("LayerNorm", OpType::LayerNorm)
        .value("RMSNorm", OpType::RMSNorm).value("FlashAttention2", OpType::FlashAttention2)
        .value("Conv2d", OpType::Conv2d).value("Conv1d", OpType::Conv1d)
        .value("Sum", OpType::Sum).value("Mean", OpType::Mean).value("Max", OpType::Max)
        .value("Min", OpType::Min).value("Reshape", OpType::Reshape)
        .value("Transpose", OpType::Transpose).value("Slice", OpType::Slice)
        .value("CrossEntropy", OpType::CrossEntropy).value("MSELoss", OpType::MSELoss)
        .value("CubeMindSurprise", OpType::CubeMindSurprise)
        .value("TemporalSurprise", OpType::TemporalSurprise)
        .value("VSAUnpackProject", OpType::VSAUnpackProject)
        .value("VSASurrogateLoss", OpType::VSASurrogateLoss)
        .value("VSALoRAExpand", OpType::VSALoRAExpand)
        .value("VSACosineBlendLoss", OpType::VSACosineBlendLoss)
        .value("FusedGLU", OpType::FusedGLU)
        .value("Embedding", OpType::Embedding)
        .export_values();

    py::class_<TensorRef>(m, "TensorRef")
        .def(py::init([]() { return TensorRef::none(); }))
        .def_readwrite("buffer_id", &TensorRef::buffer_id)
        .def_readwrite("ndim", &TensorRef::ndim)
        .def_readwrite("dtype", &TensorRef::dtype)
        .def_readwrite("requires_grad", &TensorRef::requires_grad)
        .def("numel", &TensorRef::numel)
        .def("size_bytes", &TensorRef::size_bytes)
        .def("valid", &TensorRef::valid)
        .def_static("none", &TensorRef::none)
        .def("set_shape",
             [](TensorRef& r, const std::vector<uint32_t>& shape) {
                 if (shape.size() > 8) throw py::value_error("TensorRef: at most 8 dimensions");
                 r.ndim = (uint32_t)shape.size();
                 for (uint32_t i = 0; i < r.ndim; ++i) r.shape[i] = shape[i];
             },
             py::arg("shape"))
        .def("get_shape", [](const TensorRef& r) {
            return std::vector<uint32_t>(r.shape, r.shape + r.ndim);
        });

    py::class_<TapeContext>(m, "TapeContext")
        .def(py::init<Device&, size_t>(), py::arg("device"),
             py::arg("arena_capacity") = TapeArena::kDefaultCapacity, py::keep_alive<1, 2>())
        .def("begin", &TapeContext::begin)
        .def("record_op",
             [](TapeContext& t, OpType op, const std::vector<TensorRef>& inputs,
                const std::vector<TensorRef>& outputs, py::bytes params) {
                 std::string p = params;
                 return t.record_op(op, inputs.data(), (uint32_t)inputs.size(), outputs.data(),
                                    (uint32_t)outputs.size(), p.empty() ? nullptr : p.data(),
                                    (uint32_t)p.size());
             },
             py::arg("op"), py::arg("inputs"), py::arg("outputs"), py::arg("params") = py::bytes(),
             py::return_value_policy::reference)
        .def("save_for_backward",
             [](TapeContext& t, Node* node, const std::vector<uint64_t>& ids) {
                 t.save_for_backward(node, ids.data(), (uint32_t)ids.size());
             },
             py::arg("node"), py::arg("buffer_ids"))
        .def("backward",
             [](TapeContext& t, Node* loss, uint64_t g) { t.backward(loss, g); },
             py::arg("loss_node"), py::arg("grad_output_buffer"))
        .def("get_grad_buffer", &TapeContext::get_grad_buffer, py::arg("input_buffer_id"))
        // no counterpart in the reference: the down projection's backward forms the GLU's
        // local gradients in its epilogue (the GLU output's gradient is then not kept)
        .def("set_glu_epilogue", &TapeContext::set_glu_epilogue, py::arg("on"))
        .def("glu_epilogue", &TapeContext::glu_epilogue)
        .def("record_temporal_surprise",
             [](TapeContext& t, const TensorRef& input, const TensorRef& output, float coh,
                float contra, uint32_t branches, uint32_t dt, float alpha) {
                 TemporalSurpriseParams p{coh, contra, 1.0f - 2.0f * contra, alpha, branches, dt};
                 TensorRef ins[1] = {input}, outs[1] = {output};
                 return t.record_op(OpType::TemporalSurprise, ins, 1, outs, 1, &p, sizeof(p));
             },
             py::arg("input"), py::arg("output"), py::arg("avg_coherence"),
             py::arg("avg_contradiction"), py::arg("num_branches") = 128, py::arg("dt") = 1,
             py::arg("alpha") = 1.0f, py::return_value_policy::reference)
        .def("end", &TapeContext::end)
        .def("acquire_temp", &TapeContext::acquire_temp, py::arg("nbytes"))
        .def("is_recording", &TapeContext::is_recording)
        .def("arena_bytes_used", &TapeContext::arena_bytes_used)
        .def("arena_utilization", &TapeContext::arena_utilization)
        .def("last_backward_stats", [](const TapeContext& t) { return stats_dict(t.last_backward_stats()); });

    py::class_<Node>(m, "AutogradNode")
        .def_readonly("op", &Node::op)
        .def_readonly("seq", &Node::seq)
        .def_readonly("num_inputs", &Node::num_inputs)
        .def_readonly("num_outputs", &Node::num_outputs)
        .def_readonly("num_saved", &Node::num_saved)
        .def_readonly("grad_output_buffer", &Node::grad_output_buffer)
        .def("get_grad_input_buffer",
             [](const Node& n, uint32_t i) -> uint64_t { return i < kMaxNodeIO ? n.grad_input_buffers[i] : 0; },
             py::arg("index"))
        .def("get_input",
             [](const Node& n, uint32_t i) { return i < kMaxNodeIO ? n.inputs[i] : TensorRef::none(); },
             py::arg("index"))
        .def("get_output",
             [](const Node& n, uint32_t i) { return i < kMaxNodeIO ? n.outputs[i] : TensorRef::none(); },
             py::arg("index"))
        .def("get_saved_buffer",
             [](const Node& n, uint32_t i) -> uint64_t { return i < kMaxNodeIO ? n.saved_buffer_ids[i] : 0; },
             py::arg("index"));

    // OpGraph (bindings.cpp:212-235 of the reference): recorded launches replayed as one
    // HIP graph.  The reference records with addOp from C++; here launches are recorded by
    // capturing them (begin_capture/end_capture, or capture_backward for a tape's backward).
    py::class_<OpGraph>(m, "OpGraph")
        .def(py::init<>())
        .def("size", &OpGraph::size, "Number of kernel launches recorded in the graph")
        .def("clear", &OpGraph::clear,
             "Drop the recorded launches; the buffers pinned by the captures go back to the pool")
        .def("optimize",
             [](OpGraph& g, Device& dev) {
                 FusionStats st = g.optimize(dev);
                 py::dict d;
                 d["ops_fused"] = st.opsFused;
                 d["barriers_eliminated"] = st.barriersEliminated;
                 d["original_ops"] = st.originalOps;
                 d["optimized_ops"] = st.optimizedOps;
                 return d;
             },
             py::arg("device"), "Instantiate the executable graph; returns the reference's statistics")
        .def("execute", &OpGraph::execute, py::arg("device"),
             "Replay every recorded launch with one hipGraphLaunch on the device's current stream")
        .def("begin_capture", &OpGraph::begin_capture, py::arg("device"), py::keep_alive<1, 2>(),
             "Record the launches issued on `device` until end_capture()")
        .def("end_capture", &OpGraph::end_capture)
        .def("capture_backward",
             [](OpGraph& g, TapeContext& t, Node* loss, uint64_t grad) { g.capture_backward(t, loss, grad); },
             py::arg("tape"), py::arg("loss_node"), py::arg("grad_output_buffer") = 0,
             py::keep_alive<1, 2>(),
             "Record the tape's backward pass (nothing runs until execute) and keep its gradient table")
        .def("get_grad_buffer", &OpGraph::get_grad_buffer, py::arg("input_buffer_id"))
        .def("is_capturing", &OpGraph::capturing)
        .def("replays", &OpGraph::replays)
        .def("node_counts", [](const OpGraph& g) {
            OpGraph::NodeCounts c = g.node_counts();
            py::dict d;
            d["kernel"] = c.kernel;
            d["memcpy"] = c.memcpy;
            d["memset"] = c.memset;
            d["other"] = c.other;
            return d;
        });

    // Host-only view of the bump allocator, for tests of its failure behaviour.
    py::class_<TapeArena>(m, "_TapeArena")
        .def(py::init<size_t>(), py::arg("capacity"))
        .def("allocate", [](TapeArena& a, size_t bytes, size_t align) {
            return reinterpret_cast<uintptr_t>(a.allocate_bytes(bytes, align));
        }, py::arg("nbytes"), py::arg("align") = 16)
        .def("reset", &TapeArena::reset)
        .def("bytes_used", &TapeArena::bytes_used)
        .def("utilization", &TapeArena::utilization)
        .def("save", [](const TapeArena& a) { return a.save().offset; })
        .def("restore", [](TapeArena& a, size_t off) { a.restore({off, nullptr}); });
    m.attr("NODE_BYTES") = sizeof(Node);

    // ---- GRLY v3 hypernetwork checkpoint (bindings.cpp:2965-3039) + optimizer section ----
    // dims = (d_model, vsa_dim, K, router_hidden); opt = None or dict(kind, n_states, step,
    // hyper).  The grilly_bridge functions save/load_hypernetwork_weights wrap these.
    using FArr = py::array_t<float, py::array::c_style | py::array::forcecast>;
    auto to_dims = [](const std::array<uint32_t, 4>& a) {
        ckpt::HyperDims d;
        d.d_model = a[0]; d.vsa_dim = a[1]; d.K = a[2]; d.router_hidden = a[3];
        return d;
    };
    auto to_opt = [](const py::dict& o) {
        ckpt::OptHeader h;
        h.kind = o["kind"].cast<uint32_t>();
        h.n_states = o["n_states"].cast<uint32_t>();
        h.step = o["step"].cast<uint64_t>();
        h.hyper = o["hyper"].cast<std::vector<float>>();
        return h;
    };
    auto from_opt = [](const ckpt::OptHeader& h) {
        py::dict o;
        o["kind"] = h.kind; o["n_states"] = h.n_states; o["step"] = h.step; o["hyper"] = h.hyper;
        return o;
    };
    auto to_dev = [](const std::vector<std::tuple<uint64_t, uint64_t, int>>& v) {
        std::vector<ckpt::DevTensor> out;
        for (const auto& t : v) out.push_back({std::get<0>(t), std::get<1>(t), std::get<2>(t)});
        return out;
    };
    m.def("hypernetwork_sizes", [to_dims](const std::array<uint32_t, 4>& dims) {
        return ckpt::hyper_sizes(to_dims(dims));
    }, py::arg("dims"));
    m.def("_grly_write", [to_dims, to_opt](const std::string& path, const std::array<uint32_t, 4>& dims,
                                          const std::vector<FArr>& w, py::object opt,
                                          const std::vector<FArr>& states) {
        std::vector<const float*> pw, ps;
        for (const auto& a : w) pw.push_back(a.data());
        for (const auto& a : states) ps.push_back(a.data());
        const auto sizes = ckpt::hyper_sizes(to_dims(dims));
        for (size_t i = 0; i < w.size() && i < sizes.size(); ++i)
            if ((uint64_t)w[i].size() != sizes[i]) throw std::invalid_argument("_grly_write: tensor size");
        ckpt::OptHeader h;
        if (!opt.is_none()) h = to_opt(opt.cast<py::dict>());
        for (size_t i = 0; i < states.size(); ++i)
            if (h.n_states == 0 || (uint64_t)states[i].size() != sizes[i / h.n_states])
                throw std::invalid_argument("_grly_write: state tensor size");
        ckpt::write_hyper(path, to_dims(dims), pw, opt.is_none() ? nullptr : &h, ps);
    }, py::arg("path"), py::arg("dims"), py::arg("weights"), py::arg("opt"), py::arg("states"));
    m.def("_grly_read", [to_dims, from_opt](const std::string& path, const std::array<uint32_t, 4>& dims,
                                           int opt_states) {
        const auto d = to_dims(dims);
        const auto sizes = ckpt::hyper_sizes(d);
        std::vector<FArr> w, st;
        std::vector<float*> pw, ps;
        for (uint64_t n : sizes) w.emplace_back((py::ssize_t)n);
        for (auto& a : w) pw.push_back(a.mutable_data());
        ckpt::OptHeader h;
        if (opt_states >= 0)
            for (size_t i = 0; i < sizes.size() * (size_t)opt_states; ++i) st.emplace_back((py::ssize_t)sizes[i / opt_states]);
        for (auto& a : st) ps.push_back(a.mutable_data());
        ckpt::read_hyper(path, d, pw, opt_states >= 0 ? &h : nullptr, ps, (uint32_t)std::max(opt_states, 0));
        return py::make_tuple(w, opt_states >= 0 ? py::object(from_opt(h)) : py::none(), st);
    }, py::arg("path"), py::arg("dims"), py::arg("opt_states") = -1);
    m.def("_grly_probe", [from_opt](const std::string& path) {
        ckpt::HyperDims d;
        ckpt::OptHeader h;
        const bool has = ckpt::probe_hyper(path, &d, &h);
        return py::make_tuple(std::array<uint32_t, 4>{d.d_model, d.vsa_dim, d.K, d.router_hidden},
                              has ? py::object(from_opt(h)) : py::none());
    }, py::arg("path"));
    m.def("_grly_save_device", [to_dims, to_opt, to_dev](const std::string& path, const std::array<uint32_t, 4>& dims,
                                                       const std::vector<std::tuple<uint64_t, uint64_t, int>>& w,
                                                       py::object opt,
                                                       const std::vector<std::tuple<uint64_t, uint64_t, int>>& states) {
        ckpt::OptHeader h;
        if (!opt.is_none()) h = to_opt(opt.cast<py::dict>());
        py::gil_scoped_release nogil;
        ckpt::save_hyper_device(path, to_dims(dims), to_dev(w), opt.is_none() ? nullptr : &h, to_dev(states));
    }, py::arg("path"), py::arg("dims"), py::arg("weights"), py::arg("opt"), py::arg("states"));
    m.def("_grly_load_device", [to_dims, to_dev, from_opt](const std::string& path, const std::array<uint32_t, 4>& dims,
                                                         const std::vector<std::tuple<uint64_t, uint64_t, int>>& w,
                                                         bool with_opt,
                                                         const std::vector<std::tuple<uint64_t, uint64_t, int>>& states) {
        ckpt::OptHeader h;
        {
            py::gil_scoped_release nogil;
            ckpt::load_hyper_device(path, to_dims(dims), to_dev(w), with_opt ? &h : nullptr, to_dev(states));
        }
        return with_opt ? py::object(from_opt(h)) : py::none();
    }, py::arg("path"), py::arg("dims"), py::arg("weights"), py::arg("with_opt"), py::arg("states"));

    // ---- VSA hypernetwork, its optimizer and the training step (bindings.cpp:2883-3286) ----
    using models::SurpriseMomentumOptimizer;
    using models::VSAHypernetwork;
    using U32Arr = py::array_t<uint32_t, py::array::c_style | py::array::forcecast>;
    // rows x words of a bitpacked array: [words] is one row, [rows, words] a batch
    auto rows_words = [](const U32Arr& a) {
        if (a.ndim() == 1) return std::make_pair<uint32_t, uint32_t>(1, (uint32_t)a.shape(0));
        if (a.ndim() == 2) return std::make_pair((uint32_t)a.shape(0), (uint32_t)a.shape(1));
        throw py::value_error("bitpacked state: a uint32 array [words] or [rows, words] expected");
    };
    py::class_<VSAHypernetwork>(m, "VSAHypernetwork")
        .def(py::init<Device&, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t>(), py::arg("device"),
             py::arg("d_model") = 768, py::arg("vsa_dim") = 10240, py::arg("K") = 16,
             py::arg("router_hidden") = 32, py::arg("seed") = 42, py::keep_alive<1, 2>())
        .def("forward", &VSAHypernetwork::forward, py::arg("tape"), py::arg("vsa_state"))
        .def("parameter_buffer_ids", &VSAHypernetwork::parameter_buffer_ids)
        .def("parameter_sizes", &VSAHypernetwork::parameter_sizes)
        .def("last_output_buffer_id", [](const VSAHypernetwork& h) { return h.last_output().buffer_id; })
        .def("h_t_buffer_id", [](const VSAHypernetwork& h) { return h.h_t().buffer_id; })
        .def_property_readonly("d_model", &VSAHypernetwork::d_model)
        .def_property_readonly("vsa_dim", &VSAHypernetwork::vsa_dim)
        .def_property_readonly("K", &VSAHypernetwork::K)
        .def_property_readonly("router_hidden", &VSAHypernetwork::router_hidden)
        .def("num_weight_bufs", &VSAHypernetwork::num_weight_bufs)
        .def_readwrite("gumbel_seed", &VSAHypernetwork::gumbel_seed,
                       "seed of the surrogate loss's Gumbel noise (default: the model seed)")
        .def_readwrite("gumbel_counter", &VSAHypernetwork::gumbel_counter,
                       "draw index of the next loss forward; advances once per training step")
        .def("forward_inference",
             [rows_words](VSAHypernetwork& self, Device& dev, TapeContext& tape, const U32Arr& state) {
                 const auto rw = rows_words(state);
                 if (rw.first != 1) throw py::value_error("forward_inference: one state [words] expected");
                 py::array_t<float> out({(py::ssize_t)self.K(), (py::ssize_t)self.vsa_dim()});
                 {
                     py::gil_scoped_release nogil;
                     tape.begin();
                     try {
                         TensorRef s = models::upload_bitpacked(tape, state.data(), 1, rw.second);
                         TensorRef p = self.forward(tape, s);
                         dev.download(p.buffer_id, out.mutable_data(), (size_t)self.K() * self.vsa_dim() * 4);
                     } catch (...) {
                         tape.end();
                         throw;
                     }
                     tape.end();
                 }
                 return out;
             },
             py::arg("device"), py::arg("tape"), py::arg("vsa_state"),
             "Inference forward: upload the bitpacked state, run the network, return the K x vsa_dim "
             "float32 predictions");

    py::class_<SurpriseMomentumOptimizer>(m, "SurpriseMomentumOptimizer")
        .def(py::init<Device&, const VSAHypernetwork&, float, float, float>(), py::arg("device"),
             py::arg("model"), py::arg("lr") = 0.001f, py::arg("alpha") = 0.9f, py::arg("clip") = 1.0f,
             py::keep_alive<1, 2>(), py::keep_alive<1, 3>())
        .def_readwrite("eta_base", &SurpriseMomentumOptimizer::eta_base)
        .def_readwrite("alpha_momentum", &SurpriseMomentumOptimizer::alpha_momentum)
        .def_readwrite("lambda_recall", &SurpriseMomentumOptimizer::lambda_recall)
        .def_readwrite("surprise_floor", &SurpriseMomentumOptimizer::surprise_floor)
        .def_readwrite("weight_decay", &SurpriseMomentumOptimizer::weight_decay)
        .def_readwrite("clip_max", &SurpriseMomentumOptimizer::clip_max)
        .def_readwrite("steps", &SurpriseMomentumOptimizer::steps)
        .def_readwrite("fuse_linear_updates", &SurpriseMomentumOptimizer::fuse_linear_updates,
                       "Apply a weight's step inside its Linear backward when a few rows use it "
                       "(same result bit for bit; False runs the separate optimizer pass)")
        .def("prepare", &SurpriseMomentumOptimizer::prepare, py::arg("tape"),
             "Before backward: hand the steps of Linear-only weights to the backward pass")
        .def("apply", &SurpriseMomentumOptimizer::apply, py::arg("tape"),
             "Update every parameter whose gradient the tape holds (between backward and end)")
        .def("s_bar_buffer_ids", &SurpriseMomentumOptimizer::s_bar_buffer_ids);

    m.def("upload_bitpacked",
          [rows_words](TapeContext& tape, const U32Arr& a) {
              const auto rw = rows_words(a);
              return models::upload_bitpacked(tape, a.data(), rw.first, rw.second);
          },
          py::arg("tape"), py::arg("data"), "Step-scoped u32 buffer holding the bitpacked rows");
    m.def("record_surrogate_loss", &models::record_surrogate_loss, py::arg("tape"), py::arg("predicted"),
          py::arg("true_delta"), py::return_value_policy::reference);
    m.def("vsa_loss_forward",
          [](TapeContext& tape, Node* node, uint64_t seed, uint64_t counter, bool noise) {
              py::gil_scoped_release nogil;
              return models::vsa_loss_forward(tape, node, seed, counter, noise);
          },
          py::arg("tape"), py::arg("loss_node"), py::arg("seed"), py::arg("counter"), py::arg("noise") = true);
    m.def("vsa_training_step",
          [rows_words](Device& dev, TapeContext& tape, VSAHypernetwork& model, const U32Arr& state,
                       const U32Arr& delta, py::object optimizer) {
              const auto rw = rows_words(state), rd = rows_words(delta);
              if (rw != rd) throw py::value_error("vsa_training_step: state and true_delta shapes differ");
              if (&dev != &model.device())
                  throw py::value_error("vsa_training_step: the model lives on another Device");
              SurpriseMomentumOptimizer* opt =
                  optimizer.is_none() ? nullptr : &optimizer.cast<SurpriseMomentumOptimizer&>();
              py::gil_scoped_release nogil;
              return models::vsa_training_step(tape, model, state.data(), delta.data(), rw.first,
                                               rw.second, opt);
          },
          py::arg("device"), py::arg("tape"), py::arg("model"), py::arg("vsa_state"),
          py::arg("true_delta"), py::arg("optimizer") = py::none(),
          "Run one VSA training step: forward + loss + backward + optimizer. Returns the loss.");

    // GRLY v3 checkpoint of a VSAHypernetwork (bindings.cpp:2965-3039); with a
    // SurpriseMomentumOptimizer its s_bar follows in this build's optimizer section
    auto model_dims = [](const VSAHypernetwork& h) {
        ckpt::HyperDims d;
        d.d_model = h.d_model(); d.vsa_dim = h.vsa_dim(); d.K = h.K(); d.router_hidden = h.router_hidden();
        return d;
    };
    auto dev_tensors = [](const std::vector<uint64_t>& ids, const std::vector<uint64_t>& sizes) {
        std::vector<ckpt::DevTensor> v;
        for (size_t i = 0; i < ids.size(); ++i) v.push_back({ids[i], sizes[i], 0});
        return v;
    };
    auto opt_header = [](const SurpriseMomentumOptimizer& o) {
        ckpt::OptHeader h;
        h.kind = 0;
        h.n_states = 1;
        h.step = o.steps;
        h.hyper = {o.eta_base, o.alpha_momentum, o.lambda_recall, o.surprise_floor, o.weight_decay, o.clip_max};
        return h;
    };
    m.def("save_hypernetwork_weights",
          [model_dims, dev_tensors, opt_header](VSAHypernetwork& model, const std::string& path,
                                                py::object optimizer) {
              const auto sizes = model.parameter_sizes();
              const auto w = dev_tensors(model.parameter_buffer_ids(), sizes);
              if (optimizer.is_none()) {
                  py::gil_scoped_release nogil;
                  ckpt::save_hyper_device(path, model_dims(model), w, nullptr, {});
                  return;
              }
              auto& o = optimizer.cast<SurpriseMomentumOptimizer&>();
              const ckpt::OptHeader h = opt_header(o);
              const auto st = dev_tensors(o.s_bar_buffer_ids(), sizes);
              py::gil_scoped_release nogil;
              ckpt::save_hyper_device(path, model_dims(model), w, &h, st);
          },
          py::arg("model"), py::arg("path"), py::arg("optimizer") = py::none(),
          "Save VSAHypernetwork weights (GRLY v3); with an optimizer, also its state");
    m.def("load_hypernetwork_weights",
          [model_dims, dev_tensors](VSAHypernetwork& model, const std::string& path, py::object optimizer) {
              const auto sizes = model.parameter_sizes();
              const auto w = dev_tensors(model.parameter_buffer_ids(), sizes);
              if (optimizer.is_none()) {
                  py::gil_scoped_release nogil;
                  ckpt::load_hyper_device(path, model_dims(model), w, nullptr, {});
                  return;
              }
              auto& o = optimizer.cast<SurpriseMomentumOptimizer&>();
              ckpt::HyperDims pd;
              ckpt::OptHeader info;
              if (!ckpt::probe_hyper(path, &pd, &info) || info.kind != 0 || info.n_states < 1 ||
                  info.n_states > 2)
                  throw py::value_error(path + ": no SurpriseMomentumOptimizer state in this checkpoint");
              // a second state per parameter (the update `delta`) is read and dropped
              std::vector<ckpt::DevTensor> st;
              std::vector<uint64_t> scratch;
              Device& dev = model.device();
              const auto sb = o.s_bar_buffer_ids();
              for (size_t i = 0; i < sizes.size(); ++i) {
                  st.push_back({sb[i], sizes[i], 0});
                  if (info.n_states == 2) {
                      scratch.push_back(dev.acquire(sizes[i] * 4));
                      st.push_back({scratch.back(), sizes[i], 0});
                  }
              }
              ckpt::OptHeader h;
              {
                  py::gil_scoped_release nogil;
                  try {
                      ckpt::load_hyper_device(path, model_dims(model), w, &h, st);
                  } catch (...) {
                      for (uint64_t id : scratch) dev.release(id);
                      throw;
                  }
                  dev.synchronize();
              }
              for (uint64_t id : scratch) dev.release(id);
              o.steps = h.step;
              if (h.hyper.size() >= 6) {
                  o.eta_base = h.hyper[0]; o.alpha_momentum = h.hyper[1]; o.lambda_recall = h.hyper[2];
                  o.surprise_floor = h.hyper[3]; o.weight_decay = h.hyper[4]; o.clip_max = h.hyper[5];
              }
          },
          py::arg("model"), py::arg("path"), py::arg("optimizer") = py::none(),
          "Load VSAHypernetwork weights (checks magic, dimensions and every tensor's count)");

    py::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const std::length_error& e) {
            PyErr_SetString(PyExc_OverflowError, e.what());
        }
    });
}
