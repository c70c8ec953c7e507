// Python module `edge_fm`: the reference's pybind surface (src/python/pybind_debug.cpp:
// 313-1735) for the MI355X runtime — DType / Device / ModelStage, Tensor (zero-copy
// views of device memory, DLPack export as kDLROCM, copying DLPack import), Request /
// Response, EdgeFM with generate() and last_generate_metrics(), the WeightLoader
// singleton, apply_mrope, and the layer tier (pybind_layers.cpp).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <ATen/dlpack.h>

#include "engine.hpp"

namespace py = pybind11;
using namespace edge_fm;

namespace {

DLDataType to_dl(DType d) {
    switch (d) {
        case DType::Float32: return {kDLFloat, 32, 1};
        case DType::Float16: return {kDLFloat, 16, 1};
        case DType::BFloat16: return {kDLBfloat, 16, 1};
        case DType::Int32: return {kDLInt, 32, 1};
        case DType::Int64: return {kDLInt, 64, 1};
        case DType::UInt8: return {kDLUInt, 8, 1};
        case DType::Int8: return {kDLInt, 8, 1};
    }
    return {kDLFloat, 32, 1};
}

struct DLHolder {
    Tensor t;  // keeps the storage alive
    std::vector<int64_t> shape, strides;
    DLManagedTensor managed{};
};

py::capsule to_dlpack(const Tensor& t) {
    auto* h = new DLHolder();
    h->t = t;
    h->shape = t.shape();
    h->strides.resize(h->shape.size());
    int64_t s = 1;
    for (int i = (int)h->shape.size() - 1; i >= 0; --i) {
        h->strides[i] = s;
        s *= h->shape[i];
    }
    auto [dev, did] = t.device();
    DLTensor& d = h->managed.dl_tensor;
    d.data = t.data_ptr();
    d.device = {dev == Device::GPU ? kDLROCM : kDLCPU, did};  // ROCm export (reference: kDLCUDA, tensor.cpp:40)
    d.ndim = (int32_t)h->shape.size();
    d.dtype = to_dl(t.dtype());
    d.shape = h->shape.data();
    d.strides = h->strides.data();
    d.byte_offset = 0;
    h->managed.manager_ctx = h;
    h->managed.deleter = [](DLManagedTensor* m) { delete static_cast<DLHolder*>(m->manager_ctx); };
    return py::capsule(&h->managed, "dltensor", [](PyObject* cap) {
        if (PyCapsule_IsValid(cap, "dltensor")) {
            auto* m = static_cast<DLManagedTensor*>(PyCapsule_GetPointer(cap, "dltensor"));
            if (m && m->deleter) m->deleter(m);
        }
    });
}

DType from_dl(const DLDataType& t) {
    if (t.lanes == 1) {
        if (t.code == kDLFloat && t.bits == 32) return DType::Float32;
        if (t.code == kDLFloat && t.bits == 16) return DType::Float16;
        if (t.code == kDLBfloat && t.bits == 16) return DType::BFloat16;
        if (t.code == kDLInt && t.bits == 32) return DType::Int32;
        if (t.code == kDLInt && t.bits == 64) return DType::Int64;
        if (t.code == kDLUInt && t.bits == 8) return DType::UInt8;
        if (t.code == kDLInt && t.bits == 8) return DType::Int8;
    }
    throw InvalidArgumentError("from_dlpack: unsupported dtype (code " + std::to_string(t.code) + ", bits " +
                               std::to_string(t.bits) + ")");
}

// A new tensor holding a copy of a DLPack capsule's data (Tensor.from_dlpack,
// pybind_debug.cpp:437-449: the data is copied, the capsule may be released afterwards).
// Row-major contiguous data only; a GPU source is copied after the device is idle, so
// work queued on any stream of the producer has finished.
Tensor from_dlpack(py::capsule cap) {
    PyObject* obj = cap.ptr();
    if (!PyCapsule_IsValid(obj, "dltensor"))
        throw InvalidArgumentError("from_dlpack: expected an unconsumed 'dltensor' capsule");
    auto* mt = static_cast<DLManagedTensor*>(PyCapsule_GetPointer(obj, "dltensor"));
    const DLTensor& d = mt->dl_tensor;
    std::vector<int64_t> shape(d.shape, d.shape + d.ndim);
    if (d.strides != nullptr) {
        int64_t expect = 1;
        for (int i = d.ndim - 1; i >= 0; --i) {
            if (shape[i] != 1 && d.strides[i] != expect)
                throw InvalidArgumentError("from_dlpack: tensor must be contiguous and row-major");
            expect *= shape[i];
        }
    }
    const DType dt = from_dl(d.dtype);
    const bool gpu = d.device.device_type == kDLROCM || d.device.device_type == kDLCUDA;
    if (!gpu && d.device.device_type != kDLCPU) throw InvalidArgumentError("from_dlpack: unsupported device type");
    const Device dev = gpu ? Device::GPU : Device::CPU;
    const int32_t id = gpu ? d.device.device_id : 0;
    const void* src = static_cast<const char*>(d.data) + d.byte_offset;
    if (gpu) {
        hip_check(hipSetDevice(id), "hipSetDevice");
        hip_check(hipDeviceSynchronize(), "from_dlpack sync");
    }
    Tensor t = Tensor::clone_from(src, shape, dt, dev, id, dev, id, nullptr);
    PyCapsule_SetName(obj, "used_dltensor");
    if (mt->deleter) mt->deleter(mt);
    return t;
}

}  // namespace

namespace edge_fm {
void bind_layers(py::module_& m);   // pybind_layers.cpp
}

PYBIND11_MODULE(edge_fm, m) {
    m.doc() = "EdgeFM single-request transformer runtime for AMD Instinct MI355X (gfx950)";

    // exceptions -> Python (core.h:219-407); more specific types registered last so
    // they are matched first.
    auto base = py::register_exception<Error>(m, "Error", PyExc_RuntimeError);
    py::register_exception<InvalidRequestError>(m, "InvalidRequestError", base.ptr());
    py::register_exception<DeviceError>(m, "DeviceError", base.ptr());
    py::register_exception<ConfigurationError>(m, "ConfigurationError", base.ptr());
    py::register_exception<ModelNotLoadedError>(m, "ModelNotLoadedError", base.ptr());
    py::register_exception<OutOfMemoryError>(m, "OutOfMemoryError", base.ptr());
    py::register_exception<InternalError>(m, "InternalError", base.ptr());
    py::register_exception<InvalidArgumentError>(m, "InvalidArgumentError", base.ptr());

    py::enum_<DType>(m, "DType")
        .value("Float32", DType::Float32)
        .value("Float16", DType::Float16)
        .value("BFloat16", DType::BFloat16)
        .value("Int32", DType::Int32)
        .value("Int64", DType::Int64)
        .value("UInt8", DType::UInt8)
        .value("Int8", DType::Int8);
    py::enum_<Device>(m, "Device").value("CPU", Device::CPU).value("GPU", Device::GPU);
    py::enum_<ModelStage>(m, "ModelStage").value("Prefill", ModelStage::Prefill).value("Decode", ModelStage::Decode);

    py::class_<Tensor>(m, "Tensor")
        .def(py::init<>())
        .def(py::init([](uintptr_t ptr, std::vector<int64_t> shape, DType dtype, Device device, int32_t device_id,
                         bool owned) {
                 if (owned) throw InvalidArgumentError("Tensor(ptr, ...) creates views only; pass owned=False");
                 return Tensor::view(reinterpret_cast<void*>(ptr), std::move(shape), dtype, device, device_id);
             }),
             py::arg("data_ptr"), py::arg("shape"), py::arg("dtype"), py::arg("device") = Device::GPU,
             py::arg("device_id") = 0, py::arg("owned") = false)
        .def_static("view",
                    [](uintptr_t ptr, std::vector<int64_t> shape, DType dtype, Device device, int32_t device_id) {
                        return Tensor::view(reinterpret_cast<void*>(ptr), std::move(shape), dtype, device, device_id);
                    },
                    py::arg("data_ptr"), py::arg("shape"), py::arg("dtype"), py::arg("device"),
                    py::arg("device_id") = 0)
        .def_static("from_dlpack", &from_dlpack, py::arg("capsule"))
        .def("to_dlpack", &to_dlpack)
        .def("empty", [](const Tensor& t) { return t.empty(); })
        .def("dtype", &Tensor::dtype)
        .def("shape", &Tensor::shape)
        .def("device", &Tensor::device)
        .def("nbytes", &Tensor::nbytes)
        .def("data_ptr", [](const Tensor& t) { return reinterpret_cast<uintptr_t>(t.data_ptr()); });

    py::class_<Request>(m, "Request")
        .def(py::init<int32_t, std::vector<int32_t>>(), py::arg("request_id"), py::arg("token_ids"))
        .def(py::init([](int32_t rid, std::vector<int32_t> ids, const Tensor& emb, int32_t embed_token_id) {
                 Request r(rid, std::move(ids));
                 r.embedding = emb;
                 r.embed_token_id = embed_token_id;
                 return r;
             }),
             py::arg("request_id"), py::arg("token_ids"), py::arg("embedding"), py::arg("embed_token_id") = -1)
        .def(py::init([](int32_t rid, std::vector<int32_t> ids, const Tensor& emb, int32_t embed_token_id,
                         const Tensor& pos, std::vector<int32_t> last) {
                 Request r(rid, std::move(ids));
                 r.embedding = emb;
                 r.embed_token_id = embed_token_id;
                 r.position_ids = pos;
                 r.mrope_last_pos = std::move(last);
                 return r;
             }),
             py::arg("request_id"), py::arg("token_ids"), py::arg("embedding"), py::arg("embed_token_id"),
             py::arg("position_ids"), py::arg("mrope_last_pos") = std::vector<int32_t>{})
        .def("request_id", [](const Request& r) { return r.request_id; })
        .def("token_ids", [](const Request& r) { return r.token_ids; })
        .def("embedding", [](const Request& r) { return r.embedding; })
        .def("embed_token_id", [](const Request& r) { return r.embed_token_id; })
        .def("has_embedding", &Request::has_embedding)
        .def("position_ids", [](const Request& r) { return r.position_ids; })
        .def("has_position_ids", &Request::has_position_ids)
        .def("mrope_last_pos", [](const Request& r) { return r.mrope_last_pos; })
        .def("has_mrope_last_pos", [](const Request& r) { return !r.mrope_last_pos.empty(); })
        .def("set_stop_token_ids", [](Request& r, std::vector<int32_t> v) { r.stop_token_ids = std::move(v); })
        .def("stop_token_ids", [](const Request& r) { return r.stop_token_ids; })
        .def("set_ignore_stop_tokens", [](Request& r, bool v) { r.ignore_stop_tokens = v; })
        .def("ignore_stop_tokens", [](const Request& r) { return r.ignore_stop_tokens; });

    py::class_<Response>(m, "Response").def("token_ids", [](const Response& r) { return r.token_ids; });

    m.def("linear_scratch_bytes", &linear_scratch_bytes, py::arg("device_id") = 0,
          "bytes of the split-K scratch shared by the prefill projections on a device (grow-only)");

    py::class_<EdgeFM>(m, "EdgeFM")
        .def(py::init<const std::string&>(), py::arg("config_path"), py::call_guard<py::gil_scoped_release>())
        .def("generate", &EdgeFM::generate, py::arg("request"), py::call_guard<py::gil_scoped_release>())
        .def("last_generate_metrics", &EdgeFM::last_generate_metrics)
        .def("last_logits",
             [](const EdgeFM& e) {
                 int32_t rows = 0, vocab = 0;
                 std::vector<float> v = e.last_logits(&rows, &vocab);
                 py::array_t<float> a({(py::ssize_t)rows, (py::ssize_t)vocab});
                 std::copy(v.begin(), v.end(), a.mutable_data());
                 return a;
             },
             "fp32 logits [tokens, vocab] of every token of the last generate() (runtime.debug_logits)")
        .def("model_config", [](const EdgeFM& e) {
            const ModelConfig& c = e.engine().model_config();
            py::dict d;
            d["hidden_size"] = c.hidden;
            d["intermediate_size"] = c.inter;
            d["num_hidden_layers"] = c.layers;
            d["num_attention_heads"] = c.heads;
            d["num_key_value_heads"] = c.kv_heads;
            d["head_dim"] = c.head_dim;
            d["vocab_size"] = c.vocab;
            d["mrope"] = c.mrope;
            return d;
        });

    // Compact-vocabulary id mapping of an engine config (compact_vocab.h:12-53); host
    // only, so it is usable without a GPU.
    py::class_<CompactVocab>(m, "CompactVocab")
        .def(py::init([](const std::string& config_path) { return CompactVocab(EngineConfig(config_path)); }),
             py::arg("config_path"))
        .def("enabled", &CompactVocab::enabled)
        .def("original_vocab_size", &CompactVocab::original_vocab_size)
        .def("compact_vocab_size", &CompactVocab::compact_vocab_size)
        .def("mapping_path", &CompactVocab::mapping_path)
        .def("remap_token_ids", &CompactVocab::remap_token_ids, py::arg("ids"), py::arg("context"))
        .def("remap_required_token_ids", &CompactVocab::remap_required_token_ids, py::arg("ids"), py::arg("context"))
        .def("remap_optional_token_ids", &CompactVocab::remap_optional_token_ids, py::arg("ids"), py::arg("context"))
        .def("restore_token_ids", &CompactVocab::restore_token_ids, py::arg("ids"), py::arg("context"))
        .def("remap_request", &CompactVocab::remap_request, py::arg("request"));

    py::class_<WeightLoader, std::unique_ptr<WeightLoader, py::nodelete>>(m, "WeightLoader")
        .def_static("instance", &WeightLoader::instance, py::return_value_policy::reference)
        .def("load_weights_from_file", &WeightLoader::load_weights_from_file, py::arg("model_path"),
             py::arg("stage"), py::arg("device_id") = 0, py::arg("language_model_only") = false,
             py::call_guard<py::gil_scoped_release>())
        .def("register_tensor", &WeightLoader::register_tensor, py::arg("stage"), py::arg("name"), py::arg("tensor"))
        .def("get", [](WeightLoader& w, ModelStage s) {
            py::dict d;
            for (const auto& kv : w.get(s)) d[py::str(kv.first)] = kv.second;
            return d;
        })
        .def("clear_stage", &WeightLoader::clear_stage);

    // the decode plan an engine config resolves to (operator table, no device work)
    m.def("plan_decode", [](const std::string& path, uint32_t max_kv_len) {
        py::list out;
        for (const auto& p : plan_decode(path, max_kv_len)) {
            py::dict d;
            d["attention"] = p.attention;
            d["o_proj"] = p.o_proj;
            d["gate_up"] = p.gate_up;
            d["down"] = p.down;
            d["partials_to_o_proj"] = p.partials_to_o_proj;
            out.append(d);
        }
        return out;
    }, py::arg("engine_config_path"), py::arg("max_kv_len"));

    // checkpoint reading on the host (no device work): used by the loader tests
    m.def("collect_safetensors_files", &collect_safetensors_files, py::arg("model_path"));
    m.def("vl_language_model_name", &vl_language_model_name, py::arg("name"));
    m.def("read_safetensors_header", [](const std::string& path) {
        size_t data_off = 0;
        const auto entries = read_safetensors_header(path, &data_off);
        py::dict d;
        for (const auto& kv : entries)
            d[py::str(kv.first)] = py::make_tuple(kv.second.dtype, kv.second.shape, kv.second.begin, kv.second.end);
        return py::make_tuple(d, data_off);
    }, py::arg("path"));

    m.def("apply_mrope",
          [](Tensor& q, Tensor& k, const Tensor& position_ids, std::vector<int32_t> mrope_section, float rope_theta,
             float rope_scale) {
              check<InvalidArgumentError>(mrope_section.size() == 3, "mrope_section must have 3 entries");
              check<InvalidArgumentError>(q.shape().size() == 3 && k.shape().size() == 3, "q, k must be [S, H, hd]");
              const int32_t S = (int32_t)q.shape()[0];
              efm_check(efm_mrope(q.data_ptr(), k.data_ptr(), static_cast<const int32_t*>(position_ids.data_ptr()),
                                  (int32_t)position_ids.shape().back(), S, (int32_t)q.shape()[1], (int32_t)k.shape()[1],
                                  (int32_t)q.shape()[2], 0, 0, mrope_section[0], mrope_section[1], mrope_section[2],
                                  rope_theta, rope_scale, nullptr),
                        "apply_mrope");
              hip_check(hipStreamSynchronize(nullptr), "apply_mrope sync");
          },
          py::arg("q"), py::arg("k"), py::arg("position_ids"), py::arg("mrope_section"), py::arg("rope_theta"),
          py::arg("rope_scale") = 1.0f);

    bind_layers(m);

    m.attr("__version__") = efm_version();
}
