// checkpoint.cpp -- Checkpoint (include/inferno/checkpoint/checkpoint.h), in
// the reference's file format (src/inferno/checkpoint/checkpoint.cpp).
#include "inferno/checkpoint/checkpoint.h"

#include <cstring>
#include <fstream>
#include <stdexcept>

#include "detail.h"

namespace Inferno {

static_assert(sizeof(CheckpointHeader) == 16, "checkpoint header layout");
static_assert(sizeof(TensorRecordHeader) == 28, "tensor record layout");

namespace {
constexpr char kMagic[8] = "INFERNO";
}

void Checkpoint::save(const std::string& path) const {
    std::ofstream out(path, std::ios::binary);
    if (!out) throw std::runtime_error("Failed to open file: " + path);
    CheckpointHeader header{};
    std::memcpy(header.magic, kMagic, 8);
    header.version = 0;
    header.tensor_count = static_cast<uint32_t>(m_state_dict.size());
    out.write(reinterpret_cast<const char*>(&header), sizeof(header));
    if (!out) throw std::runtime_error("Failed while writing checkpoint header");
    for (const auto& [name, tensor] : m_state_dict) {
        Tensor t = tensor.device().is_cpu() ? tensor : tensor.to(Device::cpu());
        if (!t.is_contiguous()) t = t.contiguous();
        TensorRecordHeader trh{};
        trh.name_length = static_cast<uint32_t>(name.size());
        trh.dtype = static_cast<uint32_t>(t.dtype());
        trh.ndim = static_cast<uint32_t>(t.ndim());
        trh.numel = static_cast<uint64_t>(t.numel());
        trh.nbytes = static_cast<uint64_t>(t.size());
        out.write(reinterpret_cast<const char*>(&trh), sizeof(trh));
        for (size_t dim : t.shape()) {
            const uint64_t d = dim;
            out.write(reinterpret_cast<const char*>(&d), sizeof(d));
        }
        out.write(name.data(), trh.name_length);
        out.write(static_cast<const char*>(t.data_ptr()), (std::streamsize)trh.nbytes);
        if (!out) throw std::runtime_error("Failed while writing tensor: " + name);
    }
}

void Checkpoint::set_state_dict(const StateDict& state) { m_state_dict = state; }
const StateDict& Checkpoint::state_dict() const { return m_state_dict; }

Checkpoint Checkpoint::load(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("Failed to open checkpoint file for reading: " + path);
    CheckpointHeader header{};
    in.read(reinterpret_cast<char*>(&header), sizeof(header));
    if (!in) throw std::runtime_error("Failed to read checkpoint header");
    if (std::memcmp(header.magic, kMagic, 8) != 0) throw std::runtime_error("Invalid checkpoint file: bad magic");
    if (header.version != 0) throw std::runtime_error("Unsupported checkpoint version");
    Checkpoint ckpt;
    for (uint32_t i = 0; i < header.tensor_count; ++i) {
        TensorRecordHeader trh{};
        in.read(reinterpret_cast<char*>(&trh), sizeof(trh));
        if (!in) throw std::runtime_error("Failed to read tensor record header");
        std::vector<size_t> shape;
        shape.reserve(trh.ndim);
        for (uint32_t d = 0; d < trh.ndim; ++d) {
            uint64_t dim = 0;
            in.read(reinterpret_cast<char*>(&dim), sizeof(dim));
            if (!in) throw std::runtime_error("Failed to read tensor shape");
            shape.push_back(static_cast<size_t>(dim));
        }
        std::string name(trh.name_length, '\0');
        if (trh.name_length > 0) {
            in.read(&name[0], trh.name_length);
            if (!in) throw std::runtime_error("Failed to read tensor name");
        }
        const auto dtype = static_cast<DType>(trh.dtype);
        if (trh.dtype > static_cast<uint32_t>(DType::BFloat16) || dtype == DType::Invalid)
            throw std::runtime_error("Unsupported dtype in checkpoint for: " + name);
        Tensor tensor(dtype, shape, name, Device::cpu());
        if (tensor.numel() != trh.numel) throw std::runtime_error("Tensor numel mismatch while loading: " + name);
        if (tensor.size() != trh.nbytes) throw std::runtime_error("Tensor byte size mismatch while loading: " + name);
        in.read(static_cast<char*>(tensor.data_ptr()), static_cast<std::streamsize>(trh.nbytes));
        if (!in) throw std::runtime_error("Failed to read tensor data for: " + name);
        ckpt.m_state_dict[name] = tensor;
    }
    return ckpt;
}

void Checkpoint::load_into(Module& m, const StateDict& state, bool strict) {
    StateDict own = m.state_dict();
    if (strict)
        for (const auto& [name, t] : state)
            if (!own.count(name)) throw std::runtime_error("load_into: unexpected tensor in state dict: " + name);
    for (auto& [name, dst] : own) {
        auto it = state.find(name);
        if (it == state.end()) {
            if (strict) throw std::runtime_error("load_into: missing tensor in state dict: " + name);
            continue;
        }
        const Tensor& src = it->second;
        if (src.shape() != dst.shape()) throw std::runtime_error("load_into: shape mismatch for " + name);
        if (src.dtype() != dst.dtype()) throw std::runtime_error("load_into: dtype mismatch for " + name);
        if (!dst.is_contiguous()) throw std::runtime_error("load_into: destination is not contiguous: " + name);
        Tensor h = src.device().is_cpu() ? src : src.to(Device::cpu());
        if (!h.is_contiguous()) h = h.contiguous();
        if (dst.device().is_cpu()) {
            std::memcpy(dst.data_ptr(), h.data_ptr(), h.size());
        } else {
            detail::DeviceGuard g(dst.device().index);
            hipStream_t s = detail::stream_for(dst.device().index);
            detail::hip_check(hipMemcpyAsync(dst.data_ptr(), h.data_ptr(), h.size(), hipMemcpyHostToDevice, s),
                              "hipMemcpyAsync H2D");
            detail::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
        }
    }
}

}  // namespace Inferno
