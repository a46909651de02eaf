// checkpoint.cpp -- Checkpoint (include/inferno/checkpoint/checkpoint.h).
//
// File layout, all integers little-endian and unpadded:
//   offset 0   magic      8 bytes  "INFERNO\0"
//   offset 8   version    u32      0
//   offset 12  count      u32      number of tensor records
//   then `count` records, each
//              name_len   u32
//              dtype      u32      the DType enumerator's value
//              ndim       u32
//              numel      u64      product of the dims
//              nbytes     u64      numel * bytes per element
//              dims       ndim x u64
//              name       name_len bytes (no terminator)
//              data       nbytes of elements, row-major, host byte order
// Records are written in state-dict (name) order.  This is the format of the
// reference's checkpoint files (include/inferno/checkpoint/checkpoint.h:5-26),
// so files move between the two.
//
// save() encodes each record into a byte buffer and streams it to a sibling
// temporary file that replaces `path` only once everything is written, so an
// interrupted save leaves the previous checkpoint intact.  load() knows the
// file's length before it allocates anything, and checks every record against
// it and against itself (dims vs numel, numel vs nbytes, known dtype) with an
// error that names the file, the record and the byte offset.
#include "inferno/checkpoint/checkpoint.h"

#include <cstdio>
#include <cstring>
#include <fstream>
#include <limits>
#include <stdexcept>
#include <type_traits>
#include <vector>

#include "detail.h"

namespace Inferno {

static_assert(sizeof(CheckpointHeader) == 16, "the file header is 16 packed bytes");
static_assert(sizeof(TensorRecordHeader) == 28, "a record header is 28 packed bytes");
static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "fields are stored in host order, which must be little-endian");

namespace {

constexpr char kFileMagic[8] = {'I', 'N', 'F', 'E', 'R', 'N', 'O', '\0'};
constexpr uint32_t kFileVersion = 0;

// Appends fixed-width fields to a byte string.
struct Encoder {
    std::string bytes;
    template <typename T>
    void put(T v) {
        static_assert(std::is_trivially_copyable<T>::value, "plain fields only");
        char raw[sizeof(T)];
        std::memcpy(raw, &v, sizeof(T));
        bytes.append(raw, sizeof(T));
    }
    void put_bytes(const void* p, size_t n) { bytes.append(static_cast<const char*>(p), n); }
};

// Reads fixed-width fields from a stream of known length, tracking the offset
// for error messages.
class Decoder {
public:
    Decoder(std::ifstream& in, const std::string& path, uint64_t length) : in_(in), path_(path), length_(length) {}

    uint64_t offset() const { return offset_; }
    uint64_t remaining() const { return length_ - offset_; }

    [[noreturn]] void fail(const std::string& what) const {
        throw std::runtime_error("checkpoint " + path_ + ": " + what + " (at byte " + std::to_string(offset_) + " of " +
                                 std::to_string(length_) + ")");
    }

    void get_bytes(void* dst, uint64_t n, const std::string& field) {
        if (n > remaining())
            fail("file ends inside " + field + " (" + std::to_string(n) + " bytes needed, " +
                 std::to_string(remaining()) + " left)");
        if (n && !in_.read(static_cast<char*>(dst), static_cast<std::streamsize>(n))) fail("read error in " + field);
        offset_ += n;
    }
    template <typename T>
    T get(const std::string& field) {
        T v{};
        get_bytes(&v, sizeof(T), field);
        return v;
    }

private:
    std::ifstream& in_;
    const std::string& path_;
    uint64_t length_;
    uint64_t offset_ = 0;
};

Tensor host_contiguous(const Tensor& t) {
    Tensor h = t.device().is_cpu() ? t : t.to(Device::cpu());
    return h.is_contiguous() ? h : h.contiguous();
}

bool known_dtype(uint32_t code) {
    return code <= static_cast<uint32_t>(DType::BFloat16) && code != static_cast<uint32_t>(DType::Invalid);
}

}  // namespace

void Checkpoint::save(const std::string& path) const {
    const std::string tmp = path + ".partial";
    std::ofstream out(tmp, std::ios::binary | std::ios::trunc);
    if (!out) throw std::runtime_error("checkpoint " + path + ": cannot create " + tmp + " for writing");
    auto abandon = [&](const std::string& why) {
        out.close();
        std::remove(tmp.c_str());
        throw std::runtime_error("checkpoint " + path + ": " + why + "; the previous file, if any, is unchanged");
    };

    Encoder head;
    head.put_bytes(kFileMagic, sizeof(kFileMagic));
    head.put<uint32_t>(kFileVersion);
    head.put<uint32_t>(static_cast<uint32_t>(tensors_.size()));
    if (!out.write(head.bytes.data(), static_cast<std::streamsize>(head.bytes.size()))) abandon("writing the header failed");

    for (const auto& entry : tensors_) {
        const std::string& name = entry.first;
        const Tensor t = host_contiguous(entry.second);
        Encoder rec;
        rec.put<uint32_t>(static_cast<uint32_t>(name.size()));
        rec.put<uint32_t>(static_cast<uint32_t>(t.dtype()));
        rec.put<uint32_t>(static_cast<uint32_t>(t.ndim()));
        rec.put<uint64_t>(t.numel());
        rec.put<uint64_t>(t.size());
        for (size_t d : t.shape()) rec.put<uint64_t>(d);
        rec.put_bytes(name.data(), name.size());
        if (!out.write(rec.bytes.data(), static_cast<std::streamsize>(rec.bytes.size())) ||
            !out.write(static_cast<const char*>(t.data_ptr()), static_cast<std::streamsize>(t.size())))
            abandon("writing tensor '" + name + "' failed");
    }
    out.flush();
    if (!out) abandon("flushing the file failed");
    out.close();
    if (std::rename(tmp.c_str(), path.c_str()) != 0) {
        std::remove(tmp.c_str());
        throw std::runtime_error("checkpoint " + path + ": cannot move the written file " + tmp + " into place");
    }
}

void Checkpoint::set_state_dict(const StateDict& state) { tensors_ = state; }
const StateDict& Checkpoint::state_dict() const { return tensors_; }

Checkpoint Checkpoint::load(const std::string& path) {
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) throw std::runtime_error("checkpoint " + path + ": cannot open for reading");
    const std::streamoff end = in.tellg();
    in.seekg(0);
    if (end < 0 || !in) throw std::runtime_error("checkpoint " + path + ": cannot determine the file's length");
    Decoder dec(in, path, static_cast<uint64_t>(end));

    char magic[sizeof(kFileMagic)];
    dec.get_bytes(magic, sizeof(magic), "the header");
    if (std::memcmp(magic, kFileMagic, sizeof(kFileMagic)) != 0)
        dec.fail("not an Inferno checkpoint: the first 8 bytes are not the magic \"INFERNO\\0\"");
    const uint32_t version = dec.get<uint32_t>("the header");
    if (version != kFileVersion)
        dec.fail("format version " + std::to_string(version) + " is not supported (this build reads version " +
                 std::to_string(kFileVersion) + ")");
    const uint32_t count = dec.get<uint32_t>("the header");

    Checkpoint result;
    for (uint32_t i = 0; i < count; ++i) {
        const std::string rec = "record " + std::to_string(i) + " of " + std::to_string(count);
        const uint32_t name_len = dec.get<uint32_t>(rec + "'s header");
        const uint32_t code = dec.get<uint32_t>(rec + "'s header");
        const uint32_t ndim = dec.get<uint32_t>(rec + "'s header");
        const uint64_t numel = dec.get<uint64_t>(rec + "'s header");
        const uint64_t nbytes = dec.get<uint64_t>(rec + "'s header");
        if ((uint64_t)ndim * 8 + name_len > dec.remaining()) dec.fail(rec + "'s dims and name run past the end of the file");

        std::vector<size_t> shape(ndim);
        uint64_t product = 1;
        bool overflow = false;
        for (uint32_t d = 0; d < ndim; ++d) {
            const uint64_t dim = dec.get<uint64_t>(rec + "'s dims");
            if (dim && product > std::numeric_limits<uint64_t>::max() / dim) overflow = true;
            product *= dim;
            shape[d] = static_cast<size_t>(dim);
        }
        std::string name(name_len, '\0');
        dec.get_bytes(&name[0], name_len, rec + "'s name");
        const std::string who = rec + " ('" + name + "')";

        if (!known_dtype(code)) dec.fail(who + " has an unknown dtype code " + std::to_string(code));
        const auto dtype = static_cast<DType>(code);
        if (overflow || product != numel)
            dec.fail(who + " declares " + std::to_string(numel) + " elements but its dims hold " +
                     (overflow ? std::string("more than 2^64") : std::to_string(product)));
        if (numel > std::numeric_limits<uint64_t>::max() / dtype_size(dtype) || numel * dtype_size(dtype) != nbytes)
            dec.fail(who + " declares " + std::to_string(nbytes) + " data bytes for " + std::to_string(numel) + " " +
                     dtype_name(dtype) + " elements");
        if (nbytes > dec.remaining()) dec.fail(who + "'s data runs past the end of the file");
        if (result.tensors_.count(name)) dec.fail(who + " repeats a name already read");

        Tensor t(dtype, shape, name, Device::cpu());
        dec.get_bytes(t.data_ptr(), nbytes, who + "'s data");
        result.tensors_.emplace(name, t);
    }
    if (dec.remaining() != 0)
        dec.fail(std::to_string(dec.remaining()) + " bytes follow the last of the " + std::to_string(count) + " records");
    return result;
}

void Checkpoint::load_into(Module& m, const StateDict& state, bool strict) {
    StateDict own = m.state_dict();
    if (strict) {
        for (const auto& entry : state)
            if (!own.count(entry.first))
                throw std::runtime_error("load_into: the state dict has '" + entry.first + "', which the module lacks");
    }
    for (auto& entry : own) {
        const std::string& name = entry.first;
        Tensor& dst = entry.second;
        const auto it = state.find(name);
        if (it == state.end()) {
            if (strict) throw std::runtime_error("load_into: the module's '" + name + "' is missing from the state dict");
            continue;
        }
        const Tensor& src = it->second;
        if (src.shape() != dst.shape()) throw std::runtime_error("load_into: '" + name + "' differs in shape");
        if (src.dtype() != dst.dtype()) throw std::runtime_error("load_into: '" + name + "' differs in dtype");
        if (!dst.is_contiguous()) throw std::runtime_error("load_into: the module's '" + name + "' is not contiguous");
        const Tensor h = host_contiguous(src);
        if (dst.device().is_cpu()) {
            std::memcpy(dst.data_ptr(), h.data_ptr(), h.size());
            continue;
        }
        detail::DeviceGuard guard(dst.device().index);
        hipStream_t s = detail::stream_for(dst.device().index);
        detail::hip_check(hipMemcpyAsync(dst.data_ptr(), h.data_ptr(), h.size(), hipMemcpyHostToDevice, s),
                          "hipMemcpyAsync H2D");
        detail::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    }
}

}  // namespace Inferno
