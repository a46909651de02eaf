// checkpoint.h -- state-dict files in the reference's checkpoint format
// (include/inferno/checkpoint/checkpoint.h, src/inferno/checkpoint/checkpoint.cpp):
// an 8-byte "INFERNO" magic, version 0 and the tensor count, then per tensor a
// packed record header (name length, dtype as the raw DType value, ndim, numel,
// nbytes), ndim uint64 dimensions, the name and the raw little-endian element
// bytes, in state-dict (name) order.  Files written here load in the reference
// and vice versa.  Device tensors are copied to the host to be written; loaded
// tensors are host tensors (use load_into to copy them into a module on any
// device).
#pragma once
#include <cstdint>
#include <string>
#include "inferno/modules/module.h"

namespace Inferno {

#pragma pack(push, 1)
struct CheckpointHeader {
    char magic[8];
    uint32_t version;
    uint32_t tensor_count;
};
struct TensorRecordHeader {
    uint32_t name_length;
    uint32_t dtype;
    uint32_t ndim;
    uint64_t numel;
    uint64_t nbytes;
};
// Declared as the reference's header declares it, for callers that name it;
// the files written and read here carry no training metadata.
struct TrainingMetadata {
    uint64_t step;
    uint64_t total_steps;
    uint64_t epoch;
    uint64_t total_epochs;
};
#pragma pack(pop)

class Checkpoint {
public:
    void save(const std::string& path) const;
    // Reads `path` into a new Checkpoint (as the reference's member function does).
    Checkpoint load(const std::string& path);
    void set_state_dict(const StateDict& state);
    const StateDict& state_dict() const;
    // Copies every entry of `state` whose name is in m's state dict into that
    // tensor in place (any device; shapes and dtypes must match).  With strict,
    // a name of m missing from `state`, or an extra name in `state`, throws.
    // No reference counterpart (the reference leaves this to the caller).
    static void load_into(Module& m, const StateDict& state, bool strict = true);

private:
    StateDict tensors_;
};

}  // namespace Inferno
