// The checkpoint: a mmapped safetensors file plus the architecture it describes.
// Mirrors src/weights.rs (jacobsparts/scunet-rs): the same __metadata__ keys, the same
// variant/in_nc cross-check, the same per-tensor shape list, the same derivation of
// each block's (conv, trans) widths from tensor shapes.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace scunet {

struct Tensor {
    std::vector<size_t> shape;
    const float* data = nullptr;   // into the mapping
    size_t numel = 0;
};

// The architecture of a checkpoint the caller has already loaded: Weights::arch.name(),
// in_nc, dim, head_dim, window and config of weights.rs:83-97.
struct ArchInfo {
    std::string variant;
    long in_nc = 0, dim = 0, head_dim = 0, window = 0;
    long config[7] = {0, 0, 0, 0, 0, 0, 0};
};

// A borrowed tensor: the caller's float32 data for `name` (null when it has no such tensor),
// with its shape written to shape[0..*ndim) (at most MAX_NDIM extents).
constexpr size_t MAX_NDIM = 8;
using TensorLookup = const float* (*)(void* user, const char* name, size_t* shape, size_t* ndim);

class Weights {
public:
    // weights.rs:101-185. Returns false and sets *err on any failure.
    bool load(const std::string& path, std::string* err);
    // The same checks on tensors the caller holds (the weights.rs `Weights` that
    // Cuda::new borrows, cuda.rs:192): every tensor the network uses is asked for by name
    // through `lookup`; the data is borrowed, so it is valid only until forget_data().
    bool borrow(const ArchInfo& arch, TensorLookup lookup, void* user, std::string* err);
    // Drops the host data pointers (after the upload, when the data was borrowed).
    void forget_data();
    ~Weights();

    int in_nc = 0, dim = 0, head_dim = 0, window = 0;
    int config[7] = {0, 0, 0, 0, 0, 0, 0};
    std::string variant;
    uint64_t bytes = 0;

    bool has(const std::string& name) const { return t_.count(name) != 0; }
    const Tensor& t(const std::string& name) const;   // name validated at load
    // weights.rs:196-200.
    std::pair<int, int> block_dims(const std::string& prefix) const;
    // weights.rs:298-302: (2(conv+trans), conv+trans) of the stage's first block.
    std::pair<int, int> up_conv_channels(const std::string& name) const;
    // weights.rs:284-294.
    std::pair<int, int> down_conv_channels(const std::string& name) const;
    const std::map<std::string, Tensor>& all() const { return t_; }

private:
    bool check_arch(const std::string& label, std::string* err) const;
    // Checks every shape and keeps only the tensors it checked.
    bool validate(const std::string& label, std::string* err);
    std::vector<std::string> expected_names() const;
    std::map<std::string, Tensor> t_;
    void* map_ = nullptr;
    size_t map_len_ = 0;
};

}  // namespace scunet
