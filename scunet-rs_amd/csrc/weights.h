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

class Weights {
public:
    // weights.rs:101-185. Returns false and sets *err on any failure.
    bool load(const std::string& path, std::string* err);
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
    bool validate(const std::string& path, std::string* err) const;
    std::map<std::string, Tensor> t_;
    void* map_ = nullptr;
    size_t map_len_ = 0;
};

}  // namespace scunet
