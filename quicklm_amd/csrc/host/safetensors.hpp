// Read-only safetensors access over mmap (reference: SafetensorsLoader,
// src/io/safetensors.hpp:40-81, safetensors.cpp:82-246). Tensors are exposed
// as raw views into the mapping; dtype conversion and int8 quantisation
// happen on the device after upload (see model.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace qlm {

struct TensorView {
    std::string dtype;            // "F32", "BF16", ...
    std::vector<int64_t> shape;
    const uint8_t* data = nullptr;
    size_t nbytes = 0;

    int64_t numel() const {
        int64_t n = 1;
        for (auto d : shape) n *= d;
        return n;
    }
};

// Bytes per element of a safetensors dtype string; 0 for a dtype this
// loader does not know (such tensors are only reachable by name, and every
// consumer rejects dtypes other than F32 and BF16).
size_t dtype_size(const std::string& dtype);

// Every tensor's byte range is checked at open: inside the file, end >=
// begin, and (for a known dtype) exactly prod(shape) x dtype_size bytes.
class SafetensorsFile {
   public:
    explicit SafetensorsFile(const std::string& path);
    ~SafetensorsFile();
    SafetensorsFile(const SafetensorsFile&) = delete;
    SafetensorsFile& operator=(const SafetensorsFile&) = delete;

    bool has(const std::string& name) const { return infos_.count(name) != 0; }
    TensorView get(const std::string& name) const;
    std::vector<std::string> names() const;
    const std::string& path() const { return path_; }

   private:
    struct Info {
        std::string dtype;
        std::vector<int64_t> shape;
        size_t begin = 0, end = 0;
    };
    std::string path_;
    int fd_ = -1;
    size_t size_ = 0;
    uint8_t* map_ = nullptr;
    size_t data_start_ = 0;
    std::map<std::string, Info> infos_;
};

// All *.safetensors files of a model directory, looked up by tensor name
// (reference: ModelWeights, src/model/weights.cpp:6-70). Lookups fall back
// to the "model.language_model." prefix used by multimodal Qwen3.5
// checkpoints (qwen3_5.cpp:142-149).
class WeightStore {
   public:
    explicit WeightStore(const std::string& dir);
    bool has(const std::string& name) const;
    TensorView get(const std::string& name) const;

   private:
    const SafetensorsFile* find(const std::string& name, std::string& resolved) const;
    std::vector<std::unique_ptr<SafetensorsFile>> files_;
};

}  // namespace qlm
