#include "safetensors.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <dirent.h>
#include <stdexcept>

#include "json.hpp"

namespace qlm {

size_t dtype_size(const std::string& dtype) {
    if (dtype == "F64" || dtype == "I64" || dtype == "U64") return 8;
    if (dtype == "F32" || dtype == "I32" || dtype == "U32") return 4;
    if (dtype == "BF16" || dtype == "F16" || dtype == "I16" || dtype == "U16") return 2;
    if (dtype == "I8" || dtype == "U8" || dtype == "BOOL" || dtype == "F8_E4M3" ||
        dtype == "F8_E5M2")
        return 1;
    return 0;
}

SafetensorsFile::SafetensorsFile(const std::string& path) : path_(path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw std::runtime_error("safetensors: cannot open " + path);
    struct stat st;
    if (fstat(fd_, &st) != 0) throw std::runtime_error("safetensors: cannot stat " + path);
    size_ = (size_t)st.st_size;
    if (size_ < 8) throw std::runtime_error("safetensors: truncated file " + path);
    void* m = mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd_, 0);
    if (m == MAP_FAILED) throw std::runtime_error("safetensors: mmap failed " + path);
    map_ = static_cast<uint8_t*>(m);
    uint64_t hlen = 0;
    std::memcpy(&hlen, map_, 8);
    if (hlen > size_ - 8) throw std::runtime_error("safetensors: header overruns file " + path);
    data_start_ = 8 + (size_t)hlen;
    Json root = Json::parse(std::string_view(reinterpret_cast<const char*>(map_) + 8, (size_t)hlen));
    if (!root.is_object()) throw std::runtime_error("safetensors: header is not an object");
    for (const auto& kv : root.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& t = kv.second;
        Info info;
        info.dtype = t.at("dtype").string();
        // element count, with every dimension checked: a negative or
        // non-integral dimension, or a product past 2^62, is a bad header
        uint64_t numel = 1;
        for (const auto& d : t.at("shape").arr) {
            const double v = d.number();
            if (!(v >= 0.0) || v != (double)(int64_t)v || v > (double)(1ull << 62))
                throw std::runtime_error("safetensors: bad shape for " + kv.first);
            info.shape.push_back((int64_t)v);
            if (v != 0.0 && numel > (1ull << 62) / (uint64_t)v)
                throw std::runtime_error("safetensors: shape too large for " + kv.first);
            numel *= (uint64_t)v;
        }
        const auto& off = t.at("data_offsets").arr;
        if (off.size() != 2) throw std::runtime_error("safetensors: bad data_offsets for " + kv.first);
        const double b0 = off[0].number(), b1 = off[1].number();
        if (!(b0 >= 0.0) || !(b1 >= 0.0) || b0 > (double)size_ || b1 > (double)size_)
            throw std::runtime_error("safetensors: tensor '" + kv.first + "' is out of file bounds");
        info.begin = (size_t)b0;
        info.end = (size_t)b1;
        if (info.end < info.begin || data_start_ + info.end > size_)
            throw std::runtime_error("safetensors: tensor '" + kv.first + "' is out of file bounds");
        // the byte range must hold exactly shape x element size, so every
        // consumer may size its reads and device copies by either one
        const size_t esize = dtype_size(info.dtype);
        if (esize && (uint64_t)(info.end - info.begin) != numel * esize)
            throw std::runtime_error("safetensors: tensor '" + kv.first + "' holds " +
                                     std::to_string(info.end - info.begin) + " bytes, its " +
                                     info.dtype + " shape needs " + std::to_string(numel * esize));
        infos_[kv.first] = std::move(info);
    }
}

SafetensorsFile::~SafetensorsFile() {
    if (map_) munmap(map_, size_);
    if (fd_ >= 0) ::close(fd_);
}

TensorView SafetensorsFile::get(const std::string& name) const {
    auto it = infos_.find(name);
    if (it == infos_.end()) throw std::runtime_error("safetensors: no tensor " + name);
    TensorView v;
    v.dtype = it->second.dtype;
    v.shape = it->second.shape;
    v.data = map_ + data_start_ + it->second.begin;
    v.nbytes = it->second.end - it->second.begin;
    return v;
}

std::vector<std::string> SafetensorsFile::names() const {
    std::vector<std::string> out;
    for (const auto& kv : infos_) out.push_back(kv.first);
    return out;
}

WeightStore::WeightStore(const std::string& dir) {
    DIR* d = opendir(dir.c_str());
    if (!d) throw std::runtime_error("weights: cannot open directory " + dir);
    std::vector<std::string> paths;
    while (dirent* e = readdir(d)) {
        std::string n = e->d_name;
        if (n.size() > 12 && n.substr(n.size() - 12) == ".safetensors") paths.push_back(dir + "/" + n);
    }
    closedir(d);
    std::sort(paths.begin(), paths.end());
    if (paths.empty()) throw std::runtime_error("weights: no .safetensors files in " + dir);
    for (const auto& p : paths) files_.push_back(std::make_unique<SafetensorsFile>(p));
}

const SafetensorsFile* WeightStore::find(const std::string& name, std::string& resolved) const {
    for (const auto& f : files_)
        if (f->has(name)) {
            resolved = name;
            return f.get();
        }
    if (name.rfind("model.", 0) == 0) {
        std::string alt = "model.language_model." + name.substr(6);
        for (const auto& f : files_)
            if (f->has(alt)) {
                resolved = alt;
                return f.get();
            }
    }
    return nullptr;
}

bool WeightStore::has(const std::string& name) const {
    std::string r;
    return find(name, r) != nullptr;
}

TensorView WeightStore::get(const std::string& name) const {
    std::string r;
    const SafetensorsFile* f = find(name, r);
    if (!f) throw std::runtime_error("Tensor not found in any safetensors files: " + name);
    return f->get(r);
}

}  // namespace qlm
