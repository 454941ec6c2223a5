// Test harness: opens a .safetensors file with the engine's loader
// (quicklm_amd/csrc/host/safetensors.cpp) on the CPU and reports whether the
// header was accepted. Built by tests/test_safetensors.py with g++.
#include <cstring>
#include <exception>

#include "safetensors.hpp"

extern "C" int st_open(const char* path, char* err, int n) {
    try {
        qlm::SafetensorsFile f(path);
        return (int)f.names().size();
    } catch (const std::exception& e) {
        std::strncpy(err, e.what(), (size_t)n - 1);
        err[n - 1] = 0;
        return -1;
    }
}
