// Device-side tensor carrier (reference: struct Tensor, src/tensor/tensor.hpp:
// 17-121). Same shape/stride conventions (row-major, strides in elements),
// but every data pointer is a DEVICE pointer and sizes are 64-bit. The int8
// weight form keeps the reference's Q8_0 meaning (int8 [N, K] plus fp32
// scales [N, ceil(K/G)]) with the scale group G carried explicitly (32 =
// the reference's INT8_BLOCK_SIZE, or K = one scale per output row).
// A Tensor is a view: ownership lives in DeviceBuffers held by the model.
#pragma once

#include <cstdint>
#include <vector>

namespace qlm {

struct Tensor {
    std::vector<int64_t> shape;
    std::vector<int64_t> strides;

    float* data = nullptr;                 // fp32 activations / parameters
    const int8_t* int8_data = nullptr;     // int8 weight operand
    const float* int8_scales = nullptr;
    int int8_group = 32;
    // The same weight in the matrix-core tile-major layout (qlm_mx_swizzle),
    // which every device matmul reads; null where the model keeps no such
    // copy (K not a multiple of 64). A model holding the tile-major copy keeps
    // no row-major one (int8_data and int8_scales null; with per-row scales
    // the scales stay, as int8_tile_scales).
    const int8_t* int8_tiles = nullptr;
    const float* int8_tile_scales = nullptr;
    // int4 (Q4_0) weights: the int8 fields then hold the unpacked values
    // (same scales; the reference's int4 dot is its int8 dot over them) and
    // this is their int4 tile-major copy (qlm_mx4_swizzle, scales as above),
    // which the one-row GEMV streams at half the bytes.
    const uint8_t* int4_tiles = nullptr;
    // Native (unquantised) weights, the reference's --precision bf16: fp32
    // rows (F32 checkpoint tensors) or bf16 rows (BF16 ones); no int8 form.
    const void* native_data = nullptr;
    bool native_bf16 = false;

    Tensor() = default;
    Tensor(std::vector<int64_t> shp, float* d) : shape(std::move(shp)), data(d) { compute_strides(); }

    static Tensor int8(const int8_t* q, const float* s, int64_t N, int64_t K, int group) {
        Tensor t;
        t.shape = {N, K};
        t.compute_strides();
        t.int8_data = q;
        t.int8_scales = s;
        t.int8_group = group;
        return t;
    }

    // int8 (or int4-unpacked) weights, row-major and/or tile-major
    bool is_int8() const { return int8_data != nullptr || int8_tiles != nullptr; }
    bool is_native() const { return native_data != nullptr; }

    void compute_strides() {
        strides.assign(shape.size(), 1);
        int64_t s = 1;
        for (int i = (int)shape.size() - 1; i >= 0; --i) {
            strides[i] = s;
            s *= shape[i];
        }
    }

    int64_t size() const {
        if (shape.empty()) return 0;
        int64_t n = 1;
        for (auto d : shape) n *= d;
        return n;
    }
    int64_t rows() const { return shape.size() > 1 ? shape[0] : 1; }
    int64_t cols() const { return shape.empty() ? 0 : shape.back(); }
    int64_t row_stride() const { return shape.size() > 1 ? strides[0] : cols(); }
};

}  // namespace qlm
