// Tensor-table helpers shared by the decoder and encoder loaders
// (internal/model/compat.go:15-270): name resolution with the HF aliases,
// float loads of any stored type, matrices uploaded quantised or as float.
#pragma once

#include <map>
#include <string>
#include <vector>

#include "wh_internal.h"

namespace wh {

std::string map_tensor_name(const std::string &name);  // compat.go:31-148

struct Table {
    std::map<std::string, const wh_tensor *> byname;
    const wh_tensor *resolve(const std::string &name) const;  // compat.go:15-29
};

uint64_t numel(const wh_tensor *t);
int not_found(const std::string &name);
// gguf File.Tensor(): dequantise any stored type to float32.
int load_f32(const wh_tensor *t, std::vector<float> &out);

// Float vectors gathered on the host, uploaded as one allocation; each slot is
// pointed at its vector's device copy after the upload.
struct VecArena {
    std::vector<float> host;
    std::vector<std::pair<float **, size_t>> fix;  // pointer slot, offset in floats
    int add(const std::vector<float> &v, float **slot);
};

// loadMatWeightAuto (compat.go:247-270): a quantised 2-D tensor of the wanted
// shape is uploaded as is; anything else is dequantised to f32 (transposed when
// stored [cols, rows]).
int load_matrix(const Table &tab, const std::string &name, int rows, int cols, DevMat &m);
// A float vector of at least min_len elements into the arena.
int load_vector(const Table &tab, const std::string &name, VecArena &arena, float **slot, size_t min_len);

}  // namespace wh
