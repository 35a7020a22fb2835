// model_files.hpp - the on-disk model package read by the decode library.
//
// Format (as written by the reference packer and read by
// customlib/runtime/custom_model.cpp:185-262, 423-553):
//   xqwen35_manifest.json          hyper-parameters, scanned key by key
//   embeddings_bf16.bin            [vocab][hidden] bf16
//   norm_weight.f32, layers_<i>_*.f32   fp32 vectors
//   *.xq4                          52-byte header <8s magic "XQW4A16\0", u32 version,
//                                  rows, cols, group, bits, u64 packed_bytes,
//                                  scales_count, zeros_count> then packed nibbles,
//                                  fp32 scales, fp32 zeros
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace xqh {

struct HostMatrix {
    int rows = 0, cols = 0, group = 64;
    bool affine = false;  // XQ4 version 2: w = q*s + z; version 1: w = (q - z)*s
    std::vector<uint8_t> packed;
    std::vector<float> scales, zeros;
};

std::string read_text(const std::string& path);
bool file_exists(const std::string& path);

// Manifest scan with the reference's semantics (custom_model.cpp:38-87): the
// first occurrence of "key", the first number after its colon.
int manifest_int(const std::string& json, const std::string& key, int fallback);
float manifest_float(const std::string& json, const std::string& key, float fallback);
std::string manifest_string(const std::string& json, const std::string& key, const std::string& fallback);

bool read_f32_file(const std::string& path, int count, std::vector<float>* out, std::string* error);
bool read_xq4_file(const std::string& path, HostMatrix* m, std::string* error);

// Row-wise concatenation of matrices with equal cols/group/version.
bool concat_rows(const std::vector<const HostMatrix*>& parts, HostMatrix* out, std::string* error);
// Interleave the rows of two equal-shape matrices: a0, b0, a1, b1, ...
bool interleave_rows(const HostMatrix& a, const HostMatrix& b, HostMatrix* out, std::string* error);

}  // namespace xqh
