// model_files.cpp - readers for the model package (see model_files.hpp).
#include "model_files.hpp"

#include <cctype>
#include <cstring>
#include <fstream>
#include <sstream>

namespace xqh {

std::string read_text(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return std::string();
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

bool file_exists(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return f.good();
}

namespace {
bool number_start(const std::string& js, const std::string& key, size_t* at) {
    const std::string pat = "\"" + key + "\"";
    const size_t k = js.find(pat);
    if (k == std::string::npos) return false;
    const size_t colon = js.find(':', k + pat.size());
    if (colon == std::string::npos) return false;
    const size_t s = js.find_first_of("-0123456789", colon + 1);
    if (s == std::string::npos) return false;
    *at = s;
    return true;
}
}  // namespace

int manifest_int(const std::string& js, const std::string& key, int fallback) {
    size_t s;
    if (!number_start(js, key, &s)) return fallback;
    size_t e = s + 1;
    while (e < js.size() && js[e] >= '0' && js[e] <= '9') ++e;
    try {
        return std::stoi(js.substr(s, e - s));
    } catch (...) {
        return fallback;
    }
}

float manifest_float(const std::string& js, const std::string& key, float fallback) {
    size_t s;
    if (!number_start(js, key, &s)) return fallback;
    size_t e = s + 1;
    while (e < js.size() && (std::isdigit(static_cast<unsigned char>(js[e])) || js[e] == '.' || js[e] == 'e' ||
                             js[e] == 'E' || js[e] == '-' || js[e] == '+'))
        ++e;
    try {
        return std::stof(js.substr(s, e - s));
    } catch (...) {
        return fallback;
    }
}

std::string manifest_string(const std::string& js, const std::string& key, const std::string& fallback) {
    const std::string pat = "\"" + key + "\"";
    const size_t k = js.find(pat);
    if (k == std::string::npos) return fallback;
    const size_t colon = js.find(':', k + pat.size());
    if (colon == std::string::npos) return fallback;
    const size_t q0 = js.find('"', colon + 1);
    if (q0 == std::string::npos) return fallback;
    const size_t q1 = js.find('"', q0 + 1);
    if (q1 == std::string::npos) return fallback;
    return js.substr(q0 + 1, q1 - q0 - 1);
}

bool read_f32_file(const std::string& path, int count, std::vector<float>* out, std::string* error) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        *error = "missing vector file: " + path;
        return false;
    }
    out->assign(static_cast<size_t>(count), 0.0f);
    f.read(reinterpret_cast<char*>(out->data()), static_cast<std::streamsize>(count) * 4);
    if (f.gcount() != static_cast<std::streamsize>(count) * 4) {
        *error = "short vector file: " + path;
        return false;
    }
    return true;
}

bool read_xq4_file(const std::string& path, HostMatrix* m, std::string* error) {
    std::ifstream f(path, std::ios::binary);
    if (!f) {
        *error = "missing xq4 matrix: " + path;
        return false;
    }
    char magic[8] = {};
    f.read(magic, 8);
    if (std::memcmp(magic, "XQW4A16", 7) != 0) {
        *error = "bad xq4 magic: " + path;
        return false;
    }
    uint32_t hdr[5] = {};
    uint64_t counts[3] = {};
    f.read(reinterpret_cast<char*>(hdr), sizeof(hdr));
    f.read(reinterpret_cast<char*>(counts), sizeof(counts));
    const uint32_t version = hdr[0], rows = hdr[1], cols = hdr[2], group = hdr[3], bits = hdr[4];
    if (!f || (version != 1 && version != 2) || bits != 4 || rows == 0 || cols == 0 || group == 0 ||
        counts[1] != counts[2]) {
        *error = "invalid xq4 header: " + path;
        return false;
    }
    const uint64_t need_packed = (static_cast<uint64_t>(cols) + 1) / 2 * rows;
    const uint64_t need_meta = static_cast<uint64_t>((cols + group - 1) / group) * rows;
    if (counts[0] < need_packed || counts[1] < need_meta) {
        *error = "invalid xq4 header (payload smaller than rows x cols): " + path;
        return false;
    }
    m->rows = static_cast<int>(rows);
    m->cols = static_cast<int>(cols);
    m->group = static_cast<int>(group);
    m->affine = version == 2;
    m->packed.assign(static_cast<size_t>(counts[0]), 0);
    m->scales.assign(static_cast<size_t>(counts[1]), 1.0f);
    m->zeros.assign(static_cast<size_t>(counts[2]), 0.0f);
    f.read(reinterpret_cast<char*>(m->packed.data()), static_cast<std::streamsize>(m->packed.size()));
    f.read(reinterpret_cast<char*>(m->scales.data()), static_cast<std::streamsize>(m->scales.size() * 4));
    f.read(reinterpret_cast<char*>(m->zeros.data()), static_cast<std::streamsize>(m->zeros.size() * 4));
    if (!f) {
        *error = "short xq4 payload: " + path;
        return false;
    }
    return true;
}

bool concat_rows(const std::vector<const HostMatrix*>& parts, HostMatrix* out, std::string* error) {
    if (parts.empty()) {
        *error = "concat_rows: no parts";
        return false;
    }
    const HostMatrix& p0 = *parts[0];
    *out = HostMatrix();
    out->cols = p0.cols;
    out->group = p0.group;
    out->affine = p0.affine;
    const size_t rb = (static_cast<size_t>(p0.cols) + 1) / 2;
    const size_t gpr = static_cast<size_t>((p0.cols + p0.group - 1) / p0.group);
    for (const HostMatrix* p : parts) {
        if (p->cols != p0.cols || p->group != p0.group || p->affine != p0.affine) {
            *error = "fused projections disagree in cols/group/version";
            return false;
        }
        out->rows += p->rows;
        out->packed.insert(out->packed.end(), p->packed.begin(), p->packed.begin() + rb * p->rows);
        out->scales.insert(out->scales.end(), p->scales.begin(), p->scales.begin() + gpr * p->rows);
        out->zeros.insert(out->zeros.end(), p->zeros.begin(), p->zeros.begin() + gpr * p->rows);
    }
    return true;
}

bool interleave_rows(const HostMatrix& a, const HostMatrix& b, HostMatrix* out, std::string* error) {
    if (a.rows != b.rows || a.cols != b.cols || a.group != b.group || a.affine != b.affine) {
        *error = "gate/up projections disagree in shape/group/version";
        return false;
    }
    *out = HostMatrix();
    out->rows = 2 * a.rows;
    out->cols = a.cols;
    out->group = a.group;
    out->affine = a.affine;
    const size_t rb = (static_cast<size_t>(a.cols) + 1) / 2;
    const size_t gpr = static_cast<size_t>((a.cols + a.group - 1) / a.group);
    out->packed.resize(rb * out->rows);
    out->scales.resize(gpr * out->rows);
    out->zeros.resize(gpr * out->rows);
    for (int r = 0; r < a.rows; ++r) {
        std::memcpy(&out->packed[rb * (2 * r)], &a.packed[rb * r], rb);
        std::memcpy(&out->packed[rb * (2 * r + 1)], &b.packed[rb * r], rb);
        std::memcpy(&out->scales[gpr * (2 * r)], &a.scales[gpr * r], gpr * 4);
        std::memcpy(&out->scales[gpr * (2 * r + 1)], &b.scales[gpr * r], gpr * 4);
        std::memcpy(&out->zeros[gpr * (2 * r)], &a.zeros[gpr * r], gpr * 4);
        std::memcpy(&out->zeros[gpr * (2 * r + 1)], &b.zeros[gpr * r], gpr * 4);
    }
    return true;
}

}  // namespace xqh
