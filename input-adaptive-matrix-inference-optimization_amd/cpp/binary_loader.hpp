// binary_loader.hpp - reader of the bucket-layout weight files written by
// save_bucketmul_binary (preprocess_layer_fixed_gpu.py:245-282): raw
// little-endian fp16 "<name>_buckets.bin" (1, R, C), "_stats.bin" (1, R, 4),
// "_probes.bin" (1, in) and "_meta.txt".  Same structure and checks as the
// reference reader (binary_loader.hpp:14-201); host vectors only, the caller
// uploads.  Also the raw .npy skip-header reader of
// transformer_layer.hpp:25-52 / model.hpp:54-81, with a header check, and
// the reference's fp16 debugging helpers (binary_loader.hpp:203-241).
#ifndef IAM_BINARY_LOADER_HPP
#define IAM_BINARY_LOADER_HPP

#include <cmath>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "gpu.hpp"

struct Shape3D {
    size_t dim0 = 0, dim1 = 0, dim2 = 0;
    size_t total() const { return dim0 * dim1 * dim2; }
    size_t bytes() const { return total() * sizeof(uint16_t); }
};

struct Shape2D {
    size_t dim0 = 0, dim1 = 0;
    size_t total() const { return dim0 * dim1; }
    size_t bytes() const { return total() * sizeof(uint16_t); }
};

// binary_loader.hpp:30-37
struct WeightMetadata {
    Shape3D buckets_shape;
    Shape3D stats_shape;
    Shape2D probes_shape;
    size_t in_dim = 0;
    size_t out_dim = 0;
    size_t bsize = 0;
};

// binary_loader.hpp:40-51: the loader fills the host copies only; the device
// handles stay null (the caller uploads), as in the reference
struct BucketizedWeight {
    void* buckets = nullptr;
    void* stats = nullptr;
    void* probes = nullptr;
    WeightMetadata meta;
    std::vector<uint16_t> buckets_host;
    std::vector<uint16_t> stats_host;
    std::vector<uint16_t> probes_host;
};

class BinaryWeightLoader {
public:
    // binary_loader.hpp:137-139: the device is not used by the reader (it
    // returns host vectors); it is kept for the reference's call sites
    BinaryWeightLoader(Gpu* gpu, const std::string& base_path) : gpu(gpu), base_path(base_path) {}
    explicit BinaryWeightLoader(const std::string& base_path) : base_path(base_path) {}

    // binary_loader.hpp:59-102
    static WeightMetadata readMetadata(const std::string& meta_file)
    {
        std::ifstream file(meta_file);
        if (!file) throw std::runtime_error("weight metadata not readable (" + meta_file + ")");
        WeightMetadata meta;
        std::string line;
        while (std::getline(file, line)) {
            if (line.empty() || line[0] == '#') continue;
            std::istringstream iss(line);
            std::string key;
            iss >> key;
            if (key == "buckets_shape:") iss >> meta.buckets_shape.dim0 >> meta.buckets_shape.dim1 >> meta.buckets_shape.dim2;
            else if (key == "stats_shape:") iss >> meta.stats_shape.dim0 >> meta.stats_shape.dim1 >> meta.stats_shape.dim2;
            else if (key == "probes_shape:") iss >> meta.probes_shape.dim0 >> meta.probes_shape.dim1;
            else if (key == "in_dim:") iss >> meta.in_dim;
            else if (key == "out_dim:") iss >> meta.out_dim;
            else if (key == "bsize:") iss >> meta.bsize;
        }
        if (meta.in_dim == 0 || meta.out_dim == 0) throw std::runtime_error("weight metadata lacks in_dim or out_dim");
        // the shapes must describe the layout of preprocess_layer_fixed_gpu.py:226-228
        const size_t bs = meta.bsize ? meta.bsize : 16;
        if (meta.buckets_shape.dim0 < 1 || meta.buckets_shape.dim1 != meta.in_dim * bs ||
            meta.buckets_shape.dim2 * bs != meta.out_dim || meta.stats_shape.dim0 != meta.buckets_shape.dim0 ||
            meta.stats_shape.dim1 != meta.buckets_shape.dim1 || meta.stats_shape.dim2 != 4)
            throw std::runtime_error("weight metadata shapes do not describe a bucket layout (" + meta_file + ")");
        return meta;
    }

    // binary_loader.hpp:105-134: the file size must match exactly
    static std::vector<uint16_t> readBinary(const std::string& bin_file, size_t expected_elements)
    {
        std::ifstream file(bin_file, std::ios::binary);
        if (!file) throw std::runtime_error("weight array not readable (" + bin_file + ")");
        file.seekg(0, std::ios::end);
        const size_t file_size = (size_t)file.tellg();
        file.seekg(0, std::ios::beg);
        const size_t expected_size = expected_elements * sizeof(uint16_t);
        if (file_size != expected_size) {
            std::ostringstream oss;
            oss << bin_file << ": " << file_size << " bytes on disk, the metadata asks for " << expected_size;
            throw std::runtime_error(oss.str());
        }
        std::vector<uint16_t> data(expected_elements);
        file.read(reinterpret_cast<char*>(data.data()), (std::streamsize)file_size);
        if (!file) throw std::runtime_error("short read of weight array (" + bin_file + ")");
        return data;
    }

    // binary_loader.hpp:141-193
    BucketizedWeight load(const std::string& weight_name) const
    {
        const std::string prefix = base_path + "/" + weight_name;
        BucketizedWeight w;
        w.meta = readMetadata(prefix + "_meta.txt");
        w.buckets_host = readBinary(prefix + "_buckets.bin", w.meta.buckets_shape.total());
        w.stats_host = readBinary(prefix + "_stats.bin", w.meta.stats_shape.total());
        w.probes_host = readBinary(prefix + "_probes.bin", w.meta.probes_shape.total());
        return w;
    }

    // binary_loader.hpp:196-200
    BucketizedWeight loadLayerWeight(int layer, const std::string& weight_type) const
    {
        return load("layer" + std::to_string(layer) + "_" + weight_type + "_proj_bucketmul_fp16");
    }

    // .npy of fp16 values (transformer_layer.hpp:25-52 skips the header; the
    // header is parsed here so a wrong dtype or a truncated file is an error)
    static std::vector<uint16_t> loadNpyF16(const std::string& path, std::vector<size_t>* shape = nullptr)
    {
        std::ifstream f(path, std::ios::binary);
        if (!f) throw std::runtime_error("npy file not readable (" + path + ")");
        char magic[6];
        f.read(magic, 6);
        if (!f || std::memcmp(magic, "\x93NUMPY", 6) != 0) throw std::runtime_error("no npy magic at the start of " + path);
        uint8_t major = 0, minor = 0;
        f.read(reinterpret_cast<char*>(&major), 1);
        f.read(reinterpret_cast<char*>(&minor), 1);
        uint32_t hlen = 0;
        if (major == 1) {
            uint16_t h16 = 0;
            f.read(reinterpret_cast<char*>(&h16), 2);
            hlen = h16;
        } else {
            f.read(reinterpret_cast<char*>(&hlen), 4);
        }
        std::string header(hlen, '\0');
        f.read(&header[0], hlen);
        if (!f) throw std::runtime_error("npy header cut short in " + path);
        if (header.find("'<f2'") == std::string::npos && header.find("'float16'") == std::string::npos)
            throw std::runtime_error("npy array is not little-endian fp16: " + path);
        if (header.find("'fortran_order': True") != std::string::npos)
            throw std::runtime_error("npy array is column-major (only row-major is read): " + path);
        std::vector<size_t> shp;
        const size_t l = header.find('('), r = header.find(')');
        if (l != std::string::npos && r != std::string::npos) {
            std::istringstream is(header.substr(l + 1, r - l - 1));
            std::string tok;
            while (std::getline(is, tok, ',')) {
                size_t a = tok.find_first_not_of(" ");
                if (a != std::string::npos) shp.push_back(std::stoull(tok.substr(a)));
            }
        }
        size_t n = 1;
        for (size_t d : shp) n *= d;
        std::vector<uint16_t> data(n);
        f.read(reinterpret_cast<char*>(data.data()), (std::streamsize)(n * 2));
        if (!f) throw std::runtime_error("npy data cut short in " + path);
        if (shape) *shape = shp;
        return data;
    }

private:
    Gpu* gpu = nullptr;
    std::string base_path;
};

// binary_loader.hpp:203-241: an fp16 value from its bits (subnormals, inf and
// NaN included), and the position / value fields of a packed bucket entry
// (value bits & 0xFFF0, position bits & 0xF; preprocess_layer_fixed_gpu.py:40-89)
inline float fp16_to_float(uint16_t h)
{
    const int e = (h >> 10) & 0x1f;
    const int m = h & 0x3ff;
    float mag;
    if (e == 0x1f) mag = m ? NAN : INFINITY;
    else if (e == 0) mag = std::ldexp((float)m, -24);             // zero or subnormal: m * 2^-24
    else mag = std::ldexp((float)(m | 0x400), e - 25);            // 1.m * 2^(e-15)
    return (h & 0x8000) ? -mag : mag;
}

inline int extract_position(uint16_t packed_fp16) { return packed_fp16 & 0xf; }

inline float extract_value(uint16_t packed_fp16) { return fp16_to_float((uint16_t)(packed_fp16 & 0xfff0)); }

#endif
