// The reference's `.snl` weight file (src/weights.rs:1-121, written by src/convert.rs:316-400):
//
//   bytes 0-3   "SNLQ"
//   bytes 4-7   version (u32 LE, 1)
//   bytes 8-15  header length L (u64 LE)
//   bytes 16..  JSON header {model_name, quant, config: ModelConfig, tensors: {name: {dtype,
//               shape, offset, scales_offset}}}
//   then each tensor at a 256-byte aligned absolute offset: quants (Q8_0: int8 [rows, cols];
//   Q4_0: [rows, cols/2], nibble i of LE word w = element 8w + i; f32: the values), and for the
//   quantised types one f32 scale per 32-element block at scales_offset.
//
// The reader maps the file and parses the header; the writer lays tensors out in the order given,
// each region aligned to 256 bytes, with the data starting past the header plus 4 KiB of slack,
// as the converter does.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <map>
#include <string>
#include <vector>

#include "../../include/snl.h"

namespace snl {

enum FileDType { FD_F32 = 0, FD_Q8_0 = 1, FD_Q4_0 = 2 };

struct FileTensor {
    int dtype = FD_F32;
    std::vector<int64_t> shape;
    uint64_t offset = 0, scales_offset = 0;
    int64_t rows() const { return shape.size() == 1 ? 1 : shape[0]; }
    int64_t cols() const { return shape.empty() ? 0 : shape.back(); }
    // (quant bytes, scale bytes) of the tensor (DType::sizes, src/weights.rs:47-55)
    uint64_t quant_bytes() const;
    uint64_t scale_bytes() const;
};

struct FileConfig {
    snl_config cfg{};   // has_mtp is left 0: the MTP head is a separate file
    int64_t max_position = 0;
};

class SnlFile {
public:
    ~SnlFile();
    // Map and check `path`; false with a message in *err.
    bool open(const char* path, std::string* err);
    bool config(FileConfig* out, std::string* err) const;
    const FileTensor* find(const std::string& name) const;
    // the tensor's quants (or f32 values) and scales inside the mapping
    const uint8_t* quants(const FileTensor& t) const { return base_ + t.offset; }
    const uint8_t* scales(const FileTensor& t) const { return base_ + t.scales_offset; }
    const std::string& model_name() const { return model_name_; }
    const std::string& quant() const { return quant_; }

private:
    uint8_t* base_ = nullptr;
    size_t size_ = 0;
    std::string model_name_, quant_, header_json_;
    std::map<std::string, FileTensor> tensors_;
};

struct WriteTensor {
    std::string name;
    int dtype = FD_F32;
    std::vector<int64_t> shape;
};

// Writes the header and returns each tensor's FileTensor (absolute offsets) in `placed`; the caller
// then fills the regions with write_region.  The file is created at path + ".partial" and renamed
// by finish().
class SnlWriter {
public:
    ~SnlWriter();
    bool begin(const char* path, const std::string& model_name, const std::string& quant, const FileConfig& cfg,
               const std::vector<WriteTensor>& tensors, std::vector<FileTensor>* placed, std::string* err);
    bool write_region(uint64_t offset, const void* data, size_t bytes, std::string* err);
    bool finish(std::string* err);

private:
    int fd_ = -1;
    std::string path_, tmp_;
};

}  // namespace snl
