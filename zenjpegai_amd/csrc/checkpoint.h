// Weight readers (host only): PyTorch `.pth` checkpoints (an uncompressed ZIP holding a pickled
// state dict, src/weights/mod.rs:1-11) and the packed `ZJM1` checkpoints / `ZJB1` / `ZJB2`
// bundles (src/weights/packed.rs:1-42). The pickle runs through a data-only interpreter: no
// callable is ever invoked, so parsing a checkpoint cannot execute code.
#pragma once

#include <stdint.h>

#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "error.h"

namespace zjai {

// Element types by their `ZJM1` codes (src/weights/packed.rs:62-90).
enum CkDType : int { CK_F64 = 0, CK_F32, CK_F16, CK_I64, CK_I32, CK_I16, CK_I8, CK_U8, CK_BOOL, CK_NDTYPES };
size_t ck_dtype_size(int dtype);

// f32 -> f16 bits, round to nearest even (src/weights/f16.rs:12-53), and the exact upcast
// (src/weights/f16.rs:56-67).
uint16_t f32_to_f16_bits(float v);
float f16_bits_to_f32(uint16_t h);

// A tensor as the file describes it: a strided view (in elements) into a storage. For a `.pth`
// checkpoint the storage is the archive member `<prefix>data/<storage>`; for `ZJM1` it is the
// file itself and every tensor is contiguous.
struct CkTensor {
    std::string name;
    std::string storage;
    int dtype = CK_F32;
    uint64_t offset = 0;
    std::vector<uint64_t> shape, stride;
    uint64_t numel() const;
};

class Checkpoint {
public:
    // `Checkpoint::parse` (src/weights/mod.rs:135-187): a `ZJM1` file (by its magic) or a
    // `.pth` ZIP. The bytes are copied.
    static std::unique_ptr<Checkpoint> parse(const uint8_t* data, size_t len);

    bool packed() const { return packed_; }
    const std::vector<CkTensor>& tensors() const { return tensors_; }
    const std::vector<std::pair<std::string, int64_t>>& ints() const { return ints_; }
    const std::vector<std::pair<std::string, std::vector<double>>>& lists() const { return lists_; }
    const CkTensor* find(const std::string& name) const;
    // Contiguous little-endian row-major bytes of a tensor (strided views gathered),
    // `Checkpoint::bytes` (src/weights/mod.rs:235-328).
    std::vector<uint8_t> bytes(const CkTensor& t) const;
    // An f32 tensor, or an f16 one upcast exactly (`Checkpoint::f32`, src/weights/mod.rs:342-378).
    std::vector<float> f32(const CkTensor& t) const;

private:
    std::vector<uint8_t> file_;
    bool packed_ = false;
    std::string prefix_;
    std::vector<std::pair<std::string, std::pair<size_t, size_t>>> members_;  // sorted by name
    std::vector<CkTensor> tensors_;
    std::vector<std::pair<std::string, int64_t>> ints_;
    std::vector<std::pair<std::string, std::vector<double>>> lists_;
    std::pair<const uint8_t*, size_t> storage(const CkTensor& t) const;
    void parse_zjm();
    void parse_pth();
};

// `write_zjm` / `write_zjm_f16` (src/weights/packed.rs:166-225): the named tensors and every
// integer entry of a checkpoint as a `ZJM1` file; with `f16`, f32 tensors other than
// `vr_vec.c` are stored as f16 (round to nearest even).
std::vector<uint8_t> write_zjm(const Checkpoint& ck, const std::vector<std::string>& names, bool f16);

// `PackedBundle` (src/weights/packed.rs:290-375): files of `ZJB1` / `ZJB2` bundles by their path
// relative to the model directory. A path already present keeps its first copy.
class Bundle {
public:
    void add(const uint8_t* data, size_t len);
    std::vector<std::string> paths() const;
    // (bytes, length) of a file, or (nullptr, 0) when absent; valid while the bundle lives.
    std::pair<const uint8_t*, size_t> get(const std::string& rel) const;
    std::string notice() const;

private:
    struct Part {
        std::vector<uint8_t> data;
        size_t notice_at = 0, notice_len = 0;
        std::vector<std::pair<std::string, std::pair<size_t, size_t>>> files;  // sorted by path
    };
    std::vector<Part> parts_;
};

// `write_bundle` / `write_bundle_f16` (src/weights/packed.rs:235-288).
std::vector<uint8_t> write_bundle(const std::vector<std::pair<std::string, std::vector<uint8_t>>>& files,
                                  const std::string& notice, bool f16);

}  // namespace zjai
