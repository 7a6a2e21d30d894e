// checkpoint.h — quantized transformer checkpoints of the hot path: the
// safetensors container, quantized-weight detection and loading, and the
// offline quantizer.
//
//   SafeTensorsWriter      safetensors_writer.h:12-104 (same bytes: header
//                          in insertion order, space padding to 8, tensors
//                          back to back)
//   SafeTensorsLoader      safetensors.h:40-110 (one file or a sharded
//                          index; the dtype strings of safetensors.h:79-97
//                          plus F8_E4M3). Where the reference prints "Unknown
//                          dtype" and skips the tensor (safetensors.h:94-96),
//                          load() fails and names it.
//   load_model_dir         safetensors.h:235-274
//   detect_checkpoint /
//   load_quantized_weight  transformer.h:146-199 (pre-quantized I8 or
//                          F8_E4M3 + "<name>.__scales__" F32, BF16 layers kept
//                          as BF16, other BF16 weights quantized on load)
//   quantize_checkpoint    quantize.cu:110-161, 334-341, 462-539 (the same
//                          tensor list and order; F8_E4M3 is the e4m3 mode)
#pragma once

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "kernels.h"
#include "tensor.h"

struct TensorInfo {
    std::string name;
    std::string filename;
    DType dtype = DType::BF16;
    std::string dtype_str;  // as written in the header
    std::vector<int64_t> shape;
    size_t data_offset = 0;  // from the file's data start
    size_t nbytes = 0;
};

class SafeTensorsWriter {
public:
    void add(const std::string& name, const std::string& dtype_str, const std::vector<int64_t>& shape,
             const void* data_ptr, size_t nbytes);
    bool write(const std::string& filepath) const;
    size_t num_entries() const { return entries_.size(); }

private:
    struct Entry {
        std::string name;
        std::string dtype_str;
        std::vector<int64_t> shape;
        std::vector<uint8_t> data;
    };
    std::vector<Entry> entries_;
};

class SafeTensorsLoader {
public:
    // Adds one file's tensors. False, with error(), for an unreadable file,
    // a malformed header or a tensor of unknown dtype.
    bool load_file(const std::string& filepath);
    // model.safetensors.index.json: every shard its weight_map names.
    bool load_sharded(const std::string& index_path);
    const std::string& error() const { return error_; }

    bool has_tensor(const std::string& name) const;
    const TensorInfo& get_info(const std::string& name) const;  // exits when absent, as the reference
    const std::vector<std::string>& names() const { return order_; }  // header order
    std::vector<uint8_t> read_bytes(const std::string& name) const;
    Tensor load_tensor(const std::string& name) const;  // device copy, the file's dtype

private:
    struct File {
        std::string filepath;
        size_t data_start = 0;
    };
    std::vector<File> files_;
    std::vector<TensorInfo> tensors_;
    std::vector<std::string> order_;
    std::string error_;
    const TensorInfo* find(const std::string& name) const;
    size_t data_start(const std::string& filename) const;
};

// Single merged file (model.safetensors, diffusion_pytorch_model.safetensors)
// or a sharded index under `dir`; `dir` may also name a .safetensors file.
bool load_model_dir(const std::string& dir, SafeTensorsLoader& loader);

enum class CheckpointKind { BF16 = 0, INT8 = 1, FP8 = 2 };
CheckpointKind detect_checkpoint(const SafeTensorsLoader& loader);

// One linear's weight from a checkpoint: I8 -> INT8_HADAMARD, F8_E4M3 ->
// FP8_HADAMARD (data + "<name>.__scales__", had_block_size = K & -K), BF16 ->
// QuantMode::BF16 when `keep_bf16`, else quantized to int8 on load.
QuantizedWeight load_quantized_weight(const SafeTensorsLoader& loader, const std::string& name,
                                      bool keep_bf16 = true);

// The offline quantizer's tensor list for `num_blocks` blocks (the reference
// fixes 60), in output order: (name, true) for a linear weight that is
// quantized, (name, false) for one copied through.
std::vector<std::pair<std::string, bool>> quantize_plan(int num_blocks);

// Reads the BF16 checkpoint at `in` (load_model_dir), quantizes the plan's
// linears with quantize_weight_tensor / quantize_weight_tensor_fp8 on the
// current HIP device and writes `out`. False with *err on failure.
bool quantize_checkpoint(const std::string& in, const std::string& out, QuantMode mode, int num_blocks,
                         std::string* err);
