// safetensors.hpp — the reference's checkpoint format for DenseBlock networks.
//
//   SafetensorWriter   src/io/safetensor.rs:9-203  (container: 8-byte LE header
//                      length, JSON header padded with spaces to a multiple of 8,
//                      raw little-endian tensor bytes in insertion order)
//   SafetensorFile     src/io/save.rs:118-577      (names layer<N>.<param>, shapes,
//                      which tensors are written, how a file becomes DenseBlocks)
//
// The JSON header is written the way the reference's serde_json (1.0.150,
// without `preserve_order`) pretty-prints a map: keys sorted bytewise at every
// level, two-space indentation, one array element per line.
#pragma once

#include <cstdint>
#include <istream>
#include <map>
#include <ostream>
#include <string>
#include <utility>
#include <vector>

#include "soklyn.hpp"

namespace soklyn {

// A parsed JSON value (numbers keep their source text).
struct JsonValue {
    enum class Kind { Null, Bool, Number, String, Array, Object };
    Kind kind = Kind::Null;
    std::string text;                            // String contents, Number / Bool source text
    std::vector<JsonValue> items;                // Array
    std::map<std::string, JsonValue> members;    // Object (sorted, a repeated key keeps the last value)

    static JsonValue parse(const std::string &src);   // throws Error(SerdeJSON)
    std::string to_pretty() const;                    // serde_json::to_string_pretty layout
    std::string to_compact() const;                   // serde_json::Value::to_string layout
};

struct SafetensorDescriptor {
    std::string name;
    std::vector<size_t> shape;
    std::vector<uint8_t> data;
    Precision precision;
};

class SafetensorWriter {
  public:
    void pass(std::string name, std::vector<size_t> shape, std::vector<uint8_t> data, Precision precision);
    // IndexMap::insert: a new key is appended, an existing one keeps its place
    void pass_metadata(const std::string &key, const std::string &value);
    const std::vector<SafetensorDescriptor> &get_descriptors() const { return descriptors_; }
    const std::vector<std::pair<std::string, std::string>> &get_metadata() const { return metadata_; }

    static SafetensorWriter read(std::istream &in);
    void write(std::ostream &out) const;
    std::string header_json() const;   // the padded header text write() emits

  private:
    std::vector<SafetensorDescriptor> descriptors_;
    std::vector<std::pair<std::string, std::string>> metadata_;
};

class SafetensorFile {
  public:
    SafetensorFile() = default;
    template <class T> static SafetensorFile from_ffn(const GpuContext &ctx, const FeedForwardNetwork<T> &network);
    template <class T> static SafetensorFile from_blocks(const GpuContext &ctx, const std::vector<DenseBlock<T>> &blocks);
    template <class T> void pass_blocks(const GpuContext &ctx, const std::vector<DenseBlock<T>> &blocks);
    void pass_metadata(const std::string &key, const std::string &value) { writer_.pass_metadata(key, value); }
    const std::vector<std::pair<std::string, std::string>> &get_metadata() const { return writer_.get_metadata(); }
    // layer<layer_num>.{w,b,norm_w,norm_b} in T; with training state the fp32
    // moments, then the fp32 masters that exist (save.rs:227-345)
    template <class T> void pass_layer(const GpuContext &ctx, const DenseBlock<T> &layer, size_t layer_num);
    // Written to a temporary file in the target directory, then renamed over the target.
    void save(const std::string &path) const;
    static SafetensorFile read(const std::string &path);
    // Layers 1..max as DenseBlocks with the default LayerInitConfig (save.rs:416-576).
    template <class T>
    std::vector<DenseBlock<T>> into_blocks(const GpuContext &ctx, bool is_training, size_t max_batch_size) &&;
    const SafetensorWriter &writer() const { return writer_; }

  private:
    SafetensorWriter writer_;
};

}  // namespace soklyn
