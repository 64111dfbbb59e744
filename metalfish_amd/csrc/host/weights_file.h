// Reader for MetalFish / Lc0 network files (`.pb`, `.pb.gz`) with no
// protobuf dependency: a proto2 wire-format decoder for the `Net` message of
// reference src/nn/proto/net.proto, the reference loader's legacy format
// fix-ups and layer decoding (src/nn/loader.cpp:37-251), the ConvBlock
// batch-norm fold and head resolution of src/nn/weights.cpp:91-291, and the
// tensor naming and order of the weight inventory
// (src/nn/network_weight_inventory.cpp:116-354).  Host-only code; errors are
// std::runtime_error with the reference's messages where it has one.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace mfh {
namespace wf {

// NetworkFormat (net.proto:253-343) after the legacy fix-ups.
struct NetFormat {
  int input = 0;
  int output = 0;
  int network = 0;
  int policy = 0;
  int value = 0;
  int moves_left = 0;
  int default_activation = 0;
  int smolgen_activation = 0;
  int ffn_activation = 0;
  int input_embedding = 0;
  bool has_input_embedding = false;
};

// One inventory tensor: name, decoded fp32 values, dims of the layer (or the
// flat element count when the file gives none).
struct Tensor {
  std::string name;
  std::vector<float> data;
  std::vector<uint32_t> dims;
};

struct Weights {
  NetFormat format;
  uint32_t headcount = 0;      // Weights.headcount (body attention heads)
  uint32_t pol_headcount = 0;  // pol_headcount of the selected policy head
  std::string policy_head;     // selected policy head ("vanilla")
  std::string value_head;      // selected value head ("winner")
  std::vector<Tensor> tensors; // inventory order
};

// LoadWeightsFromFile (loader.cpp:162-185): gzip-decompresses names ending
// in ".gz", then ParseWeights.
Weights LoadFile(const std::string &path);

// ParseWeightsProto + FixOlderWeightsFile (loader.cpp:86-158), then
// MultiHeadWeights (weights.cpp:216-291) and the inventory of the selected
// heads (network_weight_inventory.cpp:332-352).
Weights Parse(const uint8_t *data, size_t size);

// DecodeLayer (loader.cpp:187-251) on raw Layer fields: encoding is the
// Layer.Encoding value (0 = unknown, read as LINEAR16).
std::vector<float> DecodeLayer(int encoding, float min_val, float max_val,
                               const uint8_t *params, size_t bytes);

}  // namespace wf
}  // namespace mfh
