// MetalFish's NN backend interface, declared for this repository so the HIP
// adapter builds stand-alone.  The declarations deliberately match the
// reference interface name for name (reference src/nn/network.h:21-75,
// input_planes.h:22-29, network_output.h:17-24) so that HipNetwork drops in
// behind NN::CreateNetwork unchanged; inside the reference tree these come
// from its own headers instead.
#pragma once

#include <array>
#include <memory>
#include <string>
#include <vector>

namespace MetalFish {
namespace NN {

constexpr int kMoveHistory = 8;
constexpr int kPlanesPerBoard = 13;
constexpr int kAuxPlaneBase = kPlanesPerBoard * kMoveHistory;
constexpr int kTotalPlanes = 112;
constexpr int kPolicyOutputs = 1858;

using InputPlanes = std::array<std::array<float, 64>, kTotalPlanes>;

struct NetworkOutput {
  std::array<float, kPolicyOutputs> policy{};
  float value = 0.0f;
  float wdl[3] = {};
  bool has_wdl = false;
  float moves_left = 0.0f;
  bool has_moves_left = false;
};

struct BackendCapabilities {
  std::string actual_backend = "unknown";
  bool has_wdl = false;
  bool has_moves_left = false;
  int max_batch_size = 0;
  int stable_execution_batch_size = 0;
  int cuda_configured_device = -1;
  int cuda_selected_device = -1;
  bool cuda_graph_execution = false;
  bool cuda_deterministic_attention_softmax = false;
  bool cuda_full_buffer_clear = false;
  std::string device_name;
  std::string compute_units;
};

struct BackendConfig {
  std::string backend = "auto";
  std::string coreml_model_path;
  std::string coreml_compute_units = "cpu-ne";
  int cuda_device = -1;
  bool cuda_graph_execution = true;
  int cuda_stable_execution_batch_size = 0;
  bool cuda_deterministic_attention_softmax = true;
  bool cuda_full_buffer_clear = true;
};

class Network {
public:
  virtual ~Network() = default;
  virtual NetworkOutput Evaluate(const InputPlanes &input) = 0;
  virtual std::vector<NetworkOutput>
  EvaluateBatch(const std::vector<InputPlanes> &inputs) = 0;
  virtual std::string GetNetworkInfo() const = 0;
  virtual bool HasWDL() const { return false; }
  virtual bool HasMovesLeft() const { return false; }
  virtual BackendCapabilities GetBackendCapabilities() const {
    return BackendCapabilities{};
  }
};

}  // namespace NN
}  // namespace MetalFish
