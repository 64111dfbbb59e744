// HipNetwork: MetalFish's NN::Network implemented on the MI355X C ABI
// (include/mfhip.h).  Counterpart of the CUDA backend's CudaNetwork
// (reference src/nn/cuda/cuda_network.h, cuda_network.cpp:235-459): the
// constructor packs and uploads the weights, EvaluateBatch chunks the batch
// to the device's maximum, packs planes into pinned staging buffers and runs
// the forward on the net's stream, and a failed or invalid result is retried
// once before a std::runtime_error is thrown.
#pragma once

#include <cstdint>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "mfhip.h"
#include "nn_network.h"

namespace MetalFish {
namespace NN {
namespace Hip {

// One weight tensor as the reference's NetworkWeightTensorView exposes it
// (reference src/nn/network_weight_inventory.h:33-44): inventory name, fp32
// data, element count.
struct WeightTensor {
  std::string name;
  const float *data = nullptr;
  std::size_t elements = 0;
};

// Format fields of the weights file (reference NetworkFormat, values as in
// net.proto) and the HIP-specific knobs a BackendConfig would carry.
struct HipNetworkConfig {
  int network = MFH_NETWORK_ATTENTIONBODY_WITH_MULTIHEADFORMAT;
  int policy = MFH_POLICY_ATTENTION;
  int value = MFH_VALUE_WDL;
  int moves_left = 0;
  int input_embedding = MFH_INPUT_EMBEDDING_PE_DENSE;
  int default_activation = MFH_DEFAULT_ACTIVATION_MISH;
  int ffn_activation = MFH_ACTIVATION_DEFAULT;
  int smolgen_activation = MFH_ACTIVATION_SWISH;
  int headcount = 0;
  int pol_headcount = 0;  // policy encoder heads (0 without policy encoder layers)
  int precision = MFH_PRECISION_BF16X2;
  int max_batch = 256;  // stable execution batch; larger batches are chunked
  int device = -1;
  bool graphs = true;   // HIP graph capture/replay of the forward
  bool fused_layernorm = false;  // row-panel residual GEMM + LayerNorm (batch >= 128)
};

// Result of EvaluateBatchPriors for one position: the MCTS priors of its
// legal moves in the caller's order, and the value head output decoded as
// NetworkOutput decodes it (value = W - L for WDL nets).
struct PriorsOutput {
  std::vector<float> priors;
  float value = 0.0f;
  float wdl[3] = {};
  bool has_wdl = false;
  float moves_left = 0.0f;
  bool has_moves_left = false;
};

class HipNetwork : public Network {
public:
  HipNetwork(const std::vector<WeightTensor> &weights, const HipNetworkConfig &config);
  // From a `.pb` / `.pb.gz` network file, as CreateNetwork(weights_path, ...)
  // loads one first (reference src/nn/network.cpp:226-258): the file's
  // format fields and head count replace those of `config`; precision,
  // max_batch and device are taken from `config`.
  HipNetwork(const std::string &weights_path, const HipNetworkConfig &config);
  ~HipNetwork() override;
  HipNetwork(const HipNetwork &) = delete;
  HipNetwork &operator=(const HipNetwork &) = delete;

  NetworkOutput Evaluate(const InputPlanes &input) override;
  std::vector<NetworkOutput> EvaluateBatch(const std::vector<InputPlanes> &inputs) override;
  // The legal-move gather and prior softmax of the MCTS evaluator
  // (reference src/mcts/evaluator.cpp:181-224, src/mcts/search.cpp:127-199)
  // done on the device: move_indices[i] holds position i's policy indices
  // (MoveToNNIndex order, at most 256), and only the priors come back.
  std::vector<PriorsOutput> EvaluateBatchPriors(
      const std::vector<InputPlanes> &inputs,
      const std::vector<std::vector<std::int16_t>> &move_indices, float softmax_temp);
  std::string GetNetworkInfo() const override;
  bool HasWDL() const override { return wdl_; }
  bool HasMovesLeft() const override { return mlh_; }
  BackendCapabilities GetBackendCapabilities() const override;

private:
  void Create(mfh_net_desc desc, const mfh_tensor *tensors, int count);
  void RunChunk(const InputPlanes *inputs, int count, NetworkOutput *outputs);

  mfh_net *net_ = nullptr;
  // Held across each chunk's C call and the decode of its outputs, which
  // live in the members below (the reference's execution_mutex_, held across
  // run and decode, cuda_network.cpp:442-446): MCTS workers may call
  // EvaluateBatch and EvaluateBatchPriors concurrently.
  std::mutex mu_;
  bool graphs_ = true;
  bool wdl_ = true;
  bool mlh_ = false;
  std::vector<float> moves_;
  int max_batch_ = 0;
  std::vector<float> policy_;
  std::vector<float> value_;
  std::vector<std::uint64_t> masks_;
  std::vector<float> values_;
};

// The "hip" branch of NN::CreateNetwork (reference src/nn/network.cpp:
// 137-208, path overloads 226-258): loads a `.pb` / `.pb.gz` network file and
// builds a HipNetwork with the BackendConfig knobs the HIP backend honours
// (cuda_device -> device, cuda_graph_execution -> graph replay,
// cuda_stable_execution_batch_size -> max_batch when positive).  Accepts the
// backend names "hip", "auto" and "accelerator"; any other name throws
// std::runtime_error, as does a file or net the backend cannot run.
std::unique_ptr<Network> CreateHipNetwork(const std::string &weights_path,
                                          const BackendConfig &config);

}  // namespace Hip
}  // namespace NN
}  // namespace MetalFish
