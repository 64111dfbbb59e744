#include "hip_network.h"

#include <cmath>
#include <stdexcept>

namespace MetalFish {
namespace NN {
namespace Hip {
namespace {

std::string LastError(const char *what, int rc) {
  return std::string("HIP backend ") + what + " failed (" + std::to_string(rc) +
         "): " + mfh_last_error();
}

// Output sanity check, as the CUDA backend applies before trusting a batch
// (reference src/nn/cuda/cuda_network.cpp:199-231): finite logits and WDL
// probabilities that sum to about one.
bool OutputsValid(const float *policy, const float *value, int count, bool wdl) {
  for (int i = 0; i < count * kPolicyOutputs; ++i)
    if (!std::isfinite(policy[i]))
      return false;
  for (int b = 0; b < count; ++b) {
    if (wdl) {
      const float *v = value + 3 * b;
      const float sum = v[0] + v[1] + v[2];
      if (!std::isfinite(sum) || sum < 0.5f || sum > 1.5f)
        return false;
    } else if (!std::isfinite(value[b])) {
      return false;
    }
  }
  return true;
}

mfh_net_desc DescFromConfig(const HipNetworkConfig &config) {
  mfh_net_desc desc{};
  desc.network = config.network;
  desc.policy = config.policy;
  desc.value = config.value;
  desc.moves_left = config.moves_left;
  desc.input_embedding = config.input_embedding;
  desc.default_activation = config.default_activation;
  desc.ffn_activation = config.ffn_activation;
  desc.smolgen_activation = config.smolgen_activation;
  desc.headcount = config.headcount;
  desc.pol_headcount = config.pol_headcount;
  desc.weights_dtype = MFH_WEIGHTS_BF16;
  desc.precision = config.precision;
  desc.max_batch = config.max_batch;
  desc.device = config.device;
  desc.fused_layernorm = config.fused_layernorm ? 1 : 0;
  return desc;
}

}  // namespace

HipNetwork::HipNetwork(const std::vector<WeightTensor> &weights,
                       const HipNetworkConfig &config)
    : graphs_(config.graphs) {
  std::vector<mfh_tensor> tensors;
  tensors.reserve(weights.size());
  for (const auto &w : weights)
    tensors.push_back(mfh_tensor{w.name.c_str(), w.data, static_cast<std::uint64_t>(w.elements)});
  Create(DescFromConfig(config), tensors.data(), static_cast<int>(tensors.size()));
}

HipNetwork::HipNetwork(const std::string &weights_path, const HipNetworkConfig &config)
    : graphs_(config.graphs) {
  mfh_weights *file = nullptr;
  int rc = mfh_weights_load(weights_path.c_str(), &file);
  if (rc != MFH_OK)
    throw std::runtime_error(LastError("weights load", rc));
  mfh_net_desc desc = DescFromConfig(config);
  const mfh_tensor *tensors = nullptr;
  int count = 0;
  rc = mfh_weights_describe(file, nullptr, &desc);
  if (rc == MFH_OK)
    rc = mfh_weights_tensors(file, &tensors, &count);
  if (rc != MFH_OK) {
    const std::string msg = LastError("weights load", rc);
    mfh_weights_free(file);
    throw std::runtime_error(msg);
  }
  try {
    Create(desc, tensors, count);
  } catch (...) {
    mfh_weights_free(file);
    throw;
  }
  // The device holds its own copy of the weights now.
  mfh_weights_free(file);
}

void HipNetwork::Create(mfh_net_desc desc, const mfh_tensor *tensors, int count) {
  int rc = mfh_net_create(&desc, tensors, count, &net_);
  if (rc != MFH_OK)
    throw std::runtime_error(LastError("initialisation", rc));
  if (!graphs_) {
    rc = mfh_net_set_graphs(net_, 0);
    if (rc != MFH_OK) {
      mfh_net_destroy(net_);
      net_ = nullptr;
      throw std::runtime_error(LastError("initialisation", rc));
    }
  }
  wdl_ = desc.value == MFH_VALUE_WDL;
  mlh_ = desc.moves_left == MFH_MOVES_LEFT_V1;
  max_batch_ = desc.max_batch;
  moves_.resize(static_cast<std::size_t>(max_batch_));
  policy_.resize(static_cast<std::size_t>(max_batch_) * kPolicyOutputs);
  value_.resize(static_cast<std::size_t>(max_batch_) * 3);
}

HipNetwork::~HipNetwork() { mfh_net_destroy(net_); }

void HipNetwork::RunChunk(const InputPlanes *inputs, int count, NetworkOutput *outputs) {
  // InputPlanes is a contiguous 112x64 float array, so a run of them is the
  // planes[count*112*64] layout the C ABI takes.
  const float *planes = inputs[0][0].data();
  std::lock_guard<std::mutex> lock(mu_);
  for (int attempt = 0; attempt < 2; ++attempt) {
    const int rc = mfh_net_eval_planes(net_, count, planes, policy_.data(), value_.data(),
                                       mlh_ ? moves_.data() : nullptr);
    if (rc != MFH_OK) {
      if (attempt == 0)
        continue;
      throw std::runtime_error(LastError("evaluation", rc));
    }
    if (!OutputsValid(policy_.data(), value_.data(), count, wdl_)) {
      if (attempt == 0)
        continue;
      throw std::runtime_error("HIP backend produced invalid outputs (non-finite or WDL "
                               "not normalised) twice");
    }
    break;
  }
  // DecodeNetworkOutputBatch (reference src/nn/network_output_decoder.cpp:
  // 31-78): raw logits, WDL, value = W - L.
  for (int b = 0; b < count; ++b) {
    NetworkOutput &out = outputs[b];
    const float *p = policy_.data() + static_cast<std::size_t>(b) * kPolicyOutputs;
    for (int i = 0; i < kPolicyOutputs; ++i)
      out.policy[i] = p[i];
    if (wdl_) {
      out.has_wdl = true;
      out.wdl[0] = value_[3 * b];
      out.wdl[1] = value_[3 * b + 1];
      out.wdl[2] = value_[3 * b + 2];
      out.value = out.wdl[0] - out.wdl[2];
    } else {
      out.has_wdl = false;
      out.value = value_[b];
      out.wdl[0] = out.wdl[1] = out.wdl[2] = 0.0f;
    }
    out.has_moves_left = mlh_;
    out.moves_left = mlh_ ? moves_[b] : 0.0f;
  }
}

NetworkOutput HipNetwork::Evaluate(const InputPlanes &input) {
  NetworkOutput out;
  RunChunk(&input, 1, &out);
  return out;
}

std::vector<NetworkOutput> HipNetwork::EvaluateBatch(const std::vector<InputPlanes> &inputs) {
  std::vector<NetworkOutput> outputs(inputs.size());
  for (std::size_t start = 0; start < inputs.size(); start += max_batch_) {
    const int count = static_cast<int>(std::min<std::size_t>(max_batch_, inputs.size() - start));
    RunChunk(inputs.data() + start, count, outputs.data() + start);
  }
  return outputs;
}

std::vector<PriorsOutput> HipNetwork::EvaluateBatchPriors(
    const std::vector<InputPlanes> &inputs,
    const std::vector<std::vector<std::int16_t>> &move_indices, float softmax_temp) {
  if (move_indices.size() != inputs.size())
    throw std::runtime_error("HIP backend: one move list per position is required");
  std::vector<PriorsOutput> outputs(inputs.size());
  std::vector<std::int32_t> offsets;
  std::vector<std::int16_t> flat;
  std::vector<float> priors;
  for (std::size_t start = 0; start < inputs.size(); start += max_batch_) {
    const int count = static_cast<int>(std::min<std::size_t>(max_batch_, inputs.size() - start));
    std::lock_guard<std::mutex> lock(mu_);
    masks_.resize(static_cast<std::size_t>(count) * kTotalPlanes);
    values_.resize(masks_.size());
    int rc = mfh_pack_planes(count, inputs[start][0].data(), masks_.data(), values_.data());
    offsets.assign(1, 0);
    flat.clear();
    for (int b = 0; b < count; ++b) {
      const auto &m = move_indices[start + b];
      flat.insert(flat.end(), m.begin(), m.end());
      offsets.push_back(static_cast<std::int32_t>(flat.size()));
    }
    priors.resize(flat.size());
    if (rc == MFH_OK)
      rc = mfh_net_eval_priors(net_, count, masks_.data(), values_.data(), offsets.data(),
                               flat.data(), softmax_temp, priors.data(), value_.data(),
                               mlh_ ? moves_.data() : nullptr);
    if (rc != MFH_OK)
      throw std::runtime_error(LastError("priors evaluation", rc));
    for (int b = 0; b < count; ++b) {
      PriorsOutput &out = outputs[start + b];
      out.priors.assign(priors.begin() + offsets[b], priors.begin() + offsets[b + 1]);
      if (wdl_) {
        out.has_wdl = true;
        for (int k = 0; k < 3; ++k)
          out.wdl[k] = value_[3 * b + k];
        out.value = out.wdl[0] - out.wdl[2];
      } else {
        out.value = value_[b];
      }
      out.has_moves_left = mlh_;
      out.moves_left = mlh_ ? moves_[b] : 0.0f;
    }
  }
  return outputs;
}

std::string HipNetwork::GetNetworkInfo() const {
  char buf[1024];
  if (mfh_net_info(net_, buf, sizeof(buf)) != MFH_OK)
    return "HIP transformer backend";
  return buf;
}

BackendCapabilities HipNetwork::GetBackendCapabilities() const {
  BackendCapabilities caps;
  mfh_capabilities c{};
  caps.actual_backend = "hip";
  if (mfh_net_capabilities(net_, &c) == MFH_OK) {
    caps.has_wdl = c.has_wdl != 0;
    caps.has_moves_left = c.has_moves_left != 0;
    caps.max_batch_size = c.max_batch_size;
    caps.stable_execution_batch_size = c.max_batch_size;
    caps.device_name = std::string(c.device_name) + " (" + c.arch_name + ")";
  }
  return caps;
}

std::unique_ptr<Network> CreateHipNetwork(const std::string &weights_path,
                                          const BackendConfig &config) {
  if (config.backend != "hip" && config.backend != "auto" && config.backend != "accelerator")
    throw std::runtime_error("HIP backend cannot serve backend \"" + config.backend + "\"");
  HipNetworkConfig hc;
  hc.device = config.cuda_device;
  hc.graphs = config.cuda_graph_execution;
  if (config.cuda_stable_execution_batch_size > 0)
    hc.max_batch = config.cuda_stable_execution_batch_size;
  return std::make_unique<HipNetwork>(weights_path, hc);
}

}  // namespace Hip
}  // namespace NN
}  // namespace MetalFish
