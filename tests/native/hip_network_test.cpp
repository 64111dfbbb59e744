// Self-test driver for the C++ HipNetwork adapter (used by tests/): loads a
// net file and a planes file, builds HipNetwork, runs EvaluateBatch and
// Evaluate, and writes the NetworkOutput fields for comparison.
//
// Usage: hip_network_test NET PLANES OUT HEADS PRECISION MAX_BATCH [MOVES TEMP]
//   NET    : u32 count, then per tensor u32 name_len, name, u64 n, n floats;
//            or a network file ending in ".pb" / ".pb.gz" (HEADS unused;
//            built through CreateHipNetwork with backend $MFH_TEST_BACKEND,
//            default "hip")
//   PLANES : u32 batch, then batch*112*64 floats
//   OUT    : batch*(1858+3+1) floats from EvaluateBatch, then the same for
//            Evaluate of each position; with MOVES, then the priors of
//            EvaluateBatchPriors (offsets[batch] floats) and its batch*4
//            value fields (wdl[3], value)
//   MOVES  : i32 offsets[batch+1], then i16 policy indices[offsets[batch]]
// Exit codes: 0 ok, 2 usage or file error, 3 std::exception (message on stderr).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <exception>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "hip_network.h"

using namespace MetalFish::NN;

namespace {

bool ReadAll(const char *path, std::vector<char> &out) {
  std::FILE *f = std::fopen(path, "rb");
  if (!f)
    return false;
  std::fseek(f, 0, SEEK_END);
  out.resize(static_cast<std::size_t>(std::ftell(f)));
  std::fseek(f, 0, SEEK_SET);
  const bool ok = std::fread(out.data(), 1, out.size(), f) == out.size();
  std::fclose(f);
  return ok;
}

void Append(std::vector<float> &out, const NetworkOutput &o) {
  out.insert(out.end(), o.policy.begin(), o.policy.end());
  out.insert(out.end(), o.wdl, o.wdl + 3);
  out.push_back(o.value);
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 7 && argc != 9) {
    std::fprintf(stderr, "usage: %s NET PLANES OUT HEADS PRECISION MAX_BATCH [MOVES TEMP]\n",
                 argv[0]);
    return 2;
  }
  const std::string net_path = argv[1];
  auto ends_with = [&](const char *suffix) {
    const std::size_t n = std::strlen(suffix);
    return net_path.size() >= n && net_path.compare(net_path.size() - n, n, suffix) == 0;
  };
  const bool net_file = ends_with(".pb") || ends_with(".pb.gz");
  std::vector<char> net_bytes, plane_bytes;
  if ((!net_file && !ReadAll(argv[1], net_bytes)) || !ReadAll(argv[2], plane_bytes))
    return 2;
  std::vector<Hip::WeightTensor> weights;
  std::vector<std::string> names;
  std::size_t off = 0;
  std::uint32_t count = 0;
  if (!net_file) {
    std::memcpy(&count, net_bytes.data(), 4);
    off = 4;
  }
  names.reserve(count);
  for (std::uint32_t i = 0; i < count; ++i) {
    std::uint32_t len = 0;
    std::memcpy(&len, net_bytes.data() + off, 4);
    off += 4;
    names.emplace_back(net_bytes.data() + off, len);
    off += len;
    std::uint64_t n = 0;
    std::memcpy(&n, net_bytes.data() + off, 8);
    off += 8;
    weights.push_back(Hip::WeightTensor{names.back(),
                                        reinterpret_cast<const float *>(net_bytes.data() + off),
                                        static_cast<std::size_t>(n)});
    off += n * 4;
  }
  std::uint32_t batch = 0;
  std::memcpy(&batch, plane_bytes.data(), 4);
  std::vector<InputPlanes> inputs(batch);
  std::memcpy(inputs.data(), plane_bytes.data() + 4, sizeof(InputPlanes) * batch);

  try {
    Hip::HipNetworkConfig config;
    config.headcount = std::atoi(argv[4]);
    config.precision = std::string(argv[5]) == "bf16" ? MFH_PRECISION_BF16 : MFH_PRECISION_BF16X2;
    config.max_batch = std::atoi(argv[6]);
    // Network files go through the factory branch, with the backend name
    // from MFH_TEST_BACKEND (default "hip").
    std::unique_ptr<Network> owner;
    if (net_file) {
      BackendConfig bc;
      const char *backend = std::getenv("MFH_TEST_BACKEND");
      bc.backend = backend ? backend : "hip";
      bc.cuda_stable_execution_batch_size = config.max_batch;
      owner = Hip::CreateHipNetwork(net_path, bc);
    } else {
      owner = std::make_unique<Hip::HipNetwork>(weights, config);
    }
    Hip::HipNetwork &net = dynamic_cast<Hip::HipNetwork &>(*owner);
    std::fprintf(stderr, "%s\n", net.GetNetworkInfo().c_str());
    const BackendCapabilities caps = net.GetBackendCapabilities();
    if (caps.actual_backend != "hip" || !caps.has_wdl || caps.max_batch_size != config.max_batch)
      throw std::runtime_error("unexpected capabilities");
    if (!net.EvaluateBatch({}).empty())
      throw std::runtime_error("empty batch must give an empty result");
    std::vector<float> out;
    for (const auto &o : net.EvaluateBatch(inputs))
      Append(out, o);
    for (const auto &in : inputs)
      Append(out, net.Evaluate(in));
    if (argc == 9) {
      std::vector<char> move_bytes;
      if (!ReadAll(argv[7], move_bytes))
        return 2;
      std::vector<std::int32_t> offsets(batch + 1);
      std::memcpy(offsets.data(), move_bytes.data(), offsets.size() * 4);
      const auto *idx = reinterpret_cast<const std::int16_t *>(move_bytes.data() +
                                                              offsets.size() * 4);
      std::vector<std::vector<std::int16_t>> moves(batch);
      for (std::uint32_t b = 0; b < batch; ++b)
        moves[b].assign(idx + offsets[b], idx + offsets[b + 1]);
      const auto priors = net.EvaluateBatchPriors(inputs, moves, std::strtof(argv[8], nullptr));
      for (const auto &p : priors)
        out.insert(out.end(), p.priors.begin(), p.priors.end());
      for (const auto &p : priors) {
        out.insert(out.end(), p.wdl, p.wdl + 3);
        out.push_back(p.value);
      }
    }
    std::FILE *f = std::fopen(argv[3], "wb");
    if (!f || std::fwrite(out.data(), 4, out.size(), f) != out.size())
      return 2;
    std::fclose(f);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "%s\n", e.what());
    return 3;
  }
  return 0;
}
