// Network-file reader: proto2 wire decoding of reference
// src/nn/proto/net.proto without libprotobuf, plus the reference loader's
// semantics (src/nn/loader.cpp, src/nn/weights.cpp,
// src/nn/network_weight_inventory.cpp), cited per function below.
#include "weights_file.h"

#include <zlib.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <iterator>
#include <stdexcept>

namespace mfh {
namespace wf {
namespace {

// ---- proto2 wire format ----------------------------------------------------
//
// A message is a sequence of (key, payload) records, key = field << 3 | wire
// type.  Wire types: 0 varint, 1 fixed 64-bit, 2 length-delimited, 5 fixed
// 32-bit; 3/4 open and close a (deprecated) group, which only unknown fields
// can use here and which are skipped.  Parsing semantics follow the proto2
// rules libprotobuf applies: the last occurrence of a scalar or bytes field
// wins, occurrences of a message field merge, a known field seen with another
// wire type is kept as unknown (ignored), a repeated varint field may be
// packed, and a closed-enum value outside the enum is not stored (the field
// keeps its previous value).

struct Record {
  uint32_t field;
  uint32_t wire;
  uint64_t value;             // wire 0, 1, 5
  const uint8_t *data;        // wire 2
  size_t size;                // wire 2
};

[[noreturn]] void ParseFail() { throw std::runtime_error("Failed to parse protobuf weights file"); }

uint64_t ReadVarint(const uint8_t *&p, const uint8_t *end) {
  uint64_t v = 0;
  for (int shift = 0; shift < 70; shift += 7) {
    if (p >= end)
      ParseFail();
    const uint8_t byte = *p++;
    if (shift < 64)
      v |= static_cast<uint64_t>(byte & 0x7f) << shift;
    if (!(byte & 0x80))
      return v;
  }
  ParseFail();  // more than ten bytes
}

uint64_t ReadLittleEndian(const uint8_t *&p, const uint8_t *end, int bytes) {
  if (end - p < bytes)
    ParseFail();
  uint64_t v = 0;
  for (int i = 0; i < bytes; ++i)
    v |= static_cast<uint64_t>(p[i]) << (8 * i);
  p += bytes;
  return v;
}

// Skips records up to the end-group key of `field` (wire type 3 already read).
void SkipGroup(const uint8_t *&p, const uint8_t *end, uint32_t field, int depth) {
  if (depth > 64)
    ParseFail();
  while (true) {
    const uint64_t key = ReadVarint(p, end);
    const uint32_t f = static_cast<uint32_t>(key >> 3), wire = key & 7;
    if (f == 0 || (key >> 3) > 0x1fffffff)
      ParseFail();
    switch (wire) {
    case 0: ReadVarint(p, end); break;
    case 1: ReadLittleEndian(p, end, 8); break;
    case 2: {
      const uint64_t n = ReadVarint(p, end);
      if (n > static_cast<uint64_t>(end - p))
        ParseFail();
      p += n;
      break;
    }
    case 3: SkipGroup(p, end, f, depth + 1); break;
    case 4:
      if (f != field)
        ParseFail();
      return;
    case 5: ReadLittleEndian(p, end, 4); break;
    default: ParseFail();
    }
  }
}

class Message {
public:
  Message() = default;
  Message(const uint8_t *data, size_t size) { Merge(data, size); }

  void Merge(const uint8_t *data, size_t size) {
    const uint8_t *p = data, *end = data + size;
    while (p < end) {
      const uint64_t key = ReadVarint(p, end);
      if ((key >> 3) == 0 || (key >> 3) > 0x1fffffff)
        ParseFail();
      Record r{static_cast<uint32_t>(key >> 3), static_cast<uint32_t>(key & 7), 0, nullptr, 0};
      switch (r.wire) {
      case 0: r.value = ReadVarint(p, end); break;
      case 1: r.value = ReadLittleEndian(p, end, 8); break;
      case 2: {
        const uint64_t n = ReadVarint(p, end);
        if (n > static_cast<uint64_t>(end - p))
          ParseFail();
        r.data = p;
        r.size = static_cast<size_t>(n);
        p += n;
        break;
      }
      case 3: SkipGroup(p, end, r.field, 0); continue;
      case 5: r.value = ReadLittleEndian(p, end, 4); break;
      default: ParseFail();  // stray end-group or reserved wire type
      }
      records_.push_back(r);
    }
  }

  // Sub-message present (any length-delimited occurrence).
  bool Has(uint32_t field) const {
    for (const auto &r : records_)
      if (r.field == field && r.wire == 2)
        return true;
    return false;
  }

  // All occurrences of a message field merged, as libprotobuf does.
  Message Sub(uint32_t field) const {
    Message m;
    for (const auto &r : records_)
      if (r.field == field && r.wire == 2)
        m.Merge(r.data, r.size);
    return m;
  }

  // Each occurrence of a repeated message field.
  std::vector<Message> Each(uint32_t field) const {
    std::vector<Message> out;
    for (const auto &r : records_)
      if (r.field == field && r.wire == 2)
        out.emplace_back(r.data, r.size);
    return out;
  }

  bool HasVarint(uint32_t field) const {
    for (const auto &r : records_)
      if (r.field == field && r.wire == 0)
        return true;
    return false;
  }

  uint32_t Uint32(uint32_t field) const {
    uint32_t v = 0;
    for (const auto &r : records_)
      if (r.field == field && r.wire == 0)
        v = static_cast<uint32_t>(r.value);
    return v;
  }

  // Closed enum: the last occurrence whose value is one of `valid`.
  template <size_t N>
  bool Enum(uint32_t field, const int (&valid)[N], int *out) const {
    bool set = false;
    for (const auto &r : records_) {
      if (r.field != field || r.wire != 0)
        continue;
      const int v = static_cast<int32_t>(static_cast<uint32_t>(r.value));
      for (int ok : valid)
        if (v == ok) {
          *out = v;
          set = true;
        }
    }
    return set;
  }

  bool HasFixed32(uint32_t field) const {
    for (const auto &r : records_)
      if (r.field == field && r.wire == 5)
        return true;
    return false;
  }

  uint32_t Fixed32(uint32_t field) const {
    uint32_t v = 0;
    for (const auto &r : records_)
      if (r.field == field && r.wire == 5)
        v = static_cast<uint32_t>(r.value);
    return v;
  }

  float Float(uint32_t field) const {
    const uint32_t bits = Fixed32(field);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
  }

  // Last occurrence of a bytes field (empty if absent).
  std::pair<const uint8_t *, size_t> Bytes(uint32_t field) const {
    std::pair<const uint8_t *, size_t> v{nullptr, 0};
    for (const auto &r : records_)
      if (r.field == field && r.wire == 2)
        v = {r.data, r.size};
    return v;
  }

  // Repeated uint32, packed or not.
  std::vector<uint32_t> Uint32List(uint32_t field) const {
    std::vector<uint32_t> out;
    for (const auto &r : records_) {
      if (r.field != field)
        continue;
      if (r.wire == 0) {
        out.push_back(static_cast<uint32_t>(r.value));
      } else if (r.wire == 2) {
        const uint8_t *p = r.data, *end = r.data + r.size;
        while (p < end)
          out.push_back(static_cast<uint32_t>(ReadVarint(p, end)));
      }
    }
    return out;
  }

private:
  std::vector<Record> records_;
};

// ---- net.proto field numbers and enum values --------------------------------

namespace F {  // Weights (net.proto:17-242)
enum : uint32_t {
  kInput = 1, kResidual = 2, kPolicy = 3, kIpPolW = 4, kIpPolB = 5, kValue = 6, kIp1ValW = 7,
  kIp1ValB = 8, kIp2ValW = 9, kIp2ValB = 10, kPolicy1 = 11, kMovesLeft = 12, kIp1MovW = 13,
  kIp1MovB = 14, kIp2MovW = 15, kIp2MovB = 16, kIp2PolW = 17, kIp2PolB = 18, kIp3PolW = 19,
  kIp3PolB = 20, kPolEncoder = 21, kIp4PolW = 22, kPolHeadcount = 24, kIpEmbW = 25,
  kIpEmbB = 26, kEncoder = 27, kHeadcount = 28, kIpValW = 29, kIpValB = 30, kIpMovW = 31,
  kIpMovB = 32, kIpMultGate = 33, kIpAddGate = 34, kSmolgenW = 35, kIpEmbPreprocW = 37,
  kIpEmbPreprocB = 38, kIpEmbLnGammas = 39, kIpEmbLnBetas = 40, kIpEmbFfn = 41,
  kIpEmbFfnLnGammas = 42, kIpEmbFfnLnBetas = 43, kValueHeads = 44, kPolicyHeads = 45
};
}  // namespace F

const int kLayerEncodings[] = {0, 1, 2, 3, 4};                  // net.proto:22-28
const int kInputFormats[] = {0, 1, 2, 3, 4, 132, 5, 133};       // net.proto:255-264
const int kOutputFormats[] = {0, 1, 2};                         // net.proto:268-272
const int kNetworkStructures[] = {0, 1, 2, 3, 4, 5, 6, 7, 134}; // net.proto:277-288
const int kPolicyFormats[] = {0, 1, 2, 3};                      // net.proto:292-297
const int kValueFormats[] = {0, 1, 2, 3};                       // net.proto:301-306
const int kMovesLeftFormats[] = {0, 1};                         // net.proto:310-313
const int kActivations[] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9};      // net.proto:316-327
const int kDefaultActivations[] = {0, 1};                       // net.proto:329-332
const int kInputEmbeddings[] = {0, 1, 2};                       // net.proto:338-342

enum {
  kNetClassical = 1, kNetSe = 2, kNetClassicalHead = 3, kNetSeHead = 4, kNetAttentionHead = 6,
  kNetAttentionMultiHead = 7, kNetAbLegacyMultiHead = 134
};
enum { kInputClassical112 = 1, kOutputClassical = 1, kValueClassical = 1, kPolicyClassical = 1 };
enum { kActRelu2 = 8, kActSwish = 7 };
enum { kEmbeddingPeMap = 1, kEmbeddingPeDense = 2 };
enum { kMovesLeftV1 = 1 };
const uint32_t kWeightMagic = 0x1c0;

// ---- decoded tensors ---------------------------------------------------------

struct Vec {
  std::vector<float> v;
  std::vector<uint32_t> dims;
  bool empty() const { return v.empty(); }
};

Vec DecodeLayerMessage(const Message &layer) {
  int encoding = 0;
  layer.Enum(4, kLayerEncodings, &encoding);
  const auto params = layer.Bytes(3);
  Vec out;
  out.v = DecodeLayer(encoding, layer.Float(1), layer.Float(2), params.first, params.second);
  out.dims = layer.Uint32List(5);
  return out;
}

Vec LayerOf(const Message &parent, uint32_t field) { return DecodeLayerMessage(parent.Sub(field)); }

// BaseWeights::ConvBlock (reference src/nn/weights.cpp:91-143): missing
// batch-norm betas/gammas become 0/1 and missing biases 0 (one per mean),
// then the batch norm is folded into the convolution:
// gamma' = gamma / sqrt(stddiv + 1e-5), w[o][:] *= gamma'[o],
// b[o] = beta[o] - gamma'[o] * (mean[o] - b[o]).
struct Conv {
  Vec weights, biases;
};

Conv ConvBlockOf(const Message &parent, uint32_t field) {
  const Message m = parent.Sub(field);
  Conv c;
  c.weights = LayerOf(m, 1);
  c.biases = LayerOf(m, 2);
  Vec means = LayerOf(m, 3), stddivs = LayerOf(m, 4), gammas = LayerOf(m, 5),
      betas = LayerOf(m, 6);
  if (c.weights.empty())
    return c;
  auto flat_dims = [](Vec &x) {
    if (!x.empty() && x.dims.empty())
      x.dims.push_back(static_cast<uint32_t>(x.v.size()));
  };
  if (betas.empty()) {
    for (size_t i = 0; i < means.v.size(); ++i) {
      betas.v.push_back(0.0f);
      gammas.v.push_back(1.0f);
    }
    flat_dims(betas);
    flat_dims(gammas);
  }
  if (c.biases.empty()) {
    c.biases.v.assign(means.v.size(), 0.0f);
    flat_dims(c.biases);
  }
  if (means.empty())
    return c;
  const size_t outputs = c.biases.v.size();
  if (stddivs.v.size() > outputs || stddivs.v.size() > gammas.v.size() ||
      stddivs.v.size() > means.v.size() ||
      gammas.v.size() < outputs || betas.v.size() < outputs || means.v.size() < outputs ||
      outputs == 0 || c.weights.v.size() % outputs)
    throw std::runtime_error("Inconsistent batch-norm sizes in convolution block");
  for (size_t i = 0; i < stddivs.v.size(); ++i) {
    const float inv = 1.0f / std::sqrt(stddivs.v[i] + 1e-5f);
    gammas.v[i] = gammas.v[i] * inv;
    means.v[i] = means.v[i] - c.biases.v[i];
  }
  const size_t inputs = c.weights.v.size() / outputs;
  for (size_t o = 0; o < outputs; ++o) {
    const float g = gammas.v[o];
    for (size_t k = 0; k < inputs; ++k)
      c.weights.v[o * inputs + k] = c.weights.v[o * inputs + k] * g;
    const float shifted = (-g) * means.v[o];
    c.biases.v[o] = shifted + betas.v[o];
  }
  return c;
}

// ---- inventory ---------------------------------------------------------------

// AddVector / TensorDims (reference network_weight_inventory.cpp:21-35):
// empty tensors are left out; a tensor without dims gets its flat size.
class Inventory {
public:
  explicit Inventory(std::vector<Tensor> *out) : out_(out) {}

  void Add(const std::string &name, Vec v) {
    if (v.empty())
      return;
    Tensor t;
    t.name = name;
    t.dims = v.dims.empty() ? std::vector<uint32_t>{static_cast<uint32_t>(v.v.size())}
                            : std::move(v.dims);
    t.data = std::move(v.v);
    out_->push_back(std::move(t));
  }

  void AddConv(const std::string &prefix, Conv c) {
    Add(prefix + ".weights", std::move(c.weights));
    Add(prefix + ".biases", std::move(c.biases));
  }

  // FFN message (net.proto:88-94), network_weight_inventory.cpp:89-99.
  void AddFfn(const std::string &prefix, const Message &ffn) {
    Add(prefix + ".dense1_w", LayerOf(ffn, 1));
    Add(prefix + ".dense1_b", LayerOf(ffn, 2));
    Add(prefix + ".dense2_w", LayerOf(ffn, 3));
    Add(prefix + ".dense2_b", LayerOf(ffn, 4));
  }

  // EncoderLayer (net.proto:96-103) with its MHA (70-86) and Smolgen
  // (57-68); network_weight_inventory.cpp:45-113.  RPE weights are refused
  // as in BaseWeights::MHA (weights.cpp:145-160).
  void AddEncoder(const std::string &prefix, const Message &layer) {
    const Message mha = layer.Sub(1);
    if (mha.Has(10) || mha.Has(11) || mha.Has(12))
      throw std::runtime_error("RPE weights file not supported.");
    static const char *const kMha[] = {"q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "dense_w",
                                       "dense_b"};
    for (uint32_t f = 1; f <= 8; ++f)
      Add(prefix + ".mha." + kMha[f - 1], LayerOf(mha, f));
    if (mha.Has(9)) {
      const Message sg = mha.Sub(9);
      static const char *const kSmolgen[] = {"compress",   "dense1_w", "dense1_b",
                                             "ln1_gammas", "ln1_betas", "dense2_w",
                                             "dense2_b",   "ln2_gammas", "ln2_betas"};
      for (uint32_t f = 1; f <= 9; ++f)
        Add(prefix + ".mha.smolgen." + kSmolgen[f - 1], LayerOf(sg, f));
    }
    Add(prefix + ".ln1_gammas", LayerOf(layer, 2));
    Add(prefix + ".ln1_betas", LayerOf(layer, 3));
    AddFfn(prefix + ".ffn", layer.Sub(4));
    Add(prefix + ".ln2_gammas", LayerOf(layer, 5));
    Add(prefix + ".ln2_betas", LayerOf(layer, 6));
  }

private:
  std::vector<Tensor> *out_;
};

// FixOlderWeightsFile (reference src/nn/loader.cpp:86-135) on the format
// fields, then the PE_MAP default of DescribeNetworkFormat
// (src/nn/network_format.cpp:97-100).
NetFormat ReadFormat(const Message &net, const Message &weights) {
  const Message format = net.Sub(4);
  const bool has_network_format = format.Has(2);
  const Message nf = format.Sub(2);
  NetFormat f;
  nf.Enum(1, kInputFormats, &f.input);
  nf.Enum(2, kOutputFormats, &f.output);
  nf.Enum(3, kNetworkStructures, &f.network);
  nf.Enum(4, kPolicyFormats, &f.policy);
  nf.Enum(5, kValueFormats, &f.value);
  nf.Enum(6, kMovesLeftFormats, &f.moves_left);
  nf.Enum(7, kDefaultActivations, &f.default_activation);
  nf.Enum(8, kActivations, &f.smolgen_activation);
  nf.Enum(9, kActivations, &f.ffn_activation);
  f.has_input_embedding = nf.Enum(10, kInputEmbeddings, &f.input_embedding);

  if (!has_network_format) {
    f.input = kInputClassical112;
    f.output = kOutputClassical;
    f.network = kNetClassicalHead;
    f.value = kValueClassical;
    f.policy = kPolicyClassical;
  }
  const int structure = f.network;
  if (structure == kNetClassical) {
    f.network = kNetClassicalHead;
    f.value = kValueClassical;
    f.policy = kPolicyClassical;
  } else if (structure == kNetSe) {
    f.network = kNetSeHead;
    f.value = kValueClassical;
    f.policy = kPolicyClassical;
  } else if (structure == kNetSeHead && weights.Has(F::kEncoder)) {
    f.network = kNetAttentionHead;
    if (weights.Has(F::kSmolgenW)) {
      f.ffn_activation = kActRelu2;
      f.smolgen_activation = kActSwish;
    }
  } else if (structure == kNetAbLegacyMultiHead) {
    f.network = kNetAttentionMultiHead;
  }
  if (f.network == kNetAttentionHead) {
    if (weights.Has(F::kPolicyHeads) && weights.Has(F::kValueHeads)) {
      f.network = kNetAttentionMultiHead;
      f.input_embedding = kEmbeddingPeDense;
      f.has_input_embedding = true;
    }
    if (!f.has_input_embedding) {
      f.input_embedding = kEmbeddingPeMap;
      f.has_input_embedding = true;
    }
  }
  if (!f.has_input_embedding)
    f.input_embedding = kEmbeddingPeMap;
  return f;
}

}  // namespace

// DecodeLayer (reference src/nn/loader.cpp:187-251): FLOAT32 is raw little-
// endian floats; FLOAT16 and BFLOAT16 widen exactly; LINEAR16 (also the
// reading of an unset encoding) maps a 16-bit code q to
// min + (q / 65535) * (max - min) in float arithmetic.
std::vector<float> DecodeLayer(int encoding, float min_val, float max_val,
                               const uint8_t *params, size_t bytes) {
  if (encoding == 0)
    encoding = 1;
  std::vector<float> out;
  if (encoding == 4) {
    out.resize(bytes / 4);
    if (!out.empty())
      std::memcpy(out.data(), params, out.size() * 4);
    return out;
  }
  if (encoding < 1 || encoding > 3)
    throw std::runtime_error("Unsupported weight encoding");
  const size_t n = bytes / 2;
  out.resize(n);
  const float range = max_val - min_val;
  for (size_t i = 0; i < n; ++i) {
    const uint32_t h = static_cast<uint32_t>(params[2 * i]) |
                       (static_cast<uint32_t>(params[2 * i + 1]) << 8);
    uint32_t bits;
    if (encoding == 1) {
      const float unit = static_cast<float>(h) / 65535.0f;
      const float scaled = unit * range;
      out[i] = min_val + scaled;
      continue;
    } else if (encoding == 3) {
      bits = h << 16;
    } else {
      // IEEE binary16 -> binary32: sign, 5-bit exponent (bias 15), 10-bit
      // fraction.  Subnormals are fraction * 2^-24, exact in binary32.
      const uint32_t sign = (h & 0x8000u) << 16;
      const uint32_t exponent = (h >> 10) & 0x1f, fraction = h & 0x3ff;
      if (exponent == 0) {
        const float mag = static_cast<float>(fraction) * 5.9604644775390625e-8f;  // 2^-24
        std::memcpy(&bits, &mag, 4);
        bits |= sign;
      } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (fraction << 13);
      } else {
        bits = sign | ((exponent + 112u) << 23) | (fraction << 13);
      }
    }
    std::memcpy(&out[i], &bits, 4);
  }
  return out;
}

Weights Parse(const uint8_t *data, size_t size) {
  const Message net(data, size);
  if (net.Fixed32(1) != kWeightMagic)
    throw std::runtime_error("Invalid weight file: bad magic number");
  const Message w = net.Sub(10);

  Weights out;
  out.format = ReadFormat(net, w);
  out.headcount = w.Uint32(F::kHeadcount);
  Inventory inv(&out.tensors);

  // Body (BaseWeights, weights.cpp:50-88; inventory order
  // network_weight_inventory.cpp:116-164).
  inv.AddConv("body.input", ConvBlockOf(w, F::kInput));
  inv.Add("body.ip_emb_preproc_w", LayerOf(w, F::kIpEmbPreprocW));
  inv.Add("body.ip_emb_preproc_b", LayerOf(w, F::kIpEmbPreprocB));
  inv.Add("body.ip_emb_w", LayerOf(w, F::kIpEmbW));
  inv.Add("body.ip_emb_b", LayerOf(w, F::kIpEmbB));
  inv.Add("body.ip_emb_ln_gammas", LayerOf(w, F::kIpEmbLnGammas));
  inv.Add("body.ip_emb_ln_betas", LayerOf(w, F::kIpEmbLnBetas));
  inv.Add("body.ip_mult_gate", LayerOf(w, F::kIpMultGate));
  inv.Add("body.ip_add_gate", LayerOf(w, F::kIpAddGate));
  inv.AddFfn("body.ip_emb_ffn", w.Sub(F::kIpEmbFfn));
  inv.Add("body.ip_emb_ffn_ln_gammas", LayerOf(w, F::kIpEmbFfnLnGammas));
  inv.Add("body.ip_emb_ffn_ln_betas", LayerOf(w, F::kIpEmbFfnLnBetas));
  inv.Add("body.smolgen_w", LayerOf(w, F::kSmolgenW));
  {
    const auto encoders = w.Each(F::kEncoder);
    for (size_t i = 0; i < encoders.size(); ++i)
      inv.AddEncoder("body.encoder." + std::to_string(i), encoders[i]);
  }
  {
    const auto residuals = w.Each(F::kResidual);
    for (size_t i = 0; i < residuals.size(); ++i) {
      const std::string prefix = "body.residual." + std::to_string(i);
      inv.AddConv(prefix + ".conv1", ConvBlockOf(residuals[i], 1));
      inv.AddConv(prefix + ".conv2", ConvBlockOf(residuals[i], 2));
      if (residuals[i].Has(3)) {
        const Message se = residuals[i].Sub(3);
        inv.Add(prefix + ".se.w1", LayerOf(se, 1));
        inv.Add(prefix + ".se.b1", LayerOf(se, 2));
        inv.Add(prefix + ".se.w2", LayerOf(se, 3));
        inv.Add(prefix + ".se.b2", LayerOf(se, 4));
      }
    }
  }

  // Policy head (MultiHeadWeights, weights.cpp:216-268).  The "vanilla" head
  // always exists, so it is the selected one (SelectPolicyHeadName,
  // network_format.cpp:143-145).  Its embedding falls back to the shared
  // PolicyHeads.ip_pol_w/b, or the top-level ip_pol_w/b; a file without
  // policy_heads takes the rest of the head from the legacy top-level
  // fields.
  {
    const Message heads = w.Sub(F::kPolicyHeads);
    const Message head = heads.Sub(3);
    Vec shared_w = LayerOf(heads.Has(1) ? heads : w, heads.Has(1) ? 1 : F::kIpPolW);
    Vec shared_b = LayerOf(heads.Has(2) ? heads : w, heads.Has(2) ? 2 : F::kIpPolB);
    Vec ip_w = LayerOf(head, 1), ip_b = LayerOf(head, 2);
    if (ip_w.empty())
      ip_w = std::move(shared_w);
    if (ip_b.empty())
      ip_b = std::move(shared_b);
    const std::string p = "policy.vanilla";
    out.policy_head = "vanilla";
    if (w.Has(F::kPolicyHeads)) {
      inv.AddConv(p + ".policy1", ConvBlockOf(head, 10));
      inv.AddConv(p + ".policy", ConvBlockOf(head, 11));
      inv.Add(p + ".ip_pol_w", std::move(ip_w));
      inv.Add(p + ".ip_pol_b", std::move(ip_b));
      inv.Add(p + ".ip2_pol_w", LayerOf(head, 3));
      inv.Add(p + ".ip2_pol_b", LayerOf(head, 4));
      inv.Add(p + ".ip3_pol_w", LayerOf(head, 5));
      inv.Add(p + ".ip3_pol_b", LayerOf(head, 6));
      inv.Add(p + ".ip4_pol_w", LayerOf(head, 7));
      const auto enc = head.Each(8);
      for (size_t i = 0; i < enc.size(); ++i)
        inv.AddEncoder(p + ".encoder." + std::to_string(i), enc[i]);
      out.pol_headcount = head.Uint32(9);
    } else if (w.Has(F::kPolicy) || w.Has(F::kPolicy1) || w.Has(F::kIpPolW)) {
      inv.AddConv(p + ".policy1", ConvBlockOf(w, F::kPolicy1));
      inv.AddConv(p + ".policy", ConvBlockOf(w, F::kPolicy));
      inv.Add(p + ".ip_pol_w", std::move(ip_w));
      inv.Add(p + ".ip_pol_b", std::move(ip_b));
      inv.Add(p + ".ip2_pol_w", LayerOf(w, F::kIp2PolW));
      inv.Add(p + ".ip2_pol_b", LayerOf(w, F::kIp2PolB));
      inv.Add(p + ".ip3_pol_w", LayerOf(w, F::kIp3PolW));
      inv.Add(p + ".ip3_pol_b", LayerOf(w, F::kIp3PolB));
      inv.Add(p + ".ip4_pol_w", LayerOf(w, F::kIp4PolW));
      const auto enc = w.Each(F::kPolEncoder);
      for (size_t i = 0; i < enc.size(); ++i)
        inv.AddEncoder(p + ".encoder." + std::to_string(i), enc[i]);
      out.pol_headcount = w.Uint32(F::kPolHeadcount);
    } else {
      throw std::runtime_error("Could not find valid policy head weights.");
    }
  }

  // Value head (weights.cpp:270-290): "winner" always exists and is selected
  // (SelectValueHeadName, network_format.cpp:147-149); without value_heads
  // it comes from the legacy top-level fields.
  {
    const std::string p = "value.winner";
    out.value_head = "winner";
    const Message head = w.Sub(F::kValueHeads).Sub(1);
    if (w.Has(F::kValueHeads)) {
      inv.AddConv(p + ".value", ConvBlockOf(head, 11));
      static const char *const kValue[] = {"ip_val_w",  "ip_val_b",  "ip1_val_w",
                                           "ip1_val_b", "ip2_val_w", "ip2_val_b",
                                           "ip_val_err_w", "ip_val_err_b"};
      for (uint32_t f = 1; f <= 8; ++f)
        inv.Add(p + "." + kValue[f - 1], LayerOf(head, f));
    } else if (w.Has(F::kValue) || w.Has(F::kIpValW)) {
      inv.AddConv(p + ".value", ConvBlockOf(w, F::kValue));
      inv.Add(p + ".ip_val_w", LayerOf(w, F::kIpValW));
      inv.Add(p + ".ip_val_b", LayerOf(w, F::kIpValB));
      inv.Add(p + ".ip1_val_w", LayerOf(w, F::kIp1ValW));
      inv.Add(p + ".ip1_val_b", LayerOf(w, F::kIp1ValB));
      inv.Add(p + ".ip2_val_w", LayerOf(w, F::kIp2ValW));
      inv.Add(p + ".ip2_val_b", LayerOf(w, F::kIp2ValB));
      inv.Add(p + ".ip_val_err_w", LayerOf(head, 7));
      inv.Add(p + ".ip_val_err_b", LayerOf(head, 8));
    } else {
      throw std::runtime_error("Could not find valid value head weights.");
    }
  }

  // Moves-left head when the format has one (network_weight_inventory.cpp:
  // 166-180, 350-351).
  if (out.format.moves_left == kMovesLeftV1) {
    inv.AddConv("moves_left", ConvBlockOf(w, F::kMovesLeft));
    inv.Add("moves_left.ip_mov_w", LayerOf(w, F::kIpMovW));
    inv.Add("moves_left.ip_mov_b", LayerOf(w, F::kIpMovB));
    inv.Add("moves_left.ip1_mov_w", LayerOf(w, F::kIp1MovW));
    inv.Add("moves_left.ip1_mov_b", LayerOf(w, F::kIp1MovB));
    inv.Add("moves_left.ip2_mov_w", LayerOf(w, F::kIp2MovW));
    inv.Add("moves_left.ip2_mov_b", LayerOf(w, F::kIp2MovB));
  }
  return out;
}

// LoadWeightsFromFile (reference src/nn/loader.cpp:37-84, 162-185).
Weights LoadFile(const std::string &path) {
  std::vector<uint8_t> buffer;
  if (path.size() >= 3 && path.compare(path.size() - 3, 3, ".gz") == 0) {
    gzFile file = gzopen(path.c_str(), "rb");
    if (!file)
      throw std::runtime_error("Cannot read weights from " + path);
    size_t used = 0;
    buffer.resize(8u << 20);
    while (true) {
      if (buffer.size() - used < (1u << 20))
        buffer.resize(buffer.size() * 2);
      const unsigned want = static_cast<unsigned>(std::min<size_t>(buffer.size() - used, 1u << 30));
      const int got = gzread(file, buffer.data() + used, want);
      if (got < 0) {
        int errnum = 0;
        const char *msg = gzerror(file, &errnum);
        const std::string detail = msg ? msg : "unknown gzip error";
        gzclose(file);
        throw std::runtime_error("gzip error reading file: " + detail);
      }
      if (got == 0)
        break;
      used += static_cast<size_t>(got);
    }
    gzclose(file);
    buffer.resize(used);
  } else {
    std::ifstream in(path, std::ios::binary);
    if (!in)
      throw std::runtime_error("Cannot read weights from " + path);
    buffer.assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
  }
  if (buffer.size() < 2)
    throw std::runtime_error("Invalid weight file: too small");
  return Parse(buffer.data(), buffer.size());
}

}  // namespace wf
}  // namespace mfh
