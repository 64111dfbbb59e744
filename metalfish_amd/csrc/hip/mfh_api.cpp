// C ABI of libmfhip.so (include/mfhip.h): shape inference, weight packing,
// device arenas and the per-batch launch sequence of the transformer
// forward pass on one MI355X.
//
// The launch sequence restates the step order of the reference CPU backend
// for attention-body nets (reference src/nn/network_execution_plan.cpp:
// 94-223 and src/nn/cpu/cpu_network.cpp:580-1491) with these fusions:
//   * Q, K, V and the smolgen compression are one GEMM (one read of X);
//   * the policy "output" dense and the value "output" dense share one GEMM;
//   * the policy query and key denses (both fed by "output", reference
//     cpu_network.cpp:570-573, 871-875) are one GEMM;
//   * bias, activations and the scaled residual add run in GEMM epilogues,
//     the input gates in the LayerNorm kernel.
#include "../../../include/mfhip.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <set>
#include <sstream>
#include <string>
#include <tuple>
#include <stdexcept>
#include <vector>

#include "../host/policy_tables.h"
#include "../host/weights_file.h"
#include "mfh_kernels.h"

// Device memory of mfh_net_eval_device_noalloc: the workspace of one small
// forward (activations, split-K partials, smolgen bias) for callers that
// cannot allocate.  Every device the library runs on holds its own copy until
// the process ends; host code reaches it only through the address
// hipGetSymbolAddress gives on that device (ScratchAddress below).
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

thread_local std::string g_last_error;

int SetError(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

#define MFH_HIP_CHECK(expr)                                                    \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess)                                                      \
      return SetError(MFH_ERR_HIP, std::string(#expr) + ": " +                 \
                                       hipGetErrorString(e_));                 \
  } while (0)

// Device address of `scratch` on each device, resolved once per device with
// that device current (mfh_net_create); null until then.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char *g_scratch_addr[kMaxDevices] = {};

int ResolveScratch(int dev) {
  if (dev < 0 || dev >= kMaxDevices)
    return SetError(MFH_ERR_NO_DEVICE, "device ordinal beyond the scratch address table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev])
    return MFH_OK;
  void *addr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !addr)
    return SetError(MFH_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") +
                                     hipGetErrorString(e));
  g_scratch_addr[dev] = static_cast<unsigned char *>(addr);
  return MFH_OK;
}

unsigned char *ScratchAddress(int dev) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return dev >= 0 && dev < kMaxDevices ? g_scratch_addr[dev] : nullptr;
}

constexpr int kSquares = 64;
constexpr int kMaxMoves = 256;  // edges per node (reference src/mcts/search.cpp:49)
constexpr int kPlanes = 112;
constexpr int kPolicy = 1858;
// Largest batch whose smolgen dense1 / dense2 run as few-row GEMMs: forward
// 1.513 -> 1.434 ms at batch 2, 1.662 -> 1.586 at 4, 1.673 -> 1.625 at 8,
// 2.097 -> 2.071 at 16; from 24 up it was slower (batch 32 2.58 -> 2.78:
// every workgroup of dense1 reads all the positions' compression rows).
constexpr int kSmolgenFewRowMaxBatch = 16;
// Token rows from which each layer's smolgen chain runs on the second stream
// beside Q|K|V (its compression then a GEMM of its own): past the few-row
// batches, from 17 positions (forward at batch 24 2.57 -> 2.47 ms, 28 2.72
// -> 2.59, 20 2.31 -> 2.29; with the few-row chain at 16 positions it was
// slower, 2.07 -> 2.19).
constexpr int kSmolgenSideRows = 1088;

// BF16X2_FP8LO: the fp8 lo correction runs from this many token rows (128
// positions); below, the forward is the BF16X2 one.
constexpr int kLo8MinRows = 8192;
// From this many token rows (256 positions) the body's residual LayerNorms
// are folded into the GEMMs around them (GemmParams: the residual GEMMs write
// x o gamma with per-row partial sums, Q|K|V, the compression and FFN1 take
// the LayerNorm in their epilogue, the next residual rebuilds it), where
// the residual GEMMs (N = E) take whole rounds of 256 x 256 tiles.
constexpr long kFoldRows = 16384;
// From this many token rows (24 positions), while the residual GEMMs take
// 64 x 64 tiles over the whole K (up to 62 positions at E = 1024), the same
// folds run on those tiles (partial sums per 64 columns): LN1 (out-projection -> FFN1 and FFN2) and LN2 (FFN2
// -> Q|K|V on 256 x 128 tiles, the compression split over K with the
// LayerNorm applied by its reduce, and the next out-projection).
constexpr long kFoldLn1Rows = 1536;

std::uint16_t ToBf16(float f) {
  std::uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<std::uint16_t>(u >> 16);
}

// OCP e4m3 (bias 7, no infinities, 0x7F = NaN, largest finite 448) of a
// finite x, rounding to nearest even and saturating at +-448.
std::uint8_t EncodeE4m3(float x) {
  std::uint32_t u;
  std::memcpy(&u, &x, 4);
  const std::uint8_t sign = static_cast<std::uint8_t>((u >> 24) & 0x80u);
  u &= 0x7FFFFFFFu;
  float a;
  std::memcpy(&a, &u, 4);
  std::uint8_t code;
  if (a < 0.015625f) {  // below 2^-6: subnormal codes m * 2^-9, m = 0..8
    code = static_cast<std::uint8_t>(std::nearbyint(a * 512.0f));
  } else {
    // Keep 3 mantissa bits with round-to-nearest-even on the fp32 pattern.
    const std::uint32_t r = u + 0x7FFFFu + ((u >> 20) & 1u);
    const int e = static_cast<int>(r >> 23) - 127;
    const int m = static_cast<int>((r >> 20) & 7u);
    code = e > 8 || (e == 8 && m == 7) ? 0x7E : static_cast<std::uint8_t>(((e + 7) << 3) | m);
  }
  return static_cast<std::uint8_t>(sign | code);
}

// Row scale max|row| / 448 (1 for an all-zero row) and e4m3 codes of
// row / scale.
void QuantizeRowE4m3(const float *row, int n, std::uint8_t *codes, float *scale) {
  float mx = 0.f;
  for (int i = 0; i < n; ++i)
    mx = std::fmax(mx, std::fabs(row[i]));
  const float s = mx > 0.f ? mx / 448.0f : 1.0f;
  for (int i = 0; i < n; ++i)
    codes[i] = EncodeE4m3(row[i] / s);
  *scale = s;
}

// Value of an OCP e4m3 code (finite codes only).
float DecodeE4m3(std::uint8_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  const float v = e ? std::ldexp(1.0f + m / 8.0f, e - 7) : std::ldexp(static_cast<float>(m), -9);
  return (c & 0x80) ? -v : v;
}

int ActFromProto(int proto_act, int default_act) {
  switch (proto_act) {
  case MFH_ACTIVATION_DEFAULT: return default_act;
  case MFH_ACTIVATION_MISH: return mfh::ACT_MISH;
  case MFH_ACTIVATION_RELU: return mfh::ACT_RELU;
  case MFH_ACTIVATION_NONE: return mfh::ACT_NONE;
  case MFH_ACTIVATION_TANH: return mfh::ACT_TANH;
  case MFH_ACTIVATION_SIGMOID: return mfh::ACT_SIGMOID;
  case MFH_ACTIVATION_SELU: return mfh::ACT_SELU;
  case MFH_ACTIVATION_SWISH: return mfh::ACT_SWISH;
  case MFH_ACTIVATION_RELU_2: return mfh::ACT_RELU2;
  default: return mfh::ACT_RELU;
  }
}

const char *ActName(int act) {
  switch (act) {
  case mfh::ACT_NONE: return "none";
  case mfh::ACT_RELU: return "relu";
  case mfh::ACT_RELU2: return "relu_2";
  case mfh::ACT_TANH: return "tanh";
  case mfh::ACT_SIGMOID: return "sigmoid";
  case mfh::ACT_SWISH: return "swish";
  case mfh::ACT_MISH: return "mish";
  case mfh::ACT_SELU: return "selu";
  default: return "?";
  }
}

size_t AlignUp(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Host-side staging of the packed weight blob before one upload.
struct Blob {
  std::vector<unsigned char> bytes;
  size_t Add(const void *src, size_t n) {
    const size_t off = AlignUp(bytes.size(), 256);
    bytes.resize(off + n);
    if (src)
      std::memcpy(bytes.data() + off, src, n);
    return off;
  }
};

struct Layer {
  size_t qkv_b, out_b, ln1_g, ln1_b, ffn1_b, ffn2_b, ln2_g, ln2_b;
  size_t qkv_w[2], out_w[2], ffn1_w[2], ffn2_w[2];  // {weights, fp8 row scales}
  bool smolgen = false;
  size_t sg_d1_b, sg_ln1_g, sg_ln1_b, sg_d2_b, sg_ln2_g, sg_ln2_b;
  size_t sg_d1_w[2], sg_d2_w[2];
  // Folded LayerNorms (see kFoldRows): {fold_c, bias'} of the Q|K|V (+
  // compression) rows over the previous layer's LN2, and of FFN1 over LN1.
  size_t qkv_fold[2] = {0, 0}, ffn1_fold[2] = {0, 0};
};

struct Dims {
  int E = 0, H = 0, L = 0, F = 0, P = 0, Kin = 0, Fi = 0;
  int C = 0, Hs = 0, HG = 0, G = 0;
  int Dp = 0, Vd = 0, Vh = 0, Vout = 0;
  int Md = 0, Mh = 0;  // moves-left head: square embedding, hidden width
  int PL = 0, PH = 0, PF = 0;  // policy encoder layers: count, heads, FFN width
  bool gates = false, input_ffn = false, smolgen = false, wdl = true, mlh = false;
  bool pe_map = false;  // static position encoding (INPUT_EMBEDDING_PE_MAP)
  float eps_emb = 1e-3f;  // input-embedding LayerNorm
  bool split = false;       // lo planes on dense-layer inputs (BF16X2, BF16X2_GEMM)
  bool split_attn = false;  // lo planes on attention / smolgen operands (BF16X2)
  bool fused_ln = false;    // residual GEMM + LayerNorm as one row-panel launch
  bool fused_bias = false;  // smolgen bias generated inside the attention kernel
  bool skinny = true;       // few-row GEMMs for single-position forwards
  bool fold_ln = true;      // the body's residual LayerNorms folded (kFoldRows)
  bool fp8_act = false;     // e4m3 activations on the fp8 MFMA (FP8 precision)
  bool lo8 = false;         // BF16X2_FP8LO: e4m3 lo parts on the fp8 MFMA
  int act_default = mfh::ACT_MISH, act_ffn = mfh::ACT_MISH, act_smolgen = mfh::ACT_SWISH;
  float alpha = 1.f, eps_body = 1e-3f;
};

}  // namespace

// A decoded network file and the C views of its tensors.
struct mfh_weights {
  mfh::wf::Weights w;
  std::vector<mfh_tensor> views;
};

struct mfh_net {
  std::mutex mu;
  int device = 0;
  hipStream_t stream = nullptr;
  Dims d;
  int max_batch = 0;
  std::string arch, device_name;

  unsigned char *weights = nullptr;
  size_t weight_bytes = 0;
  // Offsets into `weights`.
  // GEMM weights are {offset, fp8 row-scale offset} pairs.
  bool fp8 = false;
  size_t pre_b, emb_b, emb_ln_g, emb_ln_b, mult_gate, add_gate;
  size_t static_pe = 0;  // PE_MAP table, fp32 [64][64]
  size_t pre_w[2], emb_w[2], in_ffn1_w[2], in_ffn2_w[2], global_w[2];
  size_t in_ffn1_b, in_ffn2_b, in_ln_g, in_ln_b;
  std::vector<Layer> layers;
  std::vector<Layer> pol_layers;  // policy encoder layers
  // BF16X2_FP8LO: offset of a dense weight's W' (bf16, with column scales) ->
  // offset of its e4m3 codes.
  std::map<size_t, size_t> lo8_codes;
  // The body's fold constants were packed (Layer::qkv_fold / ffn1_fold),
  // for kFoldRows (has_fold) or kFoldLn1Rows (has_fold1) token rows.
  bool has_fold = false, has_fold1 = false;
  size_t head_b, qk_b, promo, val1_b, val2_w, val2_b, gather;
  size_t head_w[2], qk_w[2], val1_w[2];
  size_t mov_b = 0, mov1_b = 0, mov2_w = 0, mov2_b = 0;  // moves-left head
  size_t mov_w[2] = {0, 0}, mov1_w[2] = {0, 0};

  unsigned char *ws = nullptr;
  size_t ws_bytes = 0;
  std::map<std::string, size_t> ws_off;
  // Workspace layout of mfh_net_eval_device_noalloc inside the scratch
  // array, for batches up to noalloc_max_batch (0: the net does not fit).
  std::map<std::string, size_t> noalloc_off;
  size_t noalloc_bytes = 0;
  int noalloc_max_batch = 0;
  bool noalloc_call = false;  // set during that call: no profiler events

  // Recorded after the last work that touched the workspace, on whatever
  // stream it ran; every call waits on it before its own work.  The
  // workspace is shared, so calls on different streams (mfh_net_eval on the
  // net's stream, mfh_net_eval_device on a caller's) run one after another.
  hipEvent_t last_use = nullptr;

  unsigned char *pin_in = nullptr;   // masks | values | move offsets | move indices
  unsigned char *pin_out = nullptr;  // policy | value
  int last_batch = 0;

  // Stage profiler.
  struct Pending {
    std::string name;
    double flops, bytes;
    hipEvent_t start, stop;
  };
  struct Totals {
    int launches = 0;
    double ms = 0, flops = 0, bytes = 0;
  };
  bool profiling = false;
  std::vector<Pending> pending;
  // Forward graphs, keyed by batch size and the four device buffers; a key
  // runs eagerly once before it is captured.
  struct GraphKey {
    int batch;
    const void *masks, *values, *policy, *wdl, *moves_left;
    bool operator<(const GraphKey &o) const {
      return std::tie(batch, masks, values, policy, wdl, moves_left) <
             std::tie(o.batch, o.masks, o.values, o.policy, o.wdl, o.moves_left);
    }
  };
  bool graphs = true;
  hipStream_t capture_stream = nullptr;
  // Second stream of the forward: each encoder layer's smolgen chain
  // (compression .. global projection) runs on it while Q|K|V runs on the
  // main stream; fork / join events per layer (two each).
  hipStream_t side = nullptr;
  std::vector<hipEvent_t> fork_join;
  std::map<GraphKey, hipGraphExec_t> graph_execs;
  std::set<GraphKey> graph_warm;
  std::vector<hipEvent_t> event_pool;
  std::map<std::string, Totals> totals;

  template <typename T> T *W(size_t off) const {
    return reinterpret_cast<T *>(weights + off);
  }
  template <typename T> T *S(const std::string &name) const {
    return reinterpret_cast<T *>(ws + ws_off.at(name));
  }
  // Residual plane of a bf16 activation, or null in single precision.
  std::uint16_t *Lo(const std::string &name) const {
    auto it = ws_off.find(name + "_lo");
    return it == ws_off.end() ? nullptr : reinterpret_cast<std::uint16_t *>(ws + it->second);
  }
};

namespace {

struct TensorMap {
  std::map<std::string, const mfh_tensor *> by_name;
  const mfh_tensor *Get(const std::string &n) const {
    auto it = by_name.find(n);
    return it == by_name.end() ? nullptr : it->second;
  }
};

// Reads a tensor of the given size; *ok cleared with a message if absent or
// mis-sized.
struct Loader {
  const TensorMap &tm;
  std::string error;
  const float *Need(const std::string &name, size_t count) {
    const mfh_tensor *t = tm.Get(name);
    if (!t) {
      if (error.empty())
        error = "missing tensor " + name;
      return nullptr;
    }
    if (t->count != count || !t->data) {
      if (error.empty()) {
        std::ostringstream o;
        o << "tensor " << name << " has " << t->count << " values, expected " << count;
        error = o.str();
      }
      return nullptr;
    }
    return t->data;
  }
  size_t Count(const std::string &name) const {
    const mfh_tensor *t = tm.Get(name);
    return t ? static_cast<size_t>(t->count) : 0;
  }
};

// Appends rows x cols fp32 (row-major) as bf16 padded to ld columns.
size_t AddBf16(Blob &blob, const std::vector<const float *> &parts,
               const std::vector<int> &part_rows, int cols, int ld) {
  size_t rows = 0;
  for (int r : part_rows)
    rows += r;
  std::vector<std::uint16_t> buf(rows * ld, 0);
  size_t row = 0;
  for (size_t p = 0; p < parts.size(); ++p) {
    for (int r = 0; r < part_rows[p]; ++r, ++row)
      for (int c = 0; c < cols; ++c)
        buf[row * ld + c] = parts[p] ? ToBf16(parts[p][static_cast<size_t>(r) * cols + c]) : 0;
  }
  return blob.Add(buf.data(), buf.size() * 2);
}

// A GEMM weight in the blob: bf16 [rows][ld], or e4m3 codes [rows][ld]
// plus fp32 row scales at `s`.
struct GemmW {
  size_t w = 0, s = 0;
};

GemmW AddGemmW(Blob &blob, bool fp8, const std::vector<const float *> &parts,
               const std::vector<int> &part_rows, int cols, int ld) {
  if (!fp8)
    return GemmW{AddBf16(blob, parts, part_rows, cols, ld), 0};
  size_t rows = 0;
  for (int r : part_rows)
    rows += r;
  std::vector<std::uint8_t> codes(rows * ld, 0);
  std::vector<float> scales(rows, 1.0f);
  std::vector<float> tmp(ld);
  size_t row = 0;
  for (size_t p = 0; p < parts.size(); ++p) {
    for (int r = 0; r < part_rows[p]; ++r, ++row) {
      std::fill(tmp.begin(), tmp.end(), 0.f);
      if (parts[p])
        std::memcpy(tmp.data(), parts[p] + static_cast<size_t>(r) * cols, cols * 4);
      QuantizeRowE4m3(tmp.data(), ld, codes.data() + row * ld, &scales[row]);
    }
  }
  GemmW g;
  g.w = blob.Add(codes.data(), codes.size());
  g.s = blob.Add(scales.data(), scales.size() * 4);
  return g;
}

// A GEMM weight of the BF16X2_FP8LO precision: for each output row n a
// scale s_n, the row times 2^kLo8Shift / s_n as bf16 (W'), the e4m3 codes of
// the row / s_n (W8, the fp8 lo-correction operand) and cs_n = s_n /
// 2^kLo8Shift (the GEMM's column scale), so that (hi . W'_n + lo8 . W8_n)
// cs_n = hi . W_n + lo . W_n up to the e4m3 rounding of the lo product.
// bf16 weights: s_n is the power of two with max|W_n| / s_n in (224, 448],
// so W' is exact.  fp8 weights: the codes and row scale of AddGemmW, and W'
// the codes' values times 2^kLo8Shift (exact in bf16).  Returns {W', cs}
// and the codes' offset in *codes.
GemmW AddGemmWLo8(Blob &blob, bool fp8, const std::vector<const float *> &parts,
                  const std::vector<int> &part_rows, int cols, int ld, size_t *codes_off) {
  size_t rows = 0;
  for (int r : part_rows)
    rows += r;
  std::vector<std::uint16_t> wp(rows * ld, 0);
  std::vector<std::uint8_t> codes(rows * ld, 0);
  std::vector<float> cs(rows, 1.0f);
  std::vector<float> tmp(ld);
  const float lo_scale = static_cast<float>(1 << mfh::kLo8Shift);
  size_t row = 0;
  for (size_t p = 0; p < parts.size(); ++p) {
    for (int r = 0; r < part_rows[p]; ++r, ++row) {
      std::fill(tmp.begin(), tmp.end(), 0.f);
      if (parts[p])
        std::memcpy(tmp.data(), parts[p] + static_cast<size_t>(r) * cols, cols * 4);
      std::uint8_t *c = codes.data() + row * ld;
      std::uint16_t *w = wp.data() + row * ld;
      if (fp8) {
        float ws = 1.f;
        QuantizeRowE4m3(tmp.data(), ld, c, &ws);
        for (int i = 0; i < ld; ++i)
          w[i] = ToBf16(DecodeE4m3(c[i]) * lo_scale);
        cs[row] = ws / lo_scale;
      } else {
        float mx = 0.f;
        for (int i = 0; i < ld; ++i) {
          std::uint16_t b = ToBf16(tmp[i]);
          const std::uint32_t u = static_cast<std::uint32_t>(b) << 16;
          std::memcpy(&tmp[i], &u, 4);
          mx = std::fmax(mx, std::fabs(tmp[i]));
        }
        const float sc = mx > 0.f ? std::ldexp(1.0f, static_cast<int>(std::ceil(
                                                       std::log2(mx / 448.0f))))
                                  : 1.0f;
        for (int i = 0; i < ld; ++i) {
          c[i] = EncodeE4m3(tmp[i] / sc);
          w[i] = ToBf16(tmp[i] * (lo_scale / sc));
        }
        cs[row] = sc / lo_scale;
      }
    }
  }
  GemmW g;
  g.w = blob.Add(wp.data(), wp.size() * 2);
  g.s = blob.Add(cs.data(), cs.size() * 4);
  *codes_off = blob.Add(codes.data(), codes.size());
  return g;
}

size_t AddF32(Blob &blob, const std::vector<const float *> &parts,
              const std::vector<int> &counts) {
  std::vector<float> buf;
  for (size_t p = 0; p < parts.size(); ++p)
    for (int i = 0; i < counts[p]; ++i)
      buf.push_back(parts[p] ? parts[p][i] : 0.f);
  return blob.Add(buf.data(), buf.size() * 4);
}

int Infer(const mfh_net_desc &desc, Loader &ld, Dims &d) {
  if (desc.network != MFH_NETWORK_ATTENTIONBODY_WITH_HEADFORMAT &&
      desc.network != MFH_NETWORK_ATTENTIONBODY_WITH_MULTIHEADFORMAT)
    return SetError(MFH_ERR_UNSUPPORTED, "HIP backend supports attention-body nets only");
  if (desc.policy != MFH_POLICY_ATTENTION)
    return SetError(MFH_ERR_UNSUPPORTED, "HIP backend supports the attention policy head only");
  if (desc.value != MFH_VALUE_WDL && desc.value != MFH_VALUE_CLASSICAL)
    return SetError(MFH_ERR_UNSUPPORTED, "HIP backend supports WDL or classical value heads");
  if (desc.moves_left != 0 && desc.moves_left != 1)
    return SetError(MFH_ERR_UNSUPPORTED, "unknown moves-left format (MOVES_LEFT_V1 or none)");
  if (desc.input_embedding != MFH_INPUT_EMBEDDING_PE_DENSE &&
      desc.input_embedding != MFH_INPUT_EMBEDDING_PE_MAP)
    return SetError(MFH_ERR_UNSUPPORTED,
                    "HIP backend supports the PE_DENSE and PE_MAP input embeddings");
  if (desc.weights_dtype != MFH_WEIGHTS_BF16 && desc.weights_dtype != MFH_WEIGHTS_FP8)
    return SetError(MFH_ERR_UNSUPPORTED, "unsupported weight storage type");
  if (desc.precision != MFH_PRECISION_BF16 && desc.precision != MFH_PRECISION_BF16X2 &&
      desc.precision != MFH_PRECISION_BF16X2_GEMM && desc.precision != MFH_PRECISION_FP8 &&
      desc.precision != MFH_PRECISION_BF16X2_FP8LO)
    return SetError(MFH_ERR_UNSUPPORTED, "unsupported precision mode");
  if (desc.precision == MFH_PRECISION_FP8 && desc.weights_dtype != MFH_WEIGHTS_FP8)
    return SetError(MFH_ERR_UNSUPPORTED, "the FP8 precision needs FP8 (e4m3) weights");
  d.fp8_act = desc.precision == MFH_PRECISION_FP8;
  d.lo8 = desc.precision == MFH_PRECISION_BF16X2_FP8LO;
  d.split = desc.precision == MFH_PRECISION_BF16X2 ||
            desc.precision == MFH_PRECISION_BF16X2_GEMM || d.lo8;
  d.split_attn = desc.precision == MFH_PRECISION_BF16X2 || d.lo8;
  // Measured at the BT4 shape: the panel wins with e4m3 weights (half the
  // weight bytes to stream; batch 1024 22.29k against 22.09k positions/s
  // for the tiled GEMM + LayerNorm, batch 256 even), the tiled GEMM +
  // LayerNorm kernel with bf16.  The panel has no fp8 lo correction:
  // BF16X2_FP8LO keeps the tiled GEMM.
  d.fused_ln = !d.lo8 && (desc.fused_layernorm != 0 || desc.weights_dtype == MFH_WEIGHTS_FP8);
  d.wdl = desc.value == MFH_VALUE_WDL;
  d.mlh = desc.moves_left == 1;
  d.act_default = desc.default_activation == MFH_DEFAULT_ACTIVATION_MISH ? mfh::ACT_MISH
                                                                         : mfh::ACT_RELU;
  d.act_ffn = ActFromProto(desc.ffn_activation, d.act_default);
  d.act_smolgen = ActFromProto(desc.smolgen_activation, d.act_default);

  // Shapes follow from bias sizes, as in the reference's shape inference
  // (network_execution_plan.cpp:279-289).
  d.E = static_cast<int>(ld.Count("body.ip_emb_b"));
  d.pe_map = desc.input_embedding == MFH_INPUT_EMBEDDING_PE_MAP;
  // PE_MAP: the static encoding's width is what the embedding dense takes
  // beyond the 112 planes (network_execution_plan.cpp:833-865).
  d.P = d.pe_map ? (d.E ? static_cast<int>(ld.Count("body.ip_emb_w") / d.E) - kPlanes : 0)
                 : static_cast<int>(ld.Count("body.ip_emb_preproc_b")) / kSquares;
  d.H = desc.headcount;
  while (ld.Count("body.encoder." + std::to_string(d.L) + ".mha.q_b"))
    ++d.L;
  d.F = d.L ? static_cast<int>(ld.Count("body.encoder.0.ffn.dense1_b")) : 0;
  d.Fi = static_cast<int>(ld.Count("body.ip_emb_ffn.dense1_b"));
  d.input_ffn = d.Fi > 0;
  d.gates = ld.Count("body.ip_mult_gate") || ld.Count("body.ip_add_gate");
  d.C = d.L ? static_cast<int>(ld.Count("body.encoder.0.mha.smolgen.compress")) /
                  (d.E ? d.E : 1)
            : 0;
  d.smolgen = d.C > 0;
  if (d.smolgen) {
    d.Hs = static_cast<int>(ld.Count("body.encoder.0.mha.smolgen.dense1_b"));
    d.HG = static_cast<int>(ld.Count("body.encoder.0.mha.smolgen.dense2_b"));
    d.G = d.H ? d.HG / d.H : 0;
  }
  d.Dp = static_cast<int>(ld.Count("policy.vanilla.ip2_pol_b"));
  d.Vd = static_cast<int>(ld.Count("value.winner.ip_val_b"));
  d.Vh = static_cast<int>(ld.Count("value.winner.ip1_val_b"));
  d.Vout = static_cast<int>(ld.Count("value.winner.ip2_val_b"));
  int mout = 0;
  if (d.mlh) {
    d.Md = static_cast<int>(ld.Count("moves_left.ip_mov_b"));
    d.Mh = static_cast<int>(ld.Count("moves_left.ip1_mov_b"));
    mout = static_cast<int>(ld.Count("moves_left.ip2_mov_b"));
  }
  d.Kin = static_cast<int>(AlignUp(kPlanes + d.P, 64));

  std::ostringstream why;
  if (d.E <= 0 || d.P <= 0)
    why << "missing input embedding (body.ip_emb_*, body.ip_emb_preproc_*); ";
  if (d.pe_map && d.P != mfh_policy::kPosEncodingChannels)
    why << "PE_MAP embedding input must be 112 + " << mfh_policy::kPosEncodingChannels
        << " wide; ";
  if (d.pe_map && ld.Count("body.ip_emb_preproc_w"))
    why << "PE_MAP nets carry no dynamic PE weights; ";
  if (d.E % 64)
    why << "embedding width " << d.E << " is not a multiple of 64; ";
  if (d.H <= 0 || d.E != d.H * 32)
    why << "head depth must be 32 (embedding " << d.E << ", heads " << d.H << "); ";
  if (d.H % 4)
    why << "head count must be a multiple of 4; ";
  if (d.L && d.F % 64)
    why << "FFN width must be a multiple of 64; ";
  if (d.input_ffn && d.Fi % 64)
    why << "input FFN width must be a multiple of 64; ";
  if (d.smolgen && (d.Hs % 64 || d.G % 64 || d.HG != d.G * d.H || d.C % 8))
    why << "smolgen widths must be multiples of 64 with dense2 = heads x gen; ";
  if (d.Dp <= 0 || d.Dp % 64)
    why << "policy width must be a positive multiple of 64; ";
  if (d.Vd <= 0 || d.Vh <= 0 || d.Vout != (d.wdl ? 3 : 1))
    why << "value head needs ip_val, ip1_val and ip2_val with " << (d.wdl ? 3 : 1)
        << " outputs; ";
  if (!ld.Count("body.ip_emb_ln_gammas"))
    why << "body.ip_emb_ln is required; ";
  if (ld.Count("policy.vanilla.ip_pol_b") == 0)
    why << "policy head needs ip_pol/ip2_pol/ip3_pol/ip4_pol; ";
  while (ld.Count("policy.vanilla.encoder." + std::to_string(d.PL) + ".mha.q_b"))
    ++d.PL;
  if (d.PL) {
    d.PH = desc.pol_headcount;
    d.PF = static_cast<int>(ld.Count("policy.vanilla.encoder.0.ffn.dense1_b"));
    if (d.PH <= 0 || d.E != d.PH * 32 || d.PH % 4)
      why << "policy encoder head depth must be 32 with a multiple of 4 heads (embedding "
          << d.E << ", heads " << d.PH << "); ";
    if (d.PF <= 0 || d.PF % 64)
      why << "policy encoder FFN width must be a positive multiple of 64; ";
    if (ld.Count("policy.vanilla.encoder.0.mha.smolgen.compress"))
      why << "policy encoder layers with smolgen are not supported; ";
  }
  // The value-error head (value.winner.ip_val_err_*) feeds no NetworkOutput
  // field (reference network_output_decoder.cpp:31-78), so it is accepted and
  // not computed.
  if (d.mlh && (d.Md <= 0 || d.Mh <= 0 || mout != 1 || ld.Count("moves_left.weights")))
    why << "moves-left head needs ip_mov, ip1_mov and ip2_mov (one output), no convolution; ";
  const std::string w = why.str();
  if (!w.empty())
    return SetError(MFH_ERR_UNSUPPORTED, "HIP backend cannot run this net: " + w);
  const int n_layers = d.L;
  d.alpha = std::pow(2.0f * static_cast<float>(n_layers), -0.25f);
  if (n_layers == 0)
    d.alpha = 1.0f;
  // LayerNorm epsilons (network_execution_plan.cpp:1164-1193): encoder
  // 1e-3 for PE_DENSE nets, 1e-6 otherwise; the embedding norm 1e-3 for
  // PE_DENSE, 1e-5 otherwise.
  d.eps_body = d.pe_map ? 1e-6f : 1e-3f;
  d.eps_emb = d.pe_map ? 1e-5f : 1e-3f;
  // Smolgen bias: by default the global projection runs as a GEMM into a
  // [B, H, 64, 64] bias tensor that attention reads (measured faster on
  // MI355X at every batch size: the in-kernel form streams the whole global
  // projection matrix from L2 for every 16 (position, head) pairs).  With
  // METALFISH_HIP_SMOLGEN_BIAS=attention the attention kernel generates the
  // bias itself (gen widths 64, 128 or 256) and no bias tensor exists.
  const char *bias_env = std::getenv("METALFISH_HIP_SMOLGEN_BIAS");
  d.fused_bias = d.smolgen && !d.lo8 && bias_env && std::string(bias_env) == "attention" &&
                 (d.G == 64 || d.G == 128 || d.G == 256) &&
                 mfh::AttentionSmolgenLds(d.G, d.split_attn) <= 160 * 1024;
  // Single-position forward with few-row GEMMs and deferred LayerNorms (on
  // unless METALFISH_HIP_SKINNY=0, which keeps the split-K path at batch 1).
  const char *skinny_env = std::getenv("METALFISH_HIP_SKINNY");
  d.skinny = !(skinny_env && skinny_env[0] == '0');
  // The body's residual LayerNorms folded into the GEMMs around them from
  // kFoldRows (on unless METALFISH_HIP_FOLD_LN=0).  The folded GEMMs work on
  // x o gamma and subtract mu (W . gamma) after the product, so the rounding
  // of the stored rows counts relative to |x| rather than to |x - mu|: a
  // row whose mean is large against its spread loses that factor.
  const char *fold_env = std::getenv("METALFISH_HIP_FOLD_LN");
  d.fold_ln = !(fold_env && fold_env[0] == '0');
  // BF16X2_FP8LO: the lo pass of the encoder GEMMs takes 128-byte K steps
  // over code rows laid out 128-byte aligned (K = the embedding and FFN
  // widths, in the body, the input-embedding FFN and policy encoder layers).
  if (d.lo8) {
    for (const int w : {d.E, d.F, d.input_ffn ? d.Fi : d.E, d.PL ? d.PF : d.F}) {
      if (w % 128)
        return SetError(MFH_ERR_UNSUPPORTED,
                        "the BF16X2_FP8LO precision needs embedding and FFN widths that "
                        "are multiples of 128");
    }
  }
  // FP8 precision: the row quantiser takes rows of up to 2048 values and
  // the fp8 GEMM a K that is a multiple of 128 (the encoder GEMMs' inputs
  // are E and FFN wide, in the body and in policy encoder layers).
  if (d.fp8_act) {
    for (const int w : {d.E, d.F, d.PL ? d.PF : d.F}) {
      if (w > 2048 || w % 128)
        return SetError(MFH_ERR_UNSUPPORTED,
                        "the FP8 precision needs embedding and FFN widths that are "
                        "multiples of 128 up to 2048");
    }
    // e4m3 activations move near-tied policy logits (top-1 ~80 % against
    // the fp32 CPU backend on the random-init BT4 net, policy max-abs
    // ~0.15): below the parity gates, so a caller has to ask for it.
    const char *fp8_env = std::getenv("METALFISH_HIP_EXPERIMENTAL_FP8");
    if (!(fp8_env && fp8_env[0] == '1'))
      return SetError(MFH_ERR_UNSUPPORTED,
                      "the FP8 precision is experimental and below the parity gates; "
                      "set METALFISH_HIP_EXPERIMENTAL_FP8=1 to use it");
  }
  return MFH_OK;
}

// The value the GPU multiplies for row n, column k of a packed GEMM
// weight: bf16, an e4m3 code times its row scale, or (BF16X2_FP8LO) W'
// times the column scale.
double PackedWeight(const Blob &blob, const size_t (&w)[2], bool fp8, bool lo8, int ld, int n,
                    int k) {
  const size_t i = static_cast<size_t>(n) * ld + k;
  float scale = 1.f;
  if (fp8 || lo8)
    std::memcpy(&scale, blob.bytes.data() + w[1] + 4 * static_cast<size_t>(n), 4);
  if (fp8 && !lo8)
    return static_cast<double>(DecodeE4m3(blob.bytes[w[0] + i])) * scale;
  std::uint16_t b;
  std::memcpy(&b, blob.bytes.data() + w[0] + 2 * i, 2);
  const std::uint32_t u = static_cast<std::uint32_t>(b) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return static_cast<double>(f) * scale;
}

// A LayerNorm (gamma, beta) folded into the GEMM that reads its output:
// fold_c[n] = sum_k gamma_k W[n][k] and bias'[n] = bias[n] + sum_k beta_k
// W[n][k] over the weights as the GPU holds them, summed in double.
// Returns {fold_c, bias'} blob offsets.
void AddLnFold(Blob &blob, const size_t (&w)[2], bool fp8, bool lo8, int rows, int K,
               size_t gamma, size_t beta, size_t bias, size_t (&out)[2]) {
  std::vector<float> c(rows), b(rows);
  std::vector<float> g(K), be(K), bi(rows);
  std::memcpy(g.data(), blob.bytes.data() + gamma, 4 * static_cast<size_t>(K));
  std::memcpy(be.data(), blob.bytes.data() + beta, 4 * static_cast<size_t>(K));
  std::memcpy(bi.data(), blob.bytes.data() + bias, 4 * static_cast<size_t>(rows));
  for (int n = 0; n < rows; ++n) {
    double sc = 0.0, sb = 0.0;
    for (int k = 0; k < K; ++k) {
      const double x = PackedWeight(blob, w, fp8, lo8, K, n, k);
      sc += g[k] * x;
      sb += be[k] * x;
    }
    c[n] = static_cast<float>(sc);
    b[n] = static_cast<float>(bi[n] + sb);
  }
  out[0] = blob.Add(c.data(), c.size() * 4);
  out[1] = blob.Add(b.data(), b.size() * 4);
}

void SetW(size_t (&dst)[2], const GemmW &g) {
  dst[0] = g.w;
  dst[1] = g.s;
}

int Pack(mfh_net *net, Loader &ld, Blob &blob) {
  const Dims &d = net->d;
  const int E = d.E, S = kSquares;
  auto need = [&](const std::string &n, size_t c) { return ld.Need(n, c); };
  const float *pre_w = d.pe_map ? nullptr
                                : need("body.ip_emb_preproc_w",
                                       static_cast<size_t>(S) * d.P * S * 12);
  const float *pre_b =
      d.pe_map ? nullptr : need("body.ip_emb_preproc_b", static_cast<size_t>(S) * d.P);
  const float *emb_w = need("body.ip_emb_w", static_cast<size_t>(E) * (kPlanes + d.P));
  const float *emb_b = need("body.ip_emb_b", E);
  const float *ln_g = need("body.ip_emb_ln_gammas", E);
  const float *ln_b = need("body.ip_emb_ln_betas", E);
  if (!ld.error.empty())
    return SetError(MFH_ERR_INVALID, ld.error);
  if (d.pe_map) {
    const auto &table = mfh_policy::StaticPositionEncoding();
    net->static_pe = blob.Add(table.data(), table.size() * sizeof(float));
  } else {
    SetW(net->pre_w, AddGemmW(blob, net->fp8, {pre_w}, {S * d.P}, S * 12, S * 12));
    net->pre_b = AddF32(blob, {pre_b}, {S * d.P});
  }
  SetW(net->emb_w, AddGemmW(blob, net->fp8, {emb_w}, {E}, kPlanes + d.P, d.Kin));
  net->emb_b = AddF32(blob, {emb_b}, {E});
  net->emb_ln_g = AddF32(blob, {ln_g}, {E});
  net->emb_ln_b = AddF32(blob, {ln_b}, {E});
  // The embedding gates, stored [E][64] (channel-major), go to the device
  // square-major, [64][E]: the LayerNorm kernel's lanes then read a row's
  // gate values as consecutive 16-byte vectors (channel-major, each lane's
  // values were 256 bytes apart: the embedding LayerNorm took 109 us at
  // batch 256, its L2 reads scattered over a line per value).
  auto add_gate = [&](const float *g) {
    std::vector<float> t(static_cast<size_t>(E) * S);
    for (int c = 0; c < E; ++c)
      for (int sq = 0; sq < S; ++sq)
        t[static_cast<size_t>(sq) * E + c] = g[static_cast<size_t>(c) * S + sq];
    return AddF32(blob, {t.data()}, {E * S});
  };
  net->mult_gate = net->add_gate = 0;
  if (ld.Count("body.ip_mult_gate")) {
    const float *g = need("body.ip_mult_gate", static_cast<size_t>(E) * S);
    if (g)
      net->mult_gate = add_gate(g);
  }
  if (ld.Count("body.ip_add_gate")) {
    const float *g = need("body.ip_add_gate", static_cast<size_t>(E) * S);
    if (g)
      net->add_gate = add_gate(g);
  }
  // The body's dense weights (input-embedding FFN, encoder layers); with
  // BF16X2_FP8LO they also carry e4m3 codes for the fp8 lo correction
  // (AddGemmWLo8), and every GEMM on them applies their column scales.
  auto dense_w = [&](const std::vector<const float *> &parts, const std::vector<int> &rows,
                     int cols, int ldw) {
    if (!d.lo8)
      return AddGemmW(blob, net->fp8, parts, rows, cols, ldw);
    size_t codes = 0;
    const GemmW g = AddGemmWLo8(blob, net->fp8, parts, rows, cols, ldw, &codes);
    net->lo8_codes[g.w] = codes;
    return g;
  };
  if (d.input_ffn) {
    const float *w1 = need("body.ip_emb_ffn.dense1_w", static_cast<size_t>(d.Fi) * E);
    const float *b1 = need("body.ip_emb_ffn.dense1_b", d.Fi);
    const float *w2 = need("body.ip_emb_ffn.dense2_w", static_cast<size_t>(E) * d.Fi);
    const float *b2 = need("body.ip_emb_ffn.dense2_b", E);
    const float *g = need("body.ip_emb_ffn_ln_gammas", E);
    const float *b = need("body.ip_emb_ffn_ln_betas", E);
    if (!ld.error.empty())
      return SetError(MFH_ERR_INVALID, ld.error);
    SetW(net->in_ffn1_w, dense_w({w1}, {d.Fi}, E, E));
    net->in_ffn1_b = AddF32(blob, {b1}, {d.Fi});
    SetW(net->in_ffn2_w, dense_w({w2}, {E}, d.Fi, d.Fi));
    net->in_ffn2_b = AddF32(blob, {b2}, {E});
    net->in_ln_g = AddF32(blob, {g}, {E});
    net->in_ln_b = AddF32(blob, {b}, {E});
  }
  if (d.smolgen) {
    const float *g = need("body.smolgen_w", static_cast<size_t>(S) * S * d.G);
    if (!g)
      return SetError(MFH_ERR_INVALID, ld.error);
    // Output rows (query q, key k at row 64 q + k) in the order attention
    // reads the bias tensor, so the projection writes that order; the
    // in-kernel bias reads the rows in their own order.
    std::vector<float> tiled;
    if (!d.fused_bias) {
      tiled.resize(static_cast<size_t>(S) * S * d.G);
      for (int q = 0; q < S; ++q)
        for (int k = 0; k < S; ++k)
          std::memcpy(&tiled[static_cast<size_t>(mfh::SmolgenBiasIndex(q, k)) * d.G],
                      g + static_cast<size_t>(q * S + k) * d.G, sizeof(float) * d.G);
      g = tiled.data();
    }
    SetW(net->global_w, AddGemmW(blob, net->fp8, {g}, {S * S}, d.G, d.G));
  }
  net->layers.resize(d.L);
  // One encoder layer (the reference's EncoderLayer, weights.cpp:162-180):
  // Q | K | V (| smolgen compression) fused into one weight, out-projection,
  // LayerNorms, FFN of width ffn, and the smolgen denses when present.
  auto pack_layer = [&](const std::string &p, Layer &L, int ffn, bool smolgen) -> int {
    const size_t EE = static_cast<size_t>(E) * E;
    const float *qw = need(p + ".mha.q_w", EE), *qb = need(p + ".mha.q_b", E);
    const float *kw = need(p + ".mha.k_w", EE), *kb = need(p + ".mha.k_b", E);
    const float *vw = need(p + ".mha.v_w", EE), *vb = need(p + ".mha.v_b", E);
    const float *ow = need(p + ".mha.dense_w", EE), *ob = need(p + ".mha.dense_b", E);
    const float *l1g = need(p + ".ln1_gammas", E), *l1b = need(p + ".ln1_betas", E);
    const float *f1w = need(p + ".ffn.dense1_w", static_cast<size_t>(ffn) * E);
    const float *f1b = need(p + ".ffn.dense1_b", ffn);
    const float *f2w = need(p + ".ffn.dense2_w", static_cast<size_t>(E) * ffn);
    const float *f2b = need(p + ".ffn.dense2_b", E);
    const float *l2g = need(p + ".ln2_gammas", E), *l2b = need(p + ".ln2_betas", E);
    const float *cw = nullptr;
    if (smolgen)
      cw = need(p + ".mha.smolgen.compress", static_cast<size_t>(d.C) * E);
    if (!ld.error.empty())
      return SetError(MFH_ERR_INVALID, ld.error);
    auto &gemm_w = dense_w;
    SetW(L.qkv_w, gemm_w({qw, kw, vw, cw}, {E, E, E, smolgen ? d.C : 0}, E, E));
    L.qkv_b = AddF32(blob, {qb, kb, vb, nullptr}, {E, E, E, smolgen ? d.C : 0});
    SetW(L.out_w, gemm_w({ow}, {E}, E, E));
    L.out_b = AddF32(blob, {ob}, {E});
    L.ln1_g = AddF32(blob, {l1g}, {E});
    L.ln1_b = AddF32(blob, {l1b}, {E});
    SetW(L.ffn1_w, gemm_w({f1w}, {ffn}, E, E));
    L.ffn1_b = AddF32(blob, {f1b}, {ffn});
    SetW(L.ffn2_w, gemm_w({f2w}, {E}, ffn, ffn));
    L.ffn2_b = AddF32(blob, {f2b}, {E});
    L.ln2_g = AddF32(blob, {l2g}, {E});
    L.ln2_b = AddF32(blob, {l2b}, {E});
    L.smolgen = smolgen;
    if (smolgen) {
      const std::string s = p + ".mha.smolgen";
      const float *d1w = need(s + ".dense1_w", static_cast<size_t>(d.Hs) * S * d.C);
      const float *d1b = need(s + ".dense1_b", d.Hs);
      const float *d2w = need(s + ".dense2_w", static_cast<size_t>(d.HG) * d.Hs);
      const float *d2b = need(s + ".dense2_b", d.HG);
      const float *g1 = need(s + ".ln1_gammas", d.Hs), *b1 = need(s + ".ln1_betas", d.Hs);
      const float *g2 = need(s + ".ln2_gammas", d.HG), *b2 = need(s + ".ln2_betas", d.HG);
      if (!ld.error.empty())
        return SetError(MFH_ERR_INVALID, ld.error);
      SetW(L.sg_d1_w, AddGemmW(blob, net->fp8, {d1w}, {d.Hs}, S * d.C, S * d.C));
      L.sg_d1_b = AddF32(blob, {d1b}, {d.Hs});
      L.sg_ln1_g = AddF32(blob, {g1}, {d.Hs});
      L.sg_ln1_b = AddF32(blob, {b1}, {d.Hs});
      SetW(L.sg_d2_w, AddGemmW(blob, net->fp8, {d2w}, {d.HG}, d.Hs, d.Hs));
      L.sg_d2_b = AddF32(blob, {d2b}, {d.HG});
      L.sg_ln2_g = AddF32(blob, {g2}, {d.HG});
      L.sg_ln2_b = AddF32(blob, {b2}, {d.HG});
    }
    return MFH_OK;
  };
  for (int i = 0; i < d.L; ++i) {
    const int rc = pack_layer("body.encoder." + std::to_string(i), net->layers[i], d.F, d.smolgen);
    if (rc != MFH_OK)
      return rc;
  }
  // Folded residual LayerNorms of the body (split precisions, nets sized
  // for kFoldLn1Rows token rows): Q|K|V (+ compression) of layer i > 0 over
  // layer i - 1's LN2, FFN1 of every layer over its LN1.
  const long net_rows = static_cast<long>(net->max_batch) * kSquares;
  if (d.fold_ln && d.split && !d.fp8_act && !d.fused_ln && d.E % (2 * mfh::kLnStatCols) == 0 &&
      net_rows >= kFoldLn1Rows) {
    const int qrows = 3 * E + (d.smolgen ? d.C : 0);
    for (int i = 0; i < d.L; ++i) {
      Layer &L = net->layers[i];
      const bool qlo8 = net->lo8_codes.count(L.qkv_w[0]) > 0;
      const bool flo8 = net->lo8_codes.count(L.ffn1_w[0]) > 0;
      if (i > 0) {
        const Layer &P = net->layers[i - 1];
        AddLnFold(blob, L.qkv_w, net->fp8, qlo8, qrows, E, P.ln2_g, P.ln2_b, L.qkv_b,
                  L.qkv_fold);
      }
      AddLnFold(blob, L.ffn1_w, net->fp8, flo8, d.F, E, L.ln1_g, L.ln1_b, L.ffn1_b,
                L.ffn1_fold);
    }
    net->has_fold = net_rows >= kFoldRows;
    net->has_fold1 = true;
  }
  // Policy encoder layers (weights.cpp:188-203), no smolgen.
  net->pol_layers.resize(d.PL);
  for (int i = 0; i < d.PL; ++i) {
    const int rc = pack_layer("policy.vanilla.encoder." + std::to_string(i), net->pol_layers[i],
                              d.PF, false);
    if (rc != MFH_OK)
      return rc;
  }
  const std::string pp = "policy.vanilla.", vp = "value.winner.";
  const float *pw = need(pp + "ip_pol_w", static_cast<size_t>(d.Dp) * E);
  const float *pb = need(pp + "ip_pol_b", d.Dp);
  const float *vw = need(vp + "ip_val_w", static_cast<size_t>(d.Vd) * E);
  const float *vb = need(vp + "ip_val_b", d.Vd);
  const float *q2w = need(pp + "ip2_pol_w", static_cast<size_t>(d.Dp) * d.Dp);
  const float *q2b = need(pp + "ip2_pol_b", d.Dp);
  const float *k3w = need(pp + "ip3_pol_w", static_cast<size_t>(d.Dp) * d.Dp);
  const float *k3b = need(pp + "ip3_pol_b", d.Dp);
  const float *p4 = need(pp + "ip4_pol_w", static_cast<size_t>(4) * d.Dp);
  const float *v1w = need(vp + "ip1_val_w", static_cast<size_t>(d.Vh) * S * d.Vd);
  const float *v1b = need(vp + "ip1_val_b", d.Vh);
  const float *v2w = need(vp + "ip2_val_w", static_cast<size_t>(d.Vout) * d.Vh);
  const float *v2b = need(vp + "ip2_val_b", d.Vout);
  const float *mw = nullptr, *mb = nullptr, *m1w = nullptr, *m1b = nullptr, *m2w = nullptr,
              *m2b = nullptr;
  if (d.mlh) {
    mw = need("moves_left.ip_mov_w", static_cast<size_t>(d.Md) * E);
    mb = need("moves_left.ip_mov_b", d.Md);
    m1w = need("moves_left.ip1_mov_w", static_cast<size_t>(d.Mh) * S * d.Md);
    m1b = need("moves_left.ip1_mov_b", d.Mh);
    m2w = need("moves_left.ip2_mov_w", d.Mh);
    m2b = need("moves_left.ip2_mov_b", 1);
  }
  if (!ld.error.empty())
    return SetError(MFH_ERR_INVALID, ld.error);
  if (d.mlh) {
    SetW(net->mov_w, AddGemmW(blob, net->fp8, {mw}, {d.Md}, E, E));
    net->mov_b = AddF32(blob, {mb}, {d.Md});
    SetW(net->mov1_w, AddGemmW(blob, net->fp8, {m1w}, {d.Mh}, S * d.Md, S * d.Md));
    net->mov1_b = AddF32(blob, {m1b}, {d.Mh});
    net->mov2_w = AddF32(blob, {m2w}, {d.Mh});
    net->mov2_b = AddF32(blob, {m2b}, {1});
  }
  SetW(net->head_w, AddGemmW(blob, net->fp8, {pw, vw}, {d.Dp, d.Vd}, E, E));
  net->head_b = AddF32(blob, {pb, vb}, {d.Dp, d.Vd});
  SetW(net->qk_w, AddGemmW(blob, net->fp8, {q2w, k3w}, {d.Dp, d.Dp}, d.Dp, d.Dp));
  net->qk_b = AddF32(blob, {q2b, k3b}, {d.Dp, d.Dp});
  net->promo = AddF32(blob, {p4}, {4 * d.Dp});
  SetW(net->val1_w, AddGemmW(blob, net->fp8, {v1w}, {d.Vh}, S * d.Vd, S * d.Vd));
  net->val1_b = AddF32(blob, {v1b}, {d.Vh});
  net->val2_w = AddF32(blob, {v2w}, {d.Vout * d.Vh});
  net->val2_b = AddF32(blob, {v2b}, {d.Vout});
  const auto &gather = mfh_policy::AttentionGather();
  net->gather = blob.Add(gather.data(), gather.size() * sizeof(std::int16_t));
  return MFH_OK;
}

// fp32 scratch for the split-K partials LaunchGemm may use on small batches.
constexpr size_t kSplitKFloats = size_t(8) << 20;
// The no-allocation layout's partials buffer.  GemmAutoSplits splits K only
// while the 64 x 64 tiles times the slices stay within kSplitMaxGroups
// (kSplitPairMaxGroups for a split the LayerNorm sums) workgroups, so a
// split GEMM's partials fit in this buffer as they fit in kSplitKFloats, and
// both layouts take the same splits (the same bits).
constexpr size_t kSmallSplitKFloats = size_t(512) * 64 * 64;
static_assert(kSmallSplitKFloats >= size_t(mfh::kSplitPairMaxGroups) * 64 * 64 &&
                  kSmallSplitKFloats >= size_t(mfh::kSplitMaxGroups) * 64 * 64,
              "no-allocation partials must hold the largest automatic split");
// Largest batch the no-allocation entry point takes (below 2048 token rows).
// That entry point runs the smolgen chain on the caller's stream, so its
// layout needs no second partials buffer.
constexpr int kNoAllocMaxBatch = 2048 / kSquares - 1;

// Split-K factor for the small-M GEMMs whose consumer sums partials
// (smolgen dense1 -> LayerNorm, value dense1 -> value head).  It depends on K
// only, so every position's result is bit-identical whatever the batch size
// or the batch it shares a call with.  Slices of at least 128 (16 of them
// for K = 2048): against 8 slices, forward at batch 32 2.57 -> 2.55 ms, 128
// 6.48 -> 6.43, 256 11.11 -> 11.05 (32 slices of 64 measured in between).
int SplitK(int k) {
  int s = 1;
  while (s < 16 && k % (2 * s * 64) == 0 && k / (2 * s) >= 128)
    s *= 2;
  return s;
}

// Offsets of every workspace tensor for `batch` positions, with split-K
// partial buffers of `splitk_floats` (a second one for the side stream's
// smolgen chain when `side`); returns the total size in bytes.
size_t PlanLayout(const Dims &d, int batch, size_t splitk_floats, bool side,
                  std::map<std::string, size_t> &ws_off) {
  const size_t B = static_cast<size_t>(batch);
  const size_t M = B * kSquares;
  size_t off = 0;
  ws_off.clear();
  auto add = [&](const std::string &name, size_t bytes) {
    off = AlignUp(off, 256);
    ws_off[name] = off;
    off += bytes;
  };
  // bf16 activations that feed MFMAs get a residual ("_lo") plane in split
  // precision.
  auto add16 = [&](const std::string &name, size_t elems) {
    add(name, elems * 2);
    if (d.split)
      add(name + "_lo", elems * 2);
  };
  // Attention and smolgen operands carry the pair only in full BF16X2.
  auto add16a = [&](const std::string &name, size_t elems) {
    add(name, elems * 2);
    if (d.split_attn)
      add(name + "_lo", elems * 2);
  };
  const int hid = std::max(d.F, std::max(d.Fi, d.PF));
  const int sk1 = d.smolgen ? SplitK(kSquares * d.C) : 1;
  const int skv = SplitK(kSquares * d.Vd);
  add("masks", B * kPlanes * 8);
  add("values", B * kPlanes * 4);
  add16("emb_in", M * d.Kin);
  add("pos_in", B * kSquares * 12 * 2);
  add("pe", B * kSquares * d.P * 4);
  add("pre", M * d.E * 4);
  add("resid", M * d.E * 4);
  add16("act", M * d.E);
  add16a("qkv", M * 3 * d.E);
  add16a("comp", M * (d.C ? d.C : 1));
  add("sg1", sk1 * B * (d.Hs ? d.Hs : 1) * 4);
  add16a("sg1n", B * (d.Hs ? d.Hs : 1));
  add("sg2", B * (d.HG ? d.HG : 1) * 4);
  add16a("sg2n", B * (d.HG ? d.HG : 1));
  add("bias", d.smolgen && !d.fused_bias ? B * d.H * kSquares * kSquares * (d.split_attn ? 4 : 2)
                                          : 256);
  add16("ctx", M * d.E);
  add16("hid", M * (hid ? hid : 1));
  add16("pol_emb", M * d.Dp);
  add16("val_emb", M * d.Vd);
  add16("polqk", M * 2 * d.Dp);
  add("val1", skv * B * d.Vh * 4);
  add16("mov_emb", M * (d.Md ? d.Md : 1));
  add("mov1", (d.mlh ? SplitK(kSquares * d.Md) : 1) * B * (d.Mh ? d.Mh : 1) * 4);
  add("mlh", B * 4);
  // e4m3 copies of the body GEMM inputs with their row scales (FP8).
  if (d.fp8_act) {
    add("act8", M * d.E);
    add("sc_act", M * 4);
    add("ctx8", M * d.E);
    add("sc_ctx", M * 4);
    add("hid8", M * (hid ? hid : 1));
    add("sc_hid", M * 4);
  }
  // e4m3 lo parts of the encoder GEMM inputs (BF16X2_FP8LO), at the batches
  // whose forward uses them.
  if (d.fold_ln && d.split && !d.fp8_act && !d.fused_ln &&
      d.E % (2 * mfh::kLnStatCols) == 0 && M >= static_cast<size_t>(kFoldLn1Rows)) {
    // Per-row partial sums of the folded LayerNorms' rows (LN2: "st_act",
    // LN1: "st_mid"), per 64 columns at most.
    add("st_act", M * (d.E / 64) * 2 * 4);
    add("st_mid", M * (d.E / 64) * 2 * 4);
  }
  if (d.lo8 && M >= static_cast<size_t>(kLo8MinRows)) {
    add("act_lo8", M * d.E);
    add("qkv_lo8", M * 3 * d.E);
    add("bias_lo8", d.smolgen ? B * d.H * kSquares * kSquares : 256);
    add("ctx_lo8", M * d.E);
    add("hid_lo8", M * (hid ? hid : 1));
  }
  // Row statistics of the single-position smolgen chain's deferred
  // LayerNorms (partial sums per workgroup): dense1 and dense2 outputs.
  // One (sum, sum of squares) pair per producing workgroup and row, for up
  // to kSkinnyMaxRows rows.
  const size_t stat_rows = std::min<size_t>(B, mfh::kSkinnyMaxRows);
  add("lnst_s1",
      std::max<size_t>(256, 8 * stat_rows * size_t(mfh::SkinnyGemmParts(d.Hs ? d.Hs : 4))));
  add("lnst_s2",
      std::max<size_t>(256, 8 * stat_rows * size_t(mfh::SkinnyGemmParts(d.HG ? d.HG : 4))));
  // Split-K partials of small-batch GEMMs (main stream, and the smolgen
  // chain on the side stream).
  add("splitk", splitk_floats * 4);
  if (side)
    add("splitk_sg", splitk_floats * 4);
  add("policy", B * kPolicy * 4);
  add("wdl", B * 3 * 4);
  // Legal-move priors (mfh_net_eval_priors): offsets, policy indices, priors.
  add("move_offsets", (B + 1) * 4);
  add("move_indices", B * kMaxMoves * 2);
  add("priors", B * kMaxMoves * 4);
  return AlignUp(off, 256);
}

void PlanWorkspace(mfh_net *net) {
  net->ws_bytes = PlanLayout(net->d, net->max_batch, kSplitKFloats, net->d.smolgen, net->ws_off);
  // The no-allocation entry point's layout in the scratch array: the largest
  // single-stream batch whose workspace fits.
  // The limit stays below the first batch whose Q|K|V would take whole-round
  // 256 x 256 tiles: beside the side-stream smolgen chain those tiles (and
  // the chain's) are chosen to share CUs, which the single-stream
  // no-allocation forward does not do, so its bits could differ from
  // mfh_net_eval_device's.  (For the nets here the first such batch is far
  // above the limit.)
  int limit = std::min(net->max_batch, kNoAllocMaxBatch);
  for (int b = 1; b <= limit; ++b) {
    mfh::GemmParams q;
    q.M = b * kSquares;
    q.N = 3 * net->d.E;
    q.K = net->d.E;
    if (mfh::GemmWholeRoundTiles(q)) {
      limit = b - 1;
      break;
    }
  }
  net->noalloc_max_batch = 0;
  for (int b = limit; b >= 1; --b) {
    const size_t bytes = PlanLayout(net->d, b, kSmallSplitKFloats, false, net->noalloc_off);
    if (bytes <= kScratchBytes) {
      net->noalloc_max_batch = b;
      net->noalloc_bytes = bytes;
      break;
    }
  }
}

// The workspace one forward uses: the net's own allocation, or the scratch
// array (mfh_net_eval_device_noalloc).
struct WsView {
  unsigned char *base = nullptr;
  const std::map<std::string, size_t> *off = nullptr;
  size_t splitk_floats = 0;

  template <typename T> T *S(const std::string &name) const {
    return reinterpret_cast<T *>(base + off->at(name));
  }
  bool Has(const std::string &name) const { return off->count(name) != 0; }
  // Residual plane of a bf16 activation, or null in single precision.
  std::uint16_t *Lo(const std::string &name) const {
    auto it = off->find(name + "_lo");
    return it == off->end() ? nullptr : reinterpret_cast<std::uint16_t *>(base + it->second);
  }
};

WsView MainWs(const mfh_net *net) { return WsView{net->ws, &net->ws_off, kSplitKFloats}; }

hipEvent_t TakeEvent(mfh_net *net) {
  if (!net->event_pool.empty()) {
    hipEvent_t e = net->event_pool.back();
    net->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDefault) != hipSuccess)
    return nullptr;
  return e;
}

// Brackets one launch with events on its stream when profiling is on.
struct StageTimer {
  mfh_net *net;
  hipStream_t st;
  mfh_net::Pending rec;
  bool on = false;
  StageTimer(mfh_net *n, hipStream_t s, const std::string &name, double flops, double bytes)
      : net(n), st(s) {
    if (!net->profiling || net->noalloc_call)
      return;
    rec.name = name;
    rec.flops = flops;
    rec.bytes = bytes;
    rec.start = TakeEvent(net);
    rec.stop = TakeEvent(net);
    on = rec.start && rec.stop && hipEventRecord(rec.start, st) == hipSuccess;
  }
  ~StageTimer() {
    if (on && hipEventRecord(rec.stop, st) == hipSuccess)
      net->pending.push_back(rec);
  }
};

int CollectProfile(mfh_net *net) {
  for (auto &p : net->pending) {
    MFH_HIP_CHECK(hipEventSynchronize(p.stop));
    float ms = 0.f;
    MFH_HIP_CHECK(hipEventElapsedTime(&ms, p.start, p.stop));
    auto &t = net->totals[p.name];
    t.launches += 1;
    t.ms += ms;
    t.flops += p.flops;
    t.bytes += p.bytes;
    net->event_pool.push_back(p.start);
    net->event_pool.push_back(p.stop);
  }
  net->pending.clear();
  return MFH_OK;
}

// Smallest token-row count (positions x 64) at which residual GEMMs may run
// as row-panel GEMMs with the LayerNorm fused (128 positions: 128 panels
// half-fill the 256 CUs; fewer leave most of them idle).
constexpr int kPanelMinRows = 8192;

// Profiler name of a GEMM launch: "gemm_bf16:<role>", or
// "gemm_bf16_splitk:<role>" when the caller splits K (partials summed by the
// consumer).
std::string GemmKind(const mfh::GemmParams &p, const char *role) {
  return std::string(p.k_splits > 1 ? "gemm_bf16_splitk:" : "gemm_bf16:") + role;
}

// The forward pass.  only_layer >= 0 runs body encoder layer only_layer
// alone on the residual stream already in the workspace (the encoder-layer
// microbenchmark), nothing before or after it.
int Forward(mfh_net *net, const WsView &ws, int B, const std::uint64_t *masks,
            const float *values, float *policy, float *wdl, float *moves_left, hipStream_t st,
            int only_layer = -1) {
  const bool full = only_layer < 0;
  const Dims &d = net->d;
  const int M = B * kSquares;
  const int E = d.E;
  std::string err_;
  auto fail = [&](hipError_t e) {
    return SetError(e == hipErrorInvalidValue ? MFH_ERR_INVALID : MFH_ERR_HIP,
                    err_.empty() ? std::string(hipGetErrorString(e)) : err_);
  };
#define MFH_RUN(expr)                                                          \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess)                                                      \
      return fail(e_);                                                         \
  } while (0)
#define MFH_RC(expr)                                                           \
  do {                                                                         \
    const int rc_ = (expr);                                                    \
    if (rc_ != MFH_OK)                                                         \
      return rc_;                                                              \
  } while (0)
  // GEMM with A from workspace tensor `a` (its residual plane when split).
  auto gemm = [&](const std::string &a, int lda, const size_t (&w)[2], int ldw, int m, int n,
                  int k, const float *bias, int act, int mode, void *C, void *C_lo, int ldc) {
    mfh::GemmParams p;
    p.A = ws.S<std::uint16_t>(a);
    p.A_lo = ws.Lo(a);
    p.lda = lda;
    if (net->lo8_codes.count(w[0])) {
      // A BF16X2_FP8LO weight: bf16 rows scaled per column, for the plain
      // product too.
      p.W = net->W<std::uint16_t>(w[0]);
      p.wscale = net->W<float>(w[1]);
    } else if (net->fp8) {
      p.W8 = net->W<std::uint8_t>(w[0]);
      p.wscale = net->W<float>(w[1]);
    } else {
      p.W = net->W<std::uint16_t>(w[0]);
    }
    p.ldw = ldw;
    p.M = m;
    p.N = n;
    p.K = k;
    p.bias = bias;
    p.act = act;
    p.partials = ws.S<float>("splitk");
    p.partials_floats = ws.splitk_floats;
    p.out_mode = mode;
    p.C = C;
    p.C_lo = C_lo;
    p.ldc = ldc;
    return p;
  };
  const double plane_mult = d.split ? 2.0 : 1.0;  // bytes of a bf16 activation
  // Launch on the main stream, or on `on` (the side stream's smolgen chain).
  auto run = [&](const mfh::GemmParams &p, const char *role, hipStream_t on = nullptr) {
    const double flops = 2.0 * p.M * p.N * p.K;
    const double out_bytes = p.out_mode == mfh::GEMM_OUT_BF16 ? 2.0 * plane_mult : 4.0;
    const double bytes = 2.0 * p.M * p.K * (p.A_lo ? 2.0 : 1.0) + (p.W8 ? 1.0 : 2.0) * p.N * p.K +
                         (p.A_lo8 ? 1.0 * p.M * p.K + 1.0 * p.N * p.K : 0.0) +
                         out_bytes * p.M * p.N * p.k_splits +
                         (p.out_mode == mfh::GEMM_OUT_RESID_F32 ? 4.0 * p.M * p.N : 0.0);
    hipStream_t s = on ? on : st;
    StageTimer t(net, s, GemmKind(p, role), flops, bytes);
    return mfh::LaunchGemm(p, s, &err_);
  };
  auto run_ln = [&](const mfh::LayerNormParams &lp, hipStream_t on = nullptr) {
    const double n = static_cast<double>(lp.rows) * lp.width;
    const double bytes = 4.0 * n * lp.parts + (lp.y_f32 ? 4.0 * n : 0.0) +
                         (lp.y_bf16 ? 2.0 * n * (lp.y_bf16_lo ? 2.0 : 1.0) : 0.0);
    hipStream_t s = on ? on : st;
    StageTimer t(net, s, "layernorm", 0.0, bytes);
    return mfh::LaunchLayerNorm(lp, s, &err_);
  };
  // BF16X2_FP8LO at this batch: the LayerNorms writing "act" also write its
  // e4m3 lo codes, attention and FFN1 write theirs instead of bf16 lo planes,
  // and the encoder GEMMs on those inputs add the fp8 lo product.
  const bool lo8 = d.lo8 && M >= kLo8MinRows && ws.Has("act_lo8");
  // The "act" codes are written when Q|K|V or FFN1 takes them (whole rounds
  // of 256 x 256 tiles, as lo8_gemm below decides).
  const auto whole_round = [](int m, int n) {
    mfh::GemmParams q;
    q.M = m;
    q.N = n;
    return mfh::GemmWholeRoundTiles(q);
  };
  const bool lo8_act =
      lo8 && (whole_round(M, 3 * E) || whole_round(M, d.F) || (d.input_ffn && whole_round(M, d.Fi)));
  // The body's residual LayerNorms folded into the GEMMs around them (see
  // kFoldRows): the whole forward (a single debug layer keeps them), where
  // the residual GEMMs take whole rounds of 256 x 256 tiles.
  // (Checked below: every GEMM around them must have a tile that compiles
  // the folded epilogue.)
  bool fold = net->has_fold && full && ws.Has("st_act") && whole_round(M, E) &&
              M >= kSmolgenSideRows;
  // Below whole rounds (kFoldLn1Rows on): LN1 on the 64 x 64 residual
  // tiles (partial sums per 64 columns), and LN2 too where its consumers
  // have tiles that fold it (fold2).
  bool fold1 = !fold && net->has_fold1 && full && ws.Has("st_mid") && M >= kFoldLn1Rows;
  bool fold2 = fold1 && ws.Has("st_act") && M >= kSmolgenSideRows;
  float *st_act = nullptr, *st_mid = nullptr;
  // Columns per partial sum: 128 on the whole-round 256-wide tiles, 64 on
  // the 64-wide ones (set with the fold below).
  int ln_part = 128;
  auto ln = [&](const float *x, int rows, int width, float eps, const float *g, const float *b,
                float *y32, const std::string &y16) {
    mfh::LayerNormParams lp;
    if (lo8_act && y16 == "act")
      lp.y_lo8 = ws.S<std::uint8_t>("act_lo8");
    lp.x = x;
    lp.rows = rows;
    lp.width = width;
    lp.eps = eps;
    lp.gamma = g;
    lp.beta = b;
    lp.y_f32 = y32;
    lp.y_bf16 = ws.S<std::uint16_t>(y16);
    lp.y_bf16_lo = ws.Lo(y16);
    return lp;
  };

  auto *pe = ws.S<float>("pe");
  auto *pre = ws.S<float>("pre");
  auto *resid = ws.S<float>("resid");
  // In the split precisions a LayerNorm's hi + lo output planes ("act") are
  // both the next GEMM's input and the residual of the next residual GEMM,
  // so its fp32 copy is written only where something reads it: the bf16
  // precision's residual, and the body output (debug tensor "body").
  float *res32 = d.split ? nullptr : resid;
  auto *splitk = ws.S<float>("splitk");
  auto *sg1 = ws.S<float>("sg1");
  auto *sg2 = ws.S<float>("sg2");
  auto *val1 = ws.S<float>("val1");

  // Input planes, dynamic positional encoding, embedding (cpu_network.cpp:
  // 691-890), embedding LayerNorm + gates (1399-1457, 1268-1316).
  if (full) {
    {
      StageTimer t(net, st, "input_expand", 0.0,
                   12.0 * B * kPlanes + 2.0 * M * d.Kin * plane_mult);
      MFH_RUN(mfh::LaunchExpandInputs(
          masks, values, B, ws.S<std::uint16_t>("emb_in"), ws.Lo("emb_in"), d.Kin,
          d.pe_map ? net->W<float>(net->static_pe) : nullptr, d.P,
          ws.S<std::uint16_t>("pos_in"), st, &err_));
    }
    if (!d.pe_map) {
      // The PE input holds exact plane values: single precision suffices.
      mfh::GemmParams p = gemm("pos_in", kSquares * 12, net->pre_w, kSquares * 12, B,
                               kSquares * d.P, kSquares * 12, net->W<float>(net->pre_b),
                               mfh::ACT_NONE, mfh::GEMM_OUT_F32, pe, nullptr, kSquares * d.P);
      MFH_RUN(run(p, "pe"));
    }
    if (!d.pe_map) {
      StageTimer tpe(net, st, "pe_scatter", 0.0, 4.0 * B * kSquares * d.P);
      MFH_RUN(mfh::LaunchScatterPe(pe, B, d.P, ws.S<std::uint16_t>("emb_in"), ws.Lo("emb_in"),
                                   d.Kin, st, &err_));
    }
    MFH_RUN(run(gemm("emb_in", d.Kin, net->emb_w, d.Kin, M, E, d.Kin, net->W<float>(net->emb_b),
                     d.act_default, mfh::GEMM_OUT_F32, pre, nullptr, E),
                    "embedding"));
    {
      mfh::LayerNormParams lp = ln(pre, M, E, d.eps_emb, net->W<float>(net->emb_ln_g),
                                   net->W<float>(net->emb_ln_b), res32, "act");
      lp.mult_gate = net->mult_gate ? net->W<float>(net->mult_gate) : nullptr;
      lp.add_gate = net->add_gate ? net->W<float>(net->add_gate) : nullptr;
      MFH_RUN(run_ln(lp));
    }
  }
  // FP8 precision: rows of workspace tensor `a` -> e4m3 codes "<a>8" and
  // their scales "sc_<a>", and a GEMM switched onto them.
  auto quant = [&](const std::string &a, int cols) -> int {
    StageTimer t(net, st, "quantize_e4m3", 0.0, 2.0 * M * cols + 1.0 * M * cols + 4.0 * M);
    MFH_RUN(mfh::LaunchQuantizeRowsE4m3(ws.S<std::uint16_t>(a), ws.Lo(a), cols, M, cols,
                                        ws.S<std::uint8_t>(a + "8"), cols,
                                        ws.S<float>("sc_" + a), st, &err_));
    return MFH_OK;
  };
  auto use_fp8 = [&](mfh::GemmParams &p, const std::string &a) {
    p.A8 = ws.S<std::uint8_t>(a + "8");
    p.ascale = ws.S<float>("sc_" + a);
    p.A = nullptr;
    p.A_lo = nullptr;
  };
  // BF16X2_FP8LO: the GEMM on workspace input `a` (hi plane + e4m3 lo codes
  // "<a>_lo8") with the codes of weight w_off for the fp8 lo product; false
  // (p unchanged) where this forward or weight has none.
  // Whether an encoder GEMM of m x n on weight w_off takes the fp8 lo
  // correction: its 256 x 256 tiles (the only tiles of that kernel) must fill
  // whole rounds of 256 workgroups; elsewhere (batch 256 FFN1 at 1.5 rounds,
  // batch 128) the BF16X2 tiles were faster.  Producers write e4m3 lo codes
  // exactly where their consumer takes them.
  auto lo8_gemm = [&](int m, int n, const size_t (&w_off)[2]) {
    return lo8 && net->lo8_codes.count(w_off[0]) && whole_round(m, n);
  };
  auto use_lo8 = [&](mfh::GemmParams &p, const std::string &a, const size_t (&w_off)[2]) {
    const auto it = net->lo8_codes.find(w_off[0]);
    if (!lo8_gemm(p.M, p.N, w_off) || (a == "act" && !lo8_act))
      return false;
    p.A_lo = nullptr;
    p.A_lo8 = ws.S<std::uint8_t>(a + "_lo8");
    p.lda8 = p.lda;
    p.W_lo8 = net->W<std::uint8_t>(it->second);
    p.ldw8 = p.ldw;
    p.partials = nullptr;
    return true;
  };
  auto residual_gemm = [&](const std::string &a, int k, const size_t (&w_off)[2],
                           const float *bias, const char *role, float alpha, bool f8 = false) {
    mfh::GemmParams p = gemm(a, k, w_off, k, M, E, k, bias, mfh::ACT_NONE,
                             mfh::GEMM_OUT_RESID_F32, pre, nullptr, E);
    if (f8)
      use_fp8(p, a);
    else
      use_lo8(p, a, w_off);
    if (d.split) {
      p.resid16 = ws.S<std::uint16_t>("act");
      p.resid16_lo = ws.Lo("act");
    } else {
      p.resid = resid;
    }
    p.ldr = E;
    p.alpha = alpha;
    return run(p, role);
  };
  // Residual GEMM followed by its LayerNorm, y = LN(x + alpha (A.W^T + b)),
  // onto the "act" planes (and y32 when set).  At large batches one
  // row-panel launch does both, the pre-LayerNorm rows never leaving the
  // workgroup; at small batches the LayerNorm kernel sums the GEMM's split-K
  // partials with the bias and residual; otherwise the tiled GEMM writes the
  // pre-LayerNorm rows to `pre` for the LayerNorm kernel.
  // A residual GEMM beside folded LayerNorms (kFoldRows): the residual is
  // the "act" planes, LN(x) of folded rows x o gamma when res_st is set
  // (rg / rb / res_eps that LayerNorm's); the sum x = resid + alpha (A.W^T +
  // b) leaves folded, as x o og onto "act" with its partial sums in out_st
  // (og set), or in fp32 to `pre` for the LayerNorm kernel (g / b / eps,
  // y32 as in residual_ln).
  auto residual_fold = [&](const std::string &a, int k, const size_t (&w_off)[2],
                           const float *bias, const char *role, float alpha, const float *res_st,
                           const float *rg, const float *rb, float res_eps, const float *og,
                           float *out_st, float eps, const float *g, const float *b,
                           float *y32) -> int {
    mfh::GemmParams p = gemm(a, k, w_off, k, M, E, k, bias, mfh::ACT_NONE,
                             mfh::GEMM_OUT_RESID_F32, pre, nullptr, E);
    use_lo8(p, a, w_off);
    p.partials = nullptr;
    p.resid16 = ws.S<std::uint16_t>("act");
    p.resid16_lo = ws.Lo("act");
    p.ldr = E;
    p.alpha = alpha;
    p.ln_width = E;
    p.ln_part = ln_part;
    if (res_st) {
      p.res_stats = res_st;
      p.res_gamma = rg;
      p.res_beta = rb;
      p.res_eps = res_eps;
    }
    if (og) {
      // In place: each output element is read (as the residual) and then
      // written by the same thread.
      p.out_gamma = og;
      p.out_stats = out_st;
      p.C = ws.S<std::uint16_t>("act");
      p.C_lo = ws.Lo("act");
      p.ldc = E;
      if (lo8_act) {
        p.C_lo8 = ws.S<std::uint8_t>("act_lo8");
        p.ldc8 = E;
      }
      MFH_RUN(run(p, role));
      return MFH_OK;
    }
    MFH_RUN(run(p, role));
    MFH_RUN(run_ln(ln(pre, M, E, eps, g, b, y32, "act")));
    return MFH_OK;
  };
  auto residual_ln = [&](const std::string &a, int k, const size_t (&w_off)[2],
                         const float *bias, const char *role, float alpha, float eps,
                         const float *g, const float *b, float *y32, bool f8 = false) -> int {
    // fused_layernorm (default with fp8 weights).  The panel streams each
    // weight row from L2 for only 64 activation rows, which needs every
    // weight fragment to feed two MFMAs (split activations); with bf16
    // weights the tiled GEMM's staged epilogue plus the LayerNorm kernel
    // measured faster on the BT4 shape.
    if (d.fused_ln && d.split && M >= kPanelMinRows &&
        mfh::PanelGemmShapeOk(mfh::PANEL_OUT_LN, E, k)) {
      mfh::PanelGemmParams pp;
      pp.A = ws.S<std::uint16_t>(a);
      pp.A_lo = ws.Lo(a);
      pp.lda = k;
      if (net->fp8) {
        pp.W8 = net->W<std::uint8_t>(w_off[0]);
        pp.wscale = net->W<float>(w_off[1]);
      } else {
        pp.W = net->W<std::uint16_t>(w_off[0]);
      }
      pp.ldw = k;
      pp.M = M;
      pp.N = E;
      pp.K = k;
      pp.bias = bias;
      pp.out_mode = mfh::PANEL_OUT_LN;
      pp.C = ws.S<std::uint16_t>("act");
      pp.C_lo = ws.Lo("act");
      pp.ldc = E;
      if (d.split) {
        pp.resid16 = pp.C;
        pp.resid16_lo = pp.C_lo;
      } else {
        pp.resid = resid;
      }
      pp.alpha = alpha;
      pp.eps = eps;
      pp.gamma = g;
      pp.beta = b;
      pp.y_f32 = y32;
      const double flops = 2.0 * M * E * k;
      const double bytes = 2.0 * M * k * (pp.A_lo ? 2.0 : 1.0) + (pp.W8 ? 1.0 : 2.0) * E * k +
                           2.0 * (2.0 * plane_mult * M * E) + (y32 ? 4.0 * M * E : 0.0) +
                           (d.split ? 0.0 : 4.0 * M * E);
      StageTimer t(net, st, std::string("gemm_bf16:") + role, flops, bytes);
      const hipError_t e = mfh::LaunchPanelGemm(pp, st, &err_);
      return e == hipSuccess ? MFH_OK : fail(e);
    }
    mfh::GemmParams p = gemm(a, k, w_off, k, M, E, k, bias, mfh::ACT_NONE,
                             mfh::GEMM_OUT_RESID_F32, pre, nullptr, E);
    const int splits = f8 ? 1 : mfh::GemmAutoSplits(p, true);
    if (f8) {
      MFH_RC(quant(a, k));
    } else if (splits > 1) {
      // Few positions: the K slices' raw partials go straight to the
      // LayerNorm kernel, which sums them in slice order with the bias and
      // the residual (no separate reduce launch).
      p.bias = nullptr;
      p.out_mode = mfh::GEMM_OUT_F32;
      p.C = splitk;
      p.ldc = E;
      p.k_splits = splits;
      p.partials = nullptr;
      MFH_RUN(run(p, role));
      mfh::LayerNormParams lp = ln(splitk, M, E, eps, g, b, y32, "act");
      lp.parts = splits;
      lp.bias = bias;
      if (d.split) {
        lp.resid16 = ws.S<std::uint16_t>("act");
        lp.resid16_lo = ws.Lo("act");
      } else {
        lp.resid = resid;
      }
      lp.alpha = alpha;
      MFH_RUN(run_ln(lp));
      return MFH_OK;
    }
    MFH_RUN(residual_gemm(a, k, w_off, bias, role, alpha, f8));
    MFH_RUN(run_ln(ln(pre, M, E, eps, g, b, y32, "act")));
    return MFH_OK;
  };
  if (full && d.input_ffn) {
    mfh::GemmParams pi = gemm("act", E, net->in_ffn1_w, E, M, d.Fi, E,
                              net->W<float>(net->in_ffn1_b), d.act_ffn, mfh::GEMM_OUT_BF16,
                              ws.S<std::uint16_t>("hid"), ws.Lo("hid"), d.Fi);
    use_lo8(pi, "act", net->in_ffn1_w);
    if (lo8_gemm(M, E, net->in_ffn2_w)) {
      pi.C_lo = nullptr;
      pi.C_lo8 = ws.S<std::uint8_t>("hid_lo8");
      pi.ldc8 = d.Fi;
    }
    MFH_RUN(run(pi, "input_ffn1"));
    const int rc = residual_ln("hid", d.Fi, net->in_ffn2_w, net->W<float>(net->in_ffn2_b),
                               "input_ffn2", d.alpha, 1e-3f, net->W<float>(net->in_ln_g),
                               net->W<float>(net->in_ln_b), res32);
    if (rc != MFH_OK)
      return rc;
  }

  // Single position (M <= 64 token rows, bf16 weights): the smolgen chain
  // runs as three few-row GEMM launches instead of six (split-K GEMMs with
  // their LayerNorm and reduce launches).  dense1 writes its activated rows
  // with their partial row statistics, dense2 applies dense1's LayerNorm as
  // it loads them, and the global projection applies dense2's (each of its
  // rows one head's gen-wide segment of the position's row).
  const bool few_row_smolgen =
      d.smolgen && d.skinny && M <= mfh::kSkinnyMaxRows && B * d.H <= mfh::kSkinnyMaxRows &&
      !net->fp8 && !d.fused_bias && d.HG <= 8192 &&
      mfh::SkinnyShapeOk(B, d.Hs, kSquares * d.C) && mfh::SkinnyShapeOk(B, d.HG, d.Hs) &&
      mfh::SkinnyShapeOk(B * d.H, kSquares * kSquares, d.G);
  // Up to kSmolgenFewRowMaxBatch positions: dense1 and dense2 (one row per
  // position) run as few-row GEMMs too, dense2 applying dense1's LayerNorm
  // as it loads its rows; dense2's LayerNorm and the global projection
  // (B * H rows) stay separate launches.
  const bool few_row_dense = d.smolgen && d.skinny && !few_row_smolgen &&
                             B <= kSmolgenFewRowMaxBatch && !net->fp8 &&
                             mfh::SkinnyShapeOk(B, d.Hs, kSquares * d.C) &&
                             mfh::SkinnyShapeOk(B, d.HG, d.Hs);
  auto run_sk = [&](const mfh::SkinnyParams &p, const char *role, hipStream_t on = nullptr) {
    const double flops = 2.0 * p.M * p.N * p.K;
    const double bytes = 2.0 * p.N * p.K + 4.0 * p.M * p.K + 4.0 * p.M * p.N;
    hipStream_t s = on ? on : st;
    StageTimer t(net, s, std::string("gemm_bf16:") + role, flops, bytes);
    return mfh::LaunchSkinnyGemm(p, s, &err_);
  };
  // dense1 (from the compression planes, writing its activated rows and their
  // partial statistics) and dense2 (normalising dense1's rows as it loads
  // them) as few-row GEMMs; dense2's statistics too when `dense2_stats`.
  auto smolgen_dense_few_row = [&](const Layer &L, hipStream_t on, bool dense2_stats) -> int {
    auto base = [&](const size_t (&w)[2], int m, int n, int k, const float *bias, int act,
                    int mode, void *C, int ldc) {
      mfh::SkinnyParams p;
      p.W = net->W<std::uint16_t>(w[0]);
      p.ldw = k;
      p.M = m;
      p.N = n;
      p.K = k;
      p.bias = bias;
      p.act = act;
      p.out_mode = mode;
      p.C = C;
      p.ldc = ldc;
      return p;
    };
    const int flat = kSquares * d.C;
    mfh::SkinnyParams p1 = base(L.sg_d1_w, B, d.Hs, flat, net->W<float>(L.sg_d1_b),
                                d.act_smolgen, mfh::SKINNY_OUT_F32, ws.S<float>("sg1"), d.Hs);
    p1.a16 = ws.S<std::uint16_t>("comp");
    p1.a16_lo = ws.Lo("comp");
    p1.lda = flat;
    p1.stats_out = ws.S<float>("lnst_s1");
    MFH_RUN(run_sk(p1, "smolgen_dense1", on));
    mfh::SkinnyParams p2 = base(L.sg_d2_w, B, d.HG, d.Hs, net->W<float>(L.sg_d2_b),
                                d.act_smolgen, mfh::SKINNY_OUT_F32, ws.S<float>("sg2"), d.HG);
    p2.x = ws.S<float>("sg1");
    p2.ldx = d.Hs;
    p2.ln_stats = ws.S<float>("lnst_s1");
    p2.ln_parts = mfh::SkinnyGemmParts(d.Hs);
    p2.ln_rows = B;
    p2.ln_width = d.Hs;
    p2.ln_eps = 1e-3f;
    p2.gamma = net->W<float>(L.sg_ln1_g);
    p2.beta = net->W<float>(L.sg_ln1_b);
    p2.ln_split = d.split_attn;
    if (dense2_stats)
      p2.stats_out = ws.S<float>("lnst_s2");
    MFH_RUN(run_sk(p2, "smolgen_dense2", on));
    return MFH_OK;
  };
  auto smolgen_few_row = [&](const Layer &L) -> int {
    MFH_RC(smolgen_dense_few_row(L, st, true));
    auto base = [&](const size_t (&w)[2], int m, int n, int k, const float *bias, int act,
                    int mode, void *C, int ldc) {
      mfh::SkinnyParams p;
      p.W = net->W<std::uint16_t>(w[0]);
      p.ldw = k;
      p.M = m;
      p.N = n;
      p.K = k;
      p.bias = bias;
      p.act = act;
      p.out_mode = mode;
      p.C = C;
      p.ldc = ldc;
      return p;
    };
    mfh::SkinnyParams pg =
        base(net->global_w, B * d.H, kSquares * kSquares, d.G, nullptr, mfh::ACT_NONE,
             d.split_attn ? mfh::SKINNY_OUT_F32 : mfh::SKINNY_OUT_BF16, ws.S<void>("bias"),
             kSquares * kSquares);
    pg.x = ws.S<float>("sg2");
    pg.ldx = d.HG;
    pg.rows_per_src = d.H;
    pg.ln_stats = ws.S<float>("lnst_s2");
    pg.ln_parts = mfh::SkinnyGemmParts(d.HG);
    pg.ln_rows = B;
    pg.ln_width = d.HG;
    pg.ln_eps = 1e-3f;
    pg.gamma = net->W<float>(L.sg_ln2_g);
    pg.beta = net->W<float>(L.sg_ln2_b);
    pg.ln_split = d.split_attn;
    MFH_RUN(run_sk(pg, "smolgen_global"));
    return MFH_OK;
  };

  int layer_index = 0;  // encoder layers run so far (their fork / join events)
  // One encoder layer (cpu_network.cpp:1027-1266, 1318-1457) on resid/act:
  // `heads` attention heads, FFN width `ffn`, LayerNorm epsilons after the
  // attention and the FFN, residual scale alpha.
  // The GEMMs around the folded LayerNorms of every body layer, as the
  // layer below sets them up (operands, lo8 codes, tiles beside the smolgen
  // chain), must each have a tile that compiles the folded epilogue.
  for (int li = 0; fold && li < d.L; ++li) {
    const Layer &L = net->layers[li];
    const int bf16 = mfh::GEMM_OUT_BF16, res = mfh::GEMM_OUT_RESID_F32;
    mfh::GemmParams pq = gemm("act", E, L.qkv_w, E, M, 3 * E, E, nullptr, mfh::ACT_NONE, bf16,
                              nullptr, nullptr, 3 * E);
    use_lo8(pq, "act", L.qkv_w);
    pq.beside_chain = L.smolgen && ws.Has("splitk_sg") && mfh::GemmWholeRoundTiles(pq);
    mfh::GemmParams pc = gemm("act", E, L.qkv_w, E, M, d.C, E, nullptr, mfh::ACT_NONE, bf16,
                              nullptr, nullptr, d.C);
    pc.small_lds = pq.beside_chain;
    mfh::GemmParams pf = gemm("act", E, L.ffn1_w, E, M, d.F, E, nullptr, d.act_ffn, bf16,
                              nullptr, nullptr, d.F);
    use_lo8(pf, "act", L.ffn1_w);
    mfh::GemmParams po = gemm("ctx", E, L.out_w, E, M, E, E, nullptr, mfh::ACT_NONE, res,
                              nullptr, nullptr, E);
    use_lo8(po, "ctx", L.out_w);
    mfh::GemmParams p2 = gemm("hid", d.F, L.ffn2_w, d.F, M, E, d.F, nullptr, mfh::ACT_NONE, res,
                              nullptr, nullptr, E);
    use_lo8(p2, "hid", L.ffn2_w);
    fold = (li == 0 || mfh::GemmLnFoldOk(pq)) && (li == 0 || !L.smolgen || mfh::GemmLnFoldOk(pc)) &&
           mfh::GemmLnFoldOk(pf) && mfh::GemmLnFoldOk(po) && mfh::GemmLnFoldOk(p2);
  }
  // LN1: the out-projection (writing x o gamma1 with its sums), FFN1 (its
  // consumer) and FFN2 (rebuilding the residual) on 64-wide tiles.  LN2:
  // FFN2 writing x o gamma2, Q|K|V and the compression (beside Q|K|V on
  // the side stream) of the next layer as its consumers.
  for (int li = 0; fold1 && li < d.L; ++li) {
    const Layer &L = net->layers[li];
    const int bf16 = mfh::GEMM_OUT_BF16, res = mfh::GEMM_OUT_RESID_F32;
    mfh::GemmParams pf = gemm("act", E, L.ffn1_w, E, M, d.F, E, nullptr, d.act_ffn, bf16,
                              nullptr, nullptr, d.F);
    mfh::GemmParams po = gemm("ctx", E, L.out_w, E, M, E, E, nullptr, mfh::ACT_NONE, res,
                              nullptr, nullptr, E);
    mfh::GemmParams p2 = gemm("hid", d.F, L.ffn2_w, d.F, M, E, d.F, nullptr, mfh::ACT_NONE, res,
                              nullptr, nullptr, E);
    const mfh::GemmParams *ps[3] = {&pf, &po, &p2};
    for (const mfh::GemmParams *q : ps)
      fold1 = fold1 && !q->A_lo8 && mfh::GemmLnFoldOk(*q);
    // (The residual tiles must be the 64-wide ones their sums assume.  FFN1
    // takes 64 x 64 tiles with the fold, also above 42 positions at the BT4
    // widths, where it takes 128 x 128 ones without it.)
    auto t128 = [&](int n) { return static_cast<long>((M + 127) / 128) * ((n + 127) / 128); };
    fold1 = fold1 && t128(E) < 256;
    if (li > 0 && fold2) {
      mfh::GemmParams pq = gemm("act", E, L.qkv_w, E, M, 3 * E, E, nullptr, mfh::ACT_NONE, bf16,
                                nullptr, nullptr, 3 * E);
      mfh::GemmParams pc = gemm("act", E, L.qkv_w, E, M, d.C, E, nullptr, mfh::ACT_NONE, bf16,
                                nullptr, nullptr, d.C);
      fold2 = !pq.A_lo8 && mfh::GemmLnFoldOk(pq) && (!L.smolgen || mfh::GemmLnFoldOk(pc));
    }
  }
  fold2 = fold2 && fold1;
  if (fold || fold2) {
    st_act = ws.S<float>("st_act");
    st_mid = ws.S<float>("st_mid");
  } else if (fold1) {
    st_mid = ws.S<float>("st_mid");
  }
  ln_part = fold ? 128 : 64;
  auto encoder_layer = [&](const Layer &L, int heads, int ffn, float eps_attn, float eps_ffn,
                           float alpha, bool body_out) -> int {
    // The smolgen chain (compression, dense1, LayerNorm, dense2, LayerNorm,
    // global projection; cpu_network.cpp:1065-1173) reads only the layer
    // input, like Q|K|V.  At large batches (M >= 2048) the compression rows
    // (3E .. 3E + C of the fused weight) run as their own GEMM and the whole
    // chain runs on the side stream while Q|K|V runs on the main stream; the
    // attention waits for both.  At small batches, where the cross-stream
    // fork and join cost more than the overlap saves, the compression stays
    // fused into the Q|K|V launch and the chain follows it on the main
    // stream.  With the stage profiler on, everything stays on the main
    // stream so each launch is timed alone.
    const int li = layer_index++;
    const bool side_chain = M >= kSmolgenSideRows;
    // Folded LayerNorms (body layers): LN1 always; the layer input is the
    // previous layer's folded LN2 from layer 1 on; LN2 is folded except
    // after the last layer, whose LayerNorm the heads read.
    const bool body = li < d.L;
    const bool fold_mid = (fold || fold1) && body;
    const bool fold_in = (fold || fold2) && body && li > 0;
    const bool fold_out = (fold || fold2) && body && !body_out;
    const Layer *prev = fold_in ? &net->layers[li - 1] : nullptr;
    // A GEMM reading LN(x) of folded rows (x o gamma with stats st): the
    // LayerNorm in its epilogue with the fold constants {fold_c, bias'}.
    auto fold_consumer = [&](mfh::GemmParams &p, const float *st, float eps,
                             const size_t (&fc)[2], size_t skip) {
      p.ln_stats = st;
      p.ln_width = E;
      p.ln_part = ln_part;
      p.ln_eps = eps;
      p.fold_c = net->W<float>(fc[0]) + skip;
      p.bias = net->W<float>(fc[1]) + skip;
    };
    // FP8 precision from 2048 rows: Q|K|V, out-projection and FFN GEMMs on
    // per-row e4m3 copies of their inputs (the smolgen chain stays bf16).
    const bool f8 = d.fp8_act && M >= 2048;
    // The no-allocation layout has one split-K buffer: the chain then runs
    // on the caller's stream (same kernels and splits, so the same bits).
    // The chain runs beside Q|K|V (its tiles then chosen to share CUs with
    // Q|K|V's) whenever the layout has its split-K buffer; with the stage
    // profiler on it runs on the main stream with the same tiles, so each
    // launch is timed alone as the graph runs it.
    const bool chain_beside = side_chain && ws.Has("splitk_sg");
    hipStream_t sg_stream = chain_beside && !net->profiling ? net->side : st;
    mfh::GemmParams pq = gemm("act", E, L.qkv_w, E, M,
                              3 * E + (L.smolgen && !side_chain ? d.C : 0), E, net->W<float>(L.qkv_b), mfh::ACT_NONE, mfh::GEMM_OUT_BF16,
                              ws.S<std::uint16_t>("qkv"), ws.Lo("qkv"), 3 * E);
    if (L.smolgen && !side_chain) {
      pq.split_n = 3 * E;
      pq.C2 = ws.S<std::uint16_t>("comp");
      pq.C2_lo = ws.Lo("comp");
      pq.ldc2 = d.C;
    }
    // Beside the chain, Q|K|V on whole-round 256 x 256 tiles takes two LDS
    // stages and the chain's GEMMs 24 KiB tiles, which then fit on the CUs
    // that hold Q|K|V workgroups.  Where Q|K|V takes 256 x 128 tiles (80
    // KiB), the chain's usual tiles already fit beside them and are faster
    // (24 KiB tiles there: batch 24 -1.6 %, 32 -1.1 %, 96 -1.4 %).
    const bool share_cus = L.smolgen && chain_beside && mfh::GemmWholeRoundTiles(pq);
    // BF16X2_FP8LO: the lo parts of Q|K|V as e4m3 codes (no fused smolgen
    // bias in that precision; Q|K|V without the compression columns).
    const bool qkv_codes = lo8 && !d.fused_bias && pq.N == 3 * E;
    pq.beside_chain = share_cus;
    mfh::AttentionParams ap;
    ap.qkv = ws.S<std::uint16_t>("qkv");
    ap.qkv_lo = ws.Lo("qkv");
    ap.batch = B;
    ap.heads = heads;
    ap.ctx = ws.S<std::uint16_t>("ctx");
    ap.ctx_lo = ws.Lo("ctx");
    if (lo8_gemm(M, E, L.out_w)) {
      ap.ctx_lo = nullptr;
      ap.ctx_lo8 = ws.S<std::uint8_t>("ctx_lo8");
    }
    if (qkv_codes) {
      ap.qkv_lo = nullptr;
      ap.qkv_lo8 = ws.S<std::uint8_t>("qkv_lo8");
    }
    // Dense1 on the flattened compression (split-K partials summed by the
    // LayerNorm kernel with bias and activation), dense2 (bias and
    // activation in its epilogue) and its LayerNorm, then the shared global
    // projection into the attention bias.
    auto smolgen_chain = [&](hipStream_t on) -> int {
      if (few_row_smolgen)
        return smolgen_few_row(L);
      float *sk = ws.S<float>(on == st ? "splitk" : "splitk_sg");
      auto chain_gemm = [&](const std::string &a, int lda, const size_t (&w)[2], int ldw, int m,
                            int n, int k, const float *bias, int mode, void *C, void *C_lo,
                            int ldc) {
        mfh::GemmParams q = gemm(a, lda, w, ldw, m, n, k, bias, mfh::ACT_NONE, mode, C, C_lo,
                                 ldc);
        q.partials = sk;
        q.small_lds = share_cus;
        return q;
      };
      // The shared global projection of the normalised dense2 rows into the
      // attention bias (unless attention projects the gen vectors itself).
      auto smolgen_global = [&](hipStream_t s) -> int {
        if (d.fused_bias)
          return MFH_OK;
        mfh::GemmParams pg = chain_gemm("sg2n", d.G, net->global_w, d.G, B * d.H,
                                        kSquares * kSquares, d.G, nullptr,
                                        d.split_attn ? mfh::GEMM_OUT_F32 : mfh::GEMM_OUT_BF16,
                                        ws.S<void>("bias"), nullptr, kSquares * kSquares);
        if (qkv_codes) {
          // BF16X2_FP8LO: the bias as bf16 hi plus the e4m3 codes of its lo
          // parts (3 bytes instead of fp32's 4, written here and read by
          // attention).
          pg.out_mode = mfh::GEMM_OUT_BF16;
          pg.C_lo8 = ws.S<std::uint8_t>("bias_lo8");
          pg.ldc8 = kSquares * kSquares;
        }
        MFH_RUN(run(pg, "smolgen_global", s));
        return MFH_OK;
      };
      if (side_chain) {
        const size_t skip = static_cast<size_t>(3) * E;  // rows of Q | K | V
        mfh::GemmParams pc = chain_gemm("act", E, L.qkv_w, E, M, d.C, E,
                                        net->W<float>(L.qkv_b) + skip, mfh::GEMM_OUT_BF16,
                                        ws.S<std::uint16_t>("comp"), ws.Lo("comp"), d.C);
        if (pc.W8) {
          pc.W8 += skip * E;
          pc.wscale += skip;
        } else {
          pc.W += skip * E;
          if (pc.wscale)  // BF16X2_FP8LO column scales
            pc.wscale += skip;
        }
        if (fold_in)
          fold_consumer(pc, st_act, eps_ffn, L.qkv_fold, skip);
        MFH_RUN(run(pc, "smolgen_compress", on));
      }
      if (few_row_dense) {
        MFH_RC(smolgen_dense_few_row(L, on, false));
        MFH_RUN(run_ln(ln(sg2, B, d.HG, 1e-3f, net->W<float>(L.sg_ln2_g),
                          net->W<float>(L.sg_ln2_b), nullptr, "sg2n"),
                       on));
        return smolgen_global(on);
      }
      const int flat = kSquares * d.C;
      mfh::GemmParams p1 = chain_gemm("comp", flat, L.sg_d1_w, flat, B, d.Hs, flat, nullptr,
                                      mfh::GEMM_OUT_F32, sg1, nullptr, d.Hs);
      p1.k_splits = SplitK(flat);
      MFH_RUN(run(p1, "smolgen_dense1", on));
      mfh::LayerNormParams l1 = ln(sg1, B, d.Hs, 1e-3f, net->W<float>(L.sg_ln1_g),
                                   net->W<float>(L.sg_ln1_b), nullptr, "sg1n");
      l1.parts = p1.k_splits;
      l1.bias = net->W<float>(L.sg_d1_b);
      l1.act = d.act_smolgen;
      MFH_RUN(run_ln(l1, on));
      // Dense2 over the whole K with its bias and activation in the GEMM
      // epilogue, spread over its 128+ workgroups; the 8192-wide LayerNorm
      // after it (one workgroup per row) then only normalises.  Measured
      // against a split-K dense2 whose partials, bias and activation that
      // LayerNorm summed: forward 1.1 % faster at batch 24, 0.6 % at 32,
      // 1.2 % at 64, 0.2 % at 256 (the LayerNorm alone 9.8 us at batch 32
      // against ~5 us for the other small kernels of the chain).
      mfh::GemmParams p2 = chain_gemm("sg1n", d.Hs, L.sg_d2_w, d.Hs, B, d.HG, d.Hs,
                                      net->W<float>(L.sg_d2_b), mfh::GEMM_OUT_F32, sg2, nullptr,
                                      d.HG);
      p2.act = d.act_smolgen;
      p2.partials = nullptr;  // no automatic split-K
      MFH_RUN(run(p2, "smolgen_dense2", on));
      MFH_RUN(run_ln(ln(sg2, B, d.HG, 1e-3f, net->W<float>(L.sg_ln2_g),
                        net->W<float>(L.sg_ln2_b), nullptr, "sg2n"),
                     on));
      return smolgen_global(on);
    };
    if (L.smolgen && !d.fused_bias) {
      ap.bias = ws.S<void>("bias");
      ap.bias_f32 = d.split_attn && !qkv_codes ? 1 : 0;
      if (qkv_codes)
        ap.bias_lo8 = ws.S<std::uint8_t>("bias_lo8");
    }
    if (L.smolgen && side_chain) {
      if (sg_stream != st) {
        MFH_HIP_CHECK(hipEventRecord(net->fork_join[2 * li], st));
        MFH_HIP_CHECK(hipStreamWaitEvent(sg_stream, net->fork_join[2 * li], 0));
      }
      const int rc = smolgen_chain(sg_stream);
      if (rc != MFH_OK)
        return rc;
      if (sg_stream != st)
        MFH_HIP_CHECK(hipEventRecord(net->fork_join[2 * li + 1], sg_stream));
    }
    if (f8) {
      MFH_RC(quant("act", E));
      use_fp8(pq, "act");
    } else if (pq.N == 3 * E) {
      use_lo8(pq, "act", L.qkv_w);
      if (qkv_codes) {
        // Attention reads the lo parts of Q|K|V as e4m3 codes.
        pq.C_lo = nullptr;
        pq.C_lo8 = ws.S<std::uint8_t>("qkv_lo8");
        pq.ldc8 = 3 * E;
      }
    }
    if (fold_in)
      fold_consumer(pq, st_act, eps_ffn, L.qkv_fold, 0);
    MFH_RUN(run(pq, "qkv"));
    if (L.smolgen && !side_chain) {
      const int rc = smolgen_chain(st);
      if (rc != MFH_OK)
        return rc;
    }
    if (L.smolgen && side_chain && sg_stream != st)
      MFH_HIP_CHECK(hipStreamWaitEvent(st, net->fork_join[2 * li + 1], 0));
    if (L.smolgen && d.fused_bias) {
      // Attention with the smolgen global projection in the kernel
      // (cpu_network.cpp:1164-1218): the gen vectors ("sg2n") against the
      // shared Wg, no bias tensor in HBM.
      mfh::AttentionSmolgenParams sp;
      sp.qkv = ap.qkv;
      sp.qkv_lo = ap.qkv_lo;
      sp.gen = ws.S<std::uint16_t>("sg2n");
      sp.gen_lo = ws.Lo("sg2n");
      if (net->fp8) {
        sp.wg8 = net->W<std::uint8_t>(net->global_w[0]);
        sp.wg_scale = net->W<float>(net->global_w[1]);
      } else {
        sp.wg = net->W<std::uint16_t>(net->global_w[0]);
      }
      sp.gen_width = d.G;
      sp.batch = B;
      sp.heads = heads;
      // Enough workgroups for the 256 CUs: one per 16 (position, head)
      // pairs and all four query tiles at large batches; the query tiles
      // split over 2 or 4 workgroups below that.
      const int groups = (B * heads + 15) / 16;
      sp.q_tiles = groups >= 256 ? 4 : groups >= 128 ? 2 : 1;
      sp.ctx = ap.ctx;
      sp.ctx_lo = ap.ctx_lo;
      const double pairs = static_cast<double>(B) * heads;
      const double flops =
          pairs * 2.0 * (2.0 * kSquares * kSquares * 32) + pairs * 2.0 * kSquares * kSquares * d.G;
      const double bytes = 2.0 * (d.split_attn ? 2.0 : 1.0) * 3.0 * M * E +
                           2.0 * plane_mult * M * E + 2.0 * (d.split_attn ? 2.0 : 1.0) * pairs * d.G;
      StageTimer t(net, st, "attention", flops, bytes);
      MFH_RUN(mfh::LaunchAttentionSmolgen(sp, st, &err_));
    } else {
      const double heads_total = static_cast<double>(B) * heads;
      const double flops = heads_total * 2.0 * (2.0 * kSquares * kSquares * 32);
      // Bytes per element: bf16 planes 2 each, e4m3 lo codes 1, fp32 4.
      const double in_b = ap.qkv_lo8 ? 3.0 : d.split_attn ? 4.0 : 2.0;
      const double out_b = ap.ctx_lo8 ? 3.0 : 2.0 * plane_mult;
      const double bias_b = ap.bias_lo8 ? 3.0 : ap.bias_f32 ? 4.0 : 2.0;
      const double bytes = in_b * 3.0 * M * E + out_b * M * E +
                           (ap.bias ? heads_total * kSquares * kSquares * bias_b : 0.0);
      StageTimer t(net, st, "attention", flops, bytes);
      MFH_RUN(mfh::LaunchAttention(ap, st, &err_));
    }
    int rc = fold_mid
                 ? residual_fold("ctx", E, L.out_w, net->W<float>(L.out_b), "out", alpha,
                                 fold_in ? st_act : nullptr,
                                 fold_in ? net->W<float>(prev->ln2_g) : nullptr,
                                 fold_in ? net->W<float>(prev->ln2_b) : nullptr, eps_ffn,
                                 net->W<float>(L.ln1_g), st_mid, eps_attn, nullptr, nullptr,
                                 nullptr)
                 : residual_ln("ctx", E, L.out_w, net->W<float>(L.out_b), "out", alpha,
                               eps_attn, net->W<float>(L.ln1_g), net->W<float>(L.ln1_b), res32,
                               f8);
    if (rc != MFH_OK)
      return rc;
    mfh::GemmParams pf = gemm("act", E, L.ffn1_w, E, M, ffn, E, net->W<float>(L.ffn1_b),
                              d.act_ffn, mfh::GEMM_OUT_BF16, ws.S<std::uint16_t>("hid"),
                              ws.Lo("hid"), ffn);
    if (f8) {
      MFH_RC(quant("act", E));
      use_fp8(pf, "act");
    } else {
      use_lo8(pf, "act", L.ffn1_w);
      if (lo8_gemm(M, E, L.ffn2_w)) {
        // FFN2 adds the fp8 lo product: FFN1 writes its lo parts as codes.
        pf.C_lo = nullptr;
        pf.C_lo8 = ws.S<std::uint8_t>("hid_lo8");
        pf.ldc8 = ffn;
      }
    }
    if (fold_mid)
      fold_consumer(pf, st_mid, eps_attn, L.ffn1_fold, 0);
    MFH_RUN(run(pf, "ffn1"));
    if (fold_mid)
      return residual_fold("hid", ffn, L.ffn2_w, net->W<float>(L.ffn2_b), "ffn2", alpha, st_mid,
                           net->W<float>(L.ln1_g), net->W<float>(L.ln1_b), eps_attn,
                           fold_out ? net->W<float>(L.ln2_g) : nullptr, st_act, eps_ffn,
                           net->W<float>(L.ln2_g), net->W<float>(L.ln2_b),
                           body_out ? resid : res32);
    rc = residual_ln("hid", ffn, L.ffn2_w, net->W<float>(L.ffn2_b), "ffn2", alpha, eps_ffn,
                     net->W<float>(L.ln2_g), net->W<float>(L.ln2_b), body_out ? resid : res32,
                     f8);
    return rc;
  };
  if (!full) {
    layer_index = only_layer;
    return encoder_layer(net->layers[only_layer], d.H, d.F, d.eps_body, d.eps_body, d.alpha,
                         false);
  }

  for (const Layer &L : net->layers) {
    const int rc = encoder_layer(L, d.H, d.F, d.eps_body, d.eps_body, d.alpha,
                                 &L == &net->layers.back());
    if (rc != MFH_OK)
      return rc;
  }


  // Heads: policy "output" | value "output" (default activation), policy
  // Q | K, attention policy map, value dense1 (flattened squares) and dense2.
  mfh::GemmParams ph = gemm("act", E, net->head_w, E, M, d.Dp + d.Vd, E,
                            net->W<float>(net->head_b), d.act_default, mfh::GEMM_OUT_BF16,
                            ws.S<std::uint16_t>("pol_emb"), ws.Lo("pol_emb"), d.Dp);
  ph.split_n = d.Dp;
  ph.C2 = ws.S<std::uint16_t>("val_emb");
  ph.C2_lo = ws.Lo("val_emb");
  ph.ldc2 = d.Vd;
  MFH_RUN(run(ph, "heads"));
  if (d.mlh)
    MFH_RUN(run(gemm("act", E, net->mov_w, E, M, d.Md, E, net->W<float>(net->mov_b),
                     d.act_default, mfh::GEMM_OUT_BF16, ws.S<std::uint16_t>("mov_emb"),
                     ws.Lo("mov_emb"), d.Md),
                "moves_left"));
  if (d.PL) {
    // Policy encoder layers run on the body output before the policy
    // "output" dense (network_execution_plan.cpp:199-200; the value and
    // moves-left heads above have already read the body output): no
    // residual scale, LayerNorm epsilons 1e-6 after attention and 1e-5 after
    // the FFN (network_execution_plan.cpp:1152-1193).
    for (const Layer &L : net->pol_layers) {
      const int rc = encoder_layer(L, d.PH, d.PF, 1e-6f, 1e-5f, 1.0f, false);
      if (rc != MFH_OK)
        return rc;
    }
    // The policy rows of the fused head weight come first.
    MFH_RUN(run(gemm("act", E, net->head_w, E, M, d.Dp, E, net->W<float>(net->head_b),
                     d.act_default, mfh::GEMM_OUT_BF16, ws.S<std::uint16_t>("pol_emb"),
                     ws.Lo("pol_emb"), d.Dp),
                "heads"));
  }
  MFH_RUN(run(gemm("pol_emb", d.Dp, net->qk_w, d.Dp, M, 2 * d.Dp, d.Dp,
                   net->W<float>(net->qk_b), mfh::ACT_NONE, mfh::GEMM_OUT_BF16,
                   ws.S<std::uint16_t>("polqk"), ws.Lo("polqk"), 2 * d.Dp),
              "policy_qk"));
  {
    StageTimer t(net, st, "policy_map", 2.0 * B * kSquares * kSquares * d.Dp,
                 2.0 * plane_mult * M * 2.0 * d.Dp + 4.0 * B * kPolicy);
    MFH_RUN(mfh::LaunchPolicyMap(ws.S<std::uint16_t>("polqk"), ws.Lo("polqk"), B, d.Dp,
                                 net->W<float>(net->promo), net->W<std::int16_t>(net->gather),
                                 policy, st, &err_));
  }
  const int vflat = kSquares * d.Vd;
  mfh::GemmParams pv = gemm("val_emb", vflat, net->val1_w, vflat, B, d.Vh, vflat, nullptr,
                            mfh::ACT_NONE, mfh::GEMM_OUT_F32, val1, nullptr, d.Vh);
  pv.k_splits = SplitK(vflat);
  MFH_RUN(run(pv, "value_dense1"));
  {
    StageTimer tv(net, st, "value_head", 0.0, 4.0 * pv.k_splits * B * d.Vh);
    MFH_RUN(mfh::LaunchValueHead(val1, pv.k_splits, net->W<float>(net->val1_b), d.act_default,
                                 B, d.Vh, net->W<float>(net->val2_w),
                                 net->W<float>(net->val2_b),
                                 d.wdl ? mfh::kHeadSoftmax3 : mfh::kHeadTanh, wdl, st, &err_));
  }
  if (d.mlh) {
    // Moves-left head (reference network_execution_plan.cpp:184-190, acts
    // 1107-1111): ip_mov on square rows (default activation), flatten,
    // ip1_mov (default activation), ip2_mov + relu.
    const int mflat = kSquares * d.Md;
    auto *mov1 = ws.S<float>("mov1");
    mfh::GemmParams pm = gemm("mov_emb", mflat, net->mov1_w, mflat, B, d.Mh, mflat, nullptr,
                              mfh::ACT_NONE, mfh::GEMM_OUT_F32, mov1, nullptr, d.Mh);
    pm.k_splits = SplitK(mflat);
    MFH_RUN(run(pm, "moves_left_dense1"));
    StageTimer tm(net, st, "moves_left_head", 0.0, 4.0 * pm.k_splits * B * d.Mh);
    MFH_RUN(mfh::LaunchValueHead(mov1, pm.k_splits, net->W<float>(net->mov1_b), d.act_default,
                                 B, d.Mh, net->W<float>(net->mov2_w),
                                 net->W<float>(net->mov2_b), mfh::kHeadRelu, moves_left, st,
                                 &err_));
  }
#undef MFH_RUN
#undef MFH_RC
  return MFH_OK;
}

void PackPlanes(const float *planes, int batch, std::uint64_t *masks, float *values) {
  // PackInputPlanesRaw (reference src/nn/input_plane_packing.h:30-83).
  for (int b = 0; b < batch; ++b)
    for (int p = 0; p < kPlanes; ++p) {
      const float *plane = planes + (static_cast<size_t>(b) * kPlanes + p) * kSquares;
      const size_t idx = static_cast<size_t>(b) * kPlanes + p;
      const bool uniform = (p < 104 && p % 13 == 12) || p == 106 || p == 107 || p >= 109;
      if (uniform) {
        values[idx] = plane[0];
        masks[idx] = plane[0] != 0.0f ? ~0ULL : 0ULL;
        continue;
      }
      std::uint64_t mask = 0;
      float value = 0.0f;
      for (int sq = 0; sq < kSquares; ++sq) {
        const float v = plane[sq];
        if (v != 0.0f) {
          if (mask == 0)
            value = v;
          mask |= 1ULL << sq;
        }
      }
      masks[idx] = mask;
      values[idx] = value;
    }
}

int CheckBatch(const mfh_net *net, int batch) {
  if (!net)
    return SetError(MFH_ERR_INVALID, "null net");
  if (batch < 1 || batch > net->max_batch) {
    std::ostringstream o;
    o << "batch " << batch << " outside 1.." << net->max_batch;
    return SetError(MFH_ERR_INVALID, o.str());
  }
  return MFH_OK;
}

// Runs the staged batch in pin_in through the device and leaves outputs in
// pin_out.  Caller holds net->mu.
void DropGraphs(mfh_net *net) {
  for (auto &kv : net->graph_execs)
    (void)hipGraphExecDestroy(kv.second);
  net->graph_execs.clear();
  net->graph_warm.clear();
}

// Orders this call's work on `st` after every earlier call's (BeginUse),
// and marks where it ends (EndUse).
int BeginUse(mfh_net *net, hipStream_t st) {
  MFH_HIP_CHECK(hipStreamWaitEvent(st, net->last_use, 0));
  return MFH_OK;
}
int EndUse(mfh_net *net, hipStream_t st) {
  MFH_HIP_CHECK(hipEventRecord(net->last_use, st));
  return MFH_OK;
}

// Graphs cached per net (batch size and device buffers as the key).
constexpr int kMaxGraphs = 64;

// Forward through a cached HIP graph (captured on the net's capture stream,
// launched on `st`), or eagerly while profiling, for a key's first run, or
// when graphs are off.  A graph bakes in the batch size and the buffers.
int RunForward(mfh_net *net, int B, const std::uint64_t *masks, const float *values,
               float *policy, float *wdl, float *moves_left, hipStream_t st) {
  if (!net->graphs || net->profiling)
    return Forward(net, MainWs(net), B, masks, values, policy, wdl, moves_left, st);
  const mfh_net::GraphKey key{B, masks, values, policy, wdl, moves_left};
  auto it = net->graph_execs.find(key);
  if (it == net->graph_execs.end()) {
    if (!net->graph_warm.count(key)) {
      if (net->graph_warm.size() >= static_cast<size_t>(16 * kMaxGraphs))
        net->graph_warm.clear();
      net->graph_warm.insert(key);
      return Forward(net, MainWs(net), B, masks, values, policy, wdl, moves_left, st);
    }
    // The cache is full: this key runs eagerly (no capture), so a caller
    // rotating through more buffer sets than the cache holds pays no
    // capture on every call, and the cached keys keep their graphs.
    if (net->graph_execs.size() >= static_cast<size_t>(kMaxGraphs))
      return Forward(net, MainWs(net), B, masks, values, policy, wdl, moves_left, st);
    hipGraph_t graph = nullptr;
    MFH_HIP_CHECK(hipStreamBeginCapture(net->capture_stream, hipStreamCaptureModeThreadLocal));
    const int rc = Forward(net, MainWs(net), B, masks, values, policy, wdl, moves_left, net->capture_stream);
    const hipError_t end = hipStreamEndCapture(net->capture_stream, &graph);
    if (rc != MFH_OK || end != hipSuccess || !graph) {
      if (graph)
        (void)hipGraphDestroy(graph);
      (void)hipGetLastError();
      // Capture is not available here: stay eager from now on.
      net->graphs = false;
      return rc != MFH_OK ? rc : Forward(net, MainWs(net), B, masks, values, policy, wdl, moves_left, st);
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (inst != hipSuccess) {
      (void)hipGetLastError();
      net->graphs = false;
      return Forward(net, MainWs(net), B, masks, values, policy, wdl, moves_left, st);
    }
    it = net->graph_execs.emplace(key, exec).first;
  }
  MFH_HIP_CHECK(hipGraphLaunch(it->second, st));
  return MFH_OK;
}

// Pinned output layout: policy [max_batch][1858] (or the priors), value head
// [max_batch][3], moves left [max_batch].
float *PinMovesLeft(mfh_net *net) {
  return reinterpret_cast<float *>(net->pin_out) +
         static_cast<size_t>(net->max_batch) * (kPolicy + 3);
}

int RunStaged(mfh_net *net, int batch) {
  const size_t n_in = static_cast<size_t>(batch) * kPlanes;
  auto *pin_masks = reinterpret_cast<std::uint64_t *>(net->pin_in);
  auto *pin_values =
      reinterpret_cast<float *>(net->pin_in + static_cast<size_t>(net->max_batch) * kPlanes * 8);
  auto *d_masks = net->S<std::uint64_t>("masks");
  auto *d_values = net->S<float>("values");
  auto *d_policy = net->S<float>("policy");
  auto *d_wdl = net->S<float>("wdl");
  MFH_HIP_CHECK(hipSetDevice(net->device));
  int rc = BeginUse(net, net->stream);
  if (rc != MFH_OK)
    return rc;
  MFH_HIP_CHECK(hipMemcpyAsync(d_masks, pin_masks, n_in * 8, hipMemcpyHostToDevice, net->stream));
  MFH_HIP_CHECK(hipMemcpyAsync(d_values, pin_values, n_in * 4, hipMemcpyHostToDevice, net->stream));
  rc = RunForward(net, batch, d_masks, d_values, d_policy, d_wdl, net->S<float>("mlh"), net->stream);
  if (rc != MFH_OK) {
    (void)EndUse(net, net->stream);
    (void)hipStreamSynchronize(net->stream);
    return rc;
  }
  auto *pin_policy = reinterpret_cast<float *>(net->pin_out);
  auto *pin_value = pin_policy + static_cast<size_t>(net->max_batch) * kPolicy;
  MFH_HIP_CHECK(hipMemcpyAsync(pin_policy, d_policy, static_cast<size_t>(batch) * kPolicy * 4,
                               hipMemcpyDeviceToHost, net->stream));
  MFH_HIP_CHECK(hipMemcpyAsync(pin_value, d_wdl, static_cast<size_t>(batch) * net->d.Vout * 4,
                               hipMemcpyDeviceToHost, net->stream));
  if (net->d.mlh)
    MFH_HIP_CHECK(hipMemcpyAsync(PinMovesLeft(net), net->S<float>("mlh"),
                                 static_cast<size_t>(batch) * 4, hipMemcpyDeviceToHost,
                                 net->stream));
  MFH_HIP_CHECK(hipEventRecord(net->last_use, net->stream));
  MFH_HIP_CHECK(hipStreamSynchronize(net->stream));
  net->last_batch = batch;
  return MFH_OK;
}

// Pinned input layout: masks, values, then the move offsets and indices of
// mfh_net_eval_priors (16-byte aligned).
size_t PinOffsetsOffset(int max_batch) {
  return AlignUp(static_cast<size_t>(max_batch) * kPlanes * 12, 16);
}
size_t PinMovesOffset(int max_batch) {
  return AlignUp(PinOffsetsOffset(max_batch) + (static_cast<size_t>(max_batch) + 1) * 4, 16);
}

// Forward plus the legal-move priors for a batch staged in pin_in (inputs,
// offsets and indices); priors land in the policy area of pin_out, the value
// head output after the max_batch policy rows as for RunStaged.
int RunStagedPriors(mfh_net *net, int batch, int total_moves, float inv_temp) {
  const size_t n_in = static_cast<size_t>(batch) * kPlanes;
  auto *d_masks = net->S<std::uint64_t>("masks");
  auto *d_values = net->S<float>("values");
  auto *d_policy = net->S<float>("policy");
  auto *d_wdl = net->S<float>("wdl");
  auto *d_offsets = net->S<std::int32_t>("move_offsets");
  auto *d_indices = net->S<std::int16_t>("move_indices");
  auto *d_priors = net->S<float>("priors");
  const unsigned char *pin = net->pin_in;
  const size_t mb = static_cast<size_t>(net->max_batch);
  MFH_HIP_CHECK(hipSetDevice(net->device));
  int rc = BeginUse(net, net->stream);
  if (rc != MFH_OK)
    return rc;
  MFH_HIP_CHECK(hipMemcpyAsync(d_masks, pin, n_in * 8, hipMemcpyHostToDevice, net->stream));
  MFH_HIP_CHECK(hipMemcpyAsync(d_values, pin + mb * kPlanes * 8, n_in * 4,
                               hipMemcpyHostToDevice, net->stream));
  MFH_HIP_CHECK(hipMemcpyAsync(d_offsets, pin + PinOffsetsOffset(net->max_batch),
                               (static_cast<size_t>(batch) + 1) * 4, hipMemcpyHostToDevice,
                               net->stream));
  if (total_moves > 0)
    MFH_HIP_CHECK(hipMemcpyAsync(d_indices, pin + PinMovesOffset(net->max_batch),
                                 static_cast<size_t>(total_moves) * 2, hipMemcpyHostToDevice,
                                 net->stream));
  rc = RunForward(net, batch, d_masks, d_values, d_policy, d_wdl, net->S<float>("mlh"), net->stream);
  if (rc == MFH_OK) {
    std::string err;
    if (mfh::LaunchPolicyPriors(d_policy, d_offsets, d_indices, batch, inv_temp, d_priors,
                           net->stream, &err) != hipSuccess)
      rc = SetError(MFH_ERR_HIP, "policy priors launch failed: " + err);
  }
  if (rc != MFH_OK) {
    (void)EndUse(net, net->stream);
    (void)hipStreamSynchronize(net->stream);
    return rc;
  }
  auto *pin_priors = reinterpret_cast<float *>(net->pin_out);
  auto *pin_value = pin_priors + mb * kPolicy;
  if (total_moves > 0)
    MFH_HIP_CHECK(hipMemcpyAsync(pin_priors, d_priors, static_cast<size_t>(total_moves) * 4,
                                 hipMemcpyDeviceToHost, net->stream));
  MFH_HIP_CHECK(hipMemcpyAsync(pin_value, d_wdl, static_cast<size_t>(batch) * net->d.Vout * 4,
                               hipMemcpyDeviceToHost, net->stream));
  if (net->d.mlh)
    MFH_HIP_CHECK(hipMemcpyAsync(PinMovesLeft(net), net->S<float>("mlh"),
                                 static_cast<size_t>(batch) * 4, hipMemcpyDeviceToHost,
                                 net->stream));
  MFH_HIP_CHECK(hipEventRecord(net->last_use, net->stream));
  MFH_HIP_CHECK(hipStreamSynchronize(net->stream));
  net->last_batch = batch;
  return MFH_OK;
}

// Move offsets must start at 0 and give each position 0..256 moves.
int CheckMoves(int batch, const std::int32_t *offsets, int *total) {
  if (!offsets)
    return SetError(MFH_ERR_INVALID, "null move offsets");
  if (offsets[0] != 0)
    return SetError(MFH_ERR_INVALID, "move offsets must start at 0");
  for (int b = 0; b < batch; ++b) {
    const std::int64_t n = static_cast<std::int64_t>(offsets[b + 1]) - offsets[b];
    if (n < 0 || n > kMaxMoves) {
      std::ostringstream o;
      o << "position " << b << " has " << n << " moves (allowed 0.." << kMaxMoves << ")";
      return SetError(MFH_ERR_INVALID, o.str());
    }
  }
  *total = offsets[batch];
  return MFH_OK;
}

int CopyOut(mfh_net *net, int batch, float *policy, float *wdl, float *moves_left) {
  const auto *pin_policy = reinterpret_cast<const float *>(net->pin_out);
  const auto *pin_value = pin_policy + static_cast<size_t>(net->max_batch) * kPolicy;
  if (policy)
    std::memcpy(policy, pin_policy, static_cast<size_t>(batch) * kPolicy * 4);
  if (wdl)
    std::memcpy(wdl, pin_value, static_cast<size_t>(batch) * net->d.Vout * 4);
  if (moves_left)
    std::memcpy(moves_left, PinMovesLeft(net), static_cast<size_t>(batch) * 4);
  return MFH_OK;
}

// moves_left may be requested only from a net with a moves-left head.
int CheckMovesLeftOut(const mfh_net *net, const float *moves_left, const char *fn) {
  if (moves_left && !net->d.mlh)
    return SetError(MFH_ERR_INVALID, std::string(fn) + ": the net has no moves-left head");
  return MFH_OK;
}

}  // namespace

extern "C" {

const char *mfh_last_error(void) { return g_last_error.c_str(); }

int mfh_device_count(int *count) {
  if (!count)
    return SetError(MFH_ERR_INVALID, "null count");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess)
    n = 0;
  *count = n;
  return MFH_OK;
}

int mfh_net_create(const mfh_net_desc *desc, const mfh_tensor *tensors, int n_tensors,
                   mfh_net **out) {
  if (!desc || !out || (n_tensors > 0 && !tensors) || n_tensors < 0)
    return SetError(MFH_ERR_INVALID, "mfh_net_create: null argument");
  *out = nullptr;
  if (desc->max_batch < 1)
    return SetError(MFH_ERR_INVALID, "max_batch must be >= 1");
  TensorMap tm;
  for (int i = 0; i < n_tensors; ++i) {
    if (!tensors[i].name)
      return SetError(MFH_ERR_INVALID, "tensor without a name");
    tm.by_name[tensors[i].name] = &tensors[i];
  }
  Loader ld{tm, {}};
  Dims dims;
  int rc = Infer(*desc, ld, dims);
  if (rc != MFH_OK)
    return rc;

  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return SetError(MFH_ERR_NO_DEVICE, "no HIP device available");
  int dev = desc->device;
  if (dev < 0)
    MFH_HIP_CHECK(hipGetDevice(&dev));
  if (dev >= ndev)
    return SetError(MFH_ERR_NO_DEVICE, "device ordinal out of range");
  hipDeviceProp_t prop;
  MFH_HIP_CHECK(hipGetDeviceProperties(&prop, dev));
  const std::string arch = prop.gcnArchName;
  if (arch.rfind("gfx950", 0) != 0)
    return SetError(MFH_ERR_NO_DEVICE, "device " + arch + " is not gfx950 (MI355X)");

  auto net = std::make_unique<mfh_net>();
  net->device = dev;
  net->d = dims;
  net->max_batch = desc->max_batch;
  net->arch = arch;
  net->device_name = prop.name;
  if (net->device_name.empty()) {
    // The marketing name comes from libdrm's amdgpu.ids table, which some
    // installs lack: describe the device from its properties instead.
    std::ostringstream o;
    o << "AMD " << arch.substr(0, arch.find(':')) << " GPU, " << prop.multiProcessorCount
      << " CUs, " << (prop.totalGlobalMem >> 30) << " GiB";
    net->device_name = o.str();
  }
  Blob blob;
  net->fp8 = desc->weights_dtype == MFH_WEIGHTS_FP8;
  rc = Pack(net.get(), ld, blob);
  if (rc != MFH_OK)
    return rc;
  PlanWorkspace(net.get());

  MFH_HIP_CHECK(hipSetDevice(dev));
  rc = ResolveScratch(dev);
  if (rc != MFH_OK)
    return rc;
  net->weight_bytes = blob.bytes.size();
  if (hipMalloc(&net->weights, net->weight_bytes) != hipSuccess)
    return SetError(MFH_ERR_OUT_OF_MEMORY, "weight upload allocation failed");
  mfh_net *raw = net.get();
  auto cleanup = [raw]() {
    if (raw->weights) (void)hipFree(raw->weights);
    if (raw->ws) (void)hipFree(raw->ws);
    if (raw->pin_in) (void)hipHostFree(raw->pin_in);
    if (raw->pin_out) (void)hipHostFree(raw->pin_out);
    if (raw->stream) (void)hipStreamDestroy(raw->stream);
    if (raw->capture_stream) (void)hipStreamDestroy(raw->capture_stream);
    if (raw->side) (void)hipStreamDestroy(raw->side);
    for (hipEvent_t e : raw->fork_join)
      (void)hipEventDestroy(e);
    raw->fork_join.clear();
    if (raw->last_use) (void)hipEventDestroy(raw->last_use);
    raw->last_use = nullptr;
    raw->weights = raw->ws = raw->pin_in = raw->pin_out = nullptr;
    raw->stream = raw->capture_stream = raw->side = nullptr;
  };
  if (hipMemcpy(net->weights, blob.bytes.data(), net->weight_bytes, hipMemcpyHostToDevice) !=
      hipSuccess) {
    cleanup();
    return SetError(MFH_ERR_HIP, "weight upload failed");
  }
  if (hipMalloc(&net->ws, net->ws_bytes) != hipSuccess) {
    cleanup();
    return SetError(MFH_ERR_OUT_OF_MEMORY, "workspace allocation failed");
  }
  const size_t in_bytes = PinMovesOffset(net->max_batch) +
                          static_cast<size_t>(net->max_batch) * kMaxMoves * 2;
  const size_t out_bytes = static_cast<size_t>(net->max_batch) * (kPolicy + 3 + 1) * 4;
  if (hipHostMalloc(reinterpret_cast<void **>(&net->pin_in), in_bytes, hipHostMallocDefault) !=
          hipSuccess ||
      hipHostMalloc(reinterpret_cast<void **>(&net->pin_out), out_bytes,
                    hipHostMallocDefault) != hipSuccess) {
    cleanup();
    return SetError(MFH_ERR_OUT_OF_MEMORY, "pinned staging allocation failed");
  }
  if (hipStreamCreateWithFlags(&net->stream, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&net->capture_stream, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&net->side, hipStreamNonBlocking) != hipSuccess) {
    cleanup();
    return SetError(MFH_ERR_HIP, "stream creation failed");
  }
  if (hipEventCreateWithFlags(&net->last_use, hipEventDisableTiming) != hipSuccess ||
      hipEventRecord(net->last_use, net->stream) != hipSuccess) {
    cleanup();
    return SetError(MFH_ERR_HIP, "event creation failed");
  }
  for (size_t i = 0; i < 2 * (net->layers.size() + net->pol_layers.size()); ++i) {
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      cleanup();
      return SetError(MFH_ERR_HIP, "event creation failed");
    }
    net->fork_join.push_back(e);
  }
  *out = net.release();
  return MFH_OK;
}

void mfh_net_destroy(mfh_net *net) {
  if (!net)
    return;
  (void)hipSetDevice(net->device);
  (void)hipDeviceSynchronize();
  DropGraphs(net);
  if (net->stream)
    (void)hipStreamDestroy(net->stream);
  if (net->capture_stream)
    (void)hipStreamDestroy(net->capture_stream);
  if (net->side)
    (void)hipStreamDestroy(net->side);
  for (hipEvent_t e : net->fork_join)
    (void)hipEventDestroy(e);
  if (net->last_use)
    (void)hipEventDestroy(net->last_use);
  (void)CollectProfile(net);
  for (hipEvent_t e : net->event_pool)
    (void)hipEventDestroy(e);
  if (net->weights) (void)hipFree(net->weights);
  if (net->ws) (void)hipFree(net->ws);
  if (net->pin_in) (void)hipHostFree(net->pin_in);
  if (net->pin_out) (void)hipHostFree(net->pin_out);
  delete net;
}

int mfh_net_eval(mfh_net *net, int batch, const uint64_t *masks, const float *values,
                 float *policy, float *wdl, float *moves_left) {
  int rc = CheckBatch(net, batch);
  if (rc != MFH_OK)
    return rc;
  if (!masks || !values || !policy || !wdl)
    return SetError(MFH_ERR_INVALID, "mfh_net_eval: bad output/input pointers");
  rc = CheckMovesLeftOut(net, moves_left, "mfh_net_eval");
  if (rc != MFH_OK)
    return rc;
  std::lock_guard<std::mutex> lock(net->mu);
  const size_t n_in = static_cast<size_t>(batch) * kPlanes;
  std::memcpy(net->pin_in, masks, n_in * 8);
  std::memcpy(net->pin_in + static_cast<size_t>(net->max_batch) * kPlanes * 8, values, n_in * 4);
  rc = RunStaged(net, batch);
  if (rc != MFH_OK)
    return rc;
  return CopyOut(net, batch, policy, wdl, moves_left);
}

int mfh_net_eval_planes(mfh_net *net, int batch, const float *planes, float *policy,
                        float *wdl, float *moves_left) {
  int rc = CheckBatch(net, batch);
  if (rc != MFH_OK)
    return rc;
  if (!planes || !policy || !wdl)
    return SetError(MFH_ERR_INVALID, "mfh_net_eval_planes: bad output/input pointers");
  rc = CheckMovesLeftOut(net, moves_left, "mfh_net_eval_planes");
  if (rc != MFH_OK)
    return rc;
  std::lock_guard<std::mutex> lock(net->mu);
  PackPlanes(planes, batch, reinterpret_cast<std::uint64_t *>(net->pin_in),
             reinterpret_cast<float *>(net->pin_in +
                                       static_cast<size_t>(net->max_batch) * kPlanes * 8));
  rc = RunStaged(net, batch);
  if (rc != MFH_OK)
    return rc;
  return CopyOut(net, batch, policy, wdl, moves_left);
}

int mfh_net_eval_device(mfh_net *net, int batch, const uint64_t *d_masks,
                        const float *d_values, float *d_policy, float *d_wdl, void *stream) {
  int rc = CheckBatch(net, batch);
  if (rc != MFH_OK)
    return rc;
  if (!d_masks || !d_values || !d_policy || !d_wdl)
    return SetError(MFH_ERR_INVALID, "mfh_net_eval_device: null pointer");
  std::lock_guard<std::mutex> lock(net->mu);
  MFH_HIP_CHECK(hipSetDevice(net->device));
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = BeginUse(net, st);
  if (rc != MFH_OK)
    return rc;
  rc = RunForward(net, batch, d_masks, d_values, d_policy, d_wdl, net->S<float>("mlh"), st);
  const int end = EndUse(net, st);
  if (rc == MFH_OK)
    rc = end;
  if (rc == MFH_OK)
    net->last_batch = batch;
  return rc;
}

int mfh_net_eval_device_moves_left(mfh_net *net, int batch, const uint64_t *d_masks,
                                   const float *d_values, float *d_policy, float *d_wdl,
                                   float *d_moves_left, void *stream) {
  int rc = CheckBatch(net, batch);
  if (rc != MFH_OK)
    return rc;
  if (!d_masks || !d_values || !d_policy || !d_wdl || !d_moves_left)
    return SetError(MFH_ERR_INVALID, "mfh_net_eval_device_moves_left: null pointer");
  rc = CheckMovesLeftOut(net, d_moves_left, "mfh_net_eval_device_moves_left");
  if (rc != MFH_OK)
    return rc;
  std::lock_guard<std::mutex> lock(net->mu);
  MFH_HIP_CHECK(hipSetDevice(net->device));
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = BeginUse(net, st);
  if (rc != MFH_OK)
    return rc;
  rc = RunForward(net, batch, d_masks, d_values, d_policy, d_wdl, d_moves_left, st);
  const int end = EndUse(net, st);
  if (rc == MFH_OK)
    rc = end;
  if (rc == MFH_OK)
    net->last_batch = batch;
  return rc;
}

int mfh_net_eval_device_noalloc(mfh_net *net, int batch, const uint64_t *d_masks,
                                const float *d_values, float *d_policy, float *d_wdl,
                                void *stream) {
  if (!net)
    return SetError(MFH_ERR_INVALID, "null net");
  if (!d_masks || !d_values || !d_policy || !d_wdl)
    return SetError(MFH_ERR_INVALID, "mfh_net_eval_device_noalloc: null pointer");
  if (batch < 1 || batch > net->noalloc_max_batch) {
    std::ostringstream o;
    o << "mfh_net_eval_device_noalloc: batch " << batch << " outside 1.."
      << net->noalloc_max_batch << " (the largest batch below " << kNoAllocMaxBatch + 1
      << " whose workspace fits the " << (kScratchBytes >> 20) << " MiB scratch array)";
    return SetError(MFH_ERR_INVALID, o.str());
  }
  std::lock_guard<std::mutex> lock(net->mu);
  unsigned char *base = ScratchAddress(net->device);
  if (!base)
    return SetError(MFH_ERR_HIP, "scratch array address not resolved on this device");
  MFH_HIP_CHECK(hipSetDevice(net->device));
  // The forward writes every workspace element it reads, so nothing in the
  // scratch array needs clearing between calls.
  const WsView ws{base, &net->noalloc_off, kSmallSplitKFloats};
  net->noalloc_call = true;
  int rc;
  try {
    rc = Forward(net, ws, batch, d_masks, d_values, d_policy, d_wdl, ws.S<float>("mlh"),
                 static_cast<hipStream_t>(stream));
  } catch (const std::exception &e) {
    rc = SetError(MFH_ERR_INVALID, std::string("mfh_net_eval_device_noalloc: ") + e.what());
  }
  net->noalloc_call = false;
  return rc;
}

int mfh_net_eval_priors(mfh_net *net, int batch, const uint64_t *masks, const float *values,
                        const int32_t *move_offsets, const int16_t *move_indices,
                        float softmax_temp, float *priors, float *wdl, float *moves_left) {
  int rc = CheckBatch(net, batch);
  if (rc != MFH_OK)
    return rc;
  if (!masks || !values || !wdl)
    return SetError(MFH_ERR_INVALID, "mfh_net_eval_priors: bad output/input pointers");
  rc = CheckMovesLeftOut(net, moves_left, "mfh_net_eval_priors");
  if (rc != MFH_OK)
    return rc;
  int total = 0;
  rc = CheckMoves(batch, move_offsets, &total);
  if (rc != MFH_OK)
    return rc;
  if (total > 0 && (!move_indices || !priors))
    return SetError(MFH_ERR_INVALID, "mfh_net_eval_priors: null move indices or priors");
  std::lock_guard<std::mutex> lock(net->mu);
  const size_t n_in = static_cast<size_t>(batch) * kPlanes;
  const size_t mb = static_cast<size_t>(net->max_batch);
  std::memcpy(net->pin_in, masks, n_in * 8);
  std::memcpy(net->pin_in + mb * kPlanes * 8, values, n_in * 4);
  std::memcpy(net->pin_in + PinOffsetsOffset(net->max_batch), move_offsets,
              (static_cast<size_t>(batch) + 1) * 4);
  if (total > 0)
    std::memcpy(net->pin_in + PinMovesOffset(net->max_batch), move_indices,
                static_cast<size_t>(total) * 2);
  // ApplyNNPolicyToNode (search.cpp:133) multiplies by 1 / temperature.
  rc = RunStagedPriors(net, batch, total, 1.0f / softmax_temp);
  if (rc != MFH_OK)
    return rc;
  const auto *pin_priors = reinterpret_cast<const float *>(net->pin_out);
  if (total > 0)
    std::memcpy(priors, pin_priors, static_cast<size_t>(total) * 4);
  std::memcpy(wdl, pin_priors + mb * kPolicy, static_cast<size_t>(batch) * net->d.Vout * 4);
  if (moves_left)
    std::memcpy(moves_left, PinMovesLeft(net), static_cast<size_t>(batch) * 4);
  return MFH_OK;
}

int mfh_net_eval_priors_device(mfh_net *net, int batch, const uint64_t *d_masks,
                               const float *d_values, const int32_t *d_move_offsets,
                               const int16_t *d_move_indices, float softmax_temp,
                               float *d_policy, float *d_priors, float *d_wdl, void *stream) {
  int rc = CheckBatch(net, batch);
  if (rc != MFH_OK)
    return rc;
  if (!d_masks || !d_values || !d_move_offsets || !d_move_indices || !d_policy || !d_priors ||
      !d_wdl)
    return SetError(MFH_ERR_INVALID, "mfh_net_eval_priors_device: null pointer");
  std::lock_guard<std::mutex> lock(net->mu);
  MFH_HIP_CHECK(hipSetDevice(net->device));
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = BeginUse(net, st);
  if (rc != MFH_OK)
    return rc;
  rc = RunForward(net, batch, d_masks, d_values, d_policy, d_wdl, net->S<float>("mlh"), st);
  if (rc == MFH_OK) {
    std::string err;
    if (mfh::LaunchPolicyPriors(d_policy, d_move_offsets, d_move_indices, batch,
                                1.0f / softmax_temp, d_priors, st, &err) != hipSuccess)
      rc = SetError(MFH_ERR_HIP, "policy priors launch failed: " + err);
  }
  const int end = EndUse(net, st);
  if (rc == MFH_OK)
    rc = end;
  if (rc == MFH_OK)
    net->last_batch = batch;
  return rc;
}

int mfh_net_info(const mfh_net *net, char *buf, size_t len) {
  if (!net || !buf || !len)
    return SetError(MFH_ERR_INVALID, "mfh_net_info: null argument");
  const Dims &d = net->d;
  std::ostringstream o;
  o << "HIP transformer backend (" << net->arch << ", " << net->device_name
    << "): attention body E=" << d.E << " L=" << d.L << " H=" << d.H << " FFN=" << d.F
    << " PE=" << d.P << (d.gates ? " gates" : "") << (d.input_ffn ? " input-ffn" : "");
  if (d.smolgen)
    o << " smolgen C=" << d.C << "/" << d.Hs << "/" << d.G
      << (d.fused_bias ? " (bias in attention)" : " (bias tensor)");
  o << ", policy attention Dp=" << d.Dp << ", value " << (d.wdl ? "wdl" : "scalar") << " "
    << d.Vd << "/" << d.Vh;
  if (d.mlh)
    o << ", moves left " << d.Md << "/" << d.Mh;
  o << ", activations " << ActName(d.act_default) << "/"
    << ActName(d.act_smolgen) << "/" << ActName(d.act_ffn) << ", precision "
    << (d.lo8          ? "bf16x2_fp8lo"
        : d.split_attn ? "bf16x2"
        : d.split      ? "bf16x2_gemm"
        : d.fp8_act    ? "fp8"
                       : "bf16")
    << ", weights "
    << (net->fp8 ? "e4m3 " : "bf16 ") << net->weight_bytes << " B, workspace " << net->ws_bytes << " B, max_batch "
    << net->max_batch << ", no-allocation batch <= " << net->noalloc_max_batch;
  const std::string s = o.str();
  std::snprintf(buf, len, "%s", s.c_str());
  return MFH_OK;
}

int mfh_net_capabilities(const mfh_net *net, mfh_capabilities *out) {
  if (!net || !out)
    return SetError(MFH_ERR_INVALID, "mfh_net_capabilities: null argument");
  std::memset(out, 0, sizeof(*out));
  out->has_wdl = net->d.wdl ? 1 : 0;
  out->has_moves_left = net->d.mlh ? 1 : 0;
  out->max_batch_size = net->max_batch;
  out->device = net->device;
  std::snprintf(out->device_name, sizeof(out->device_name), "%s", net->device_name.c_str());
  std::snprintf(out->arch_name, sizeof(out->arch_name), "%s", net->arch.c_str());
  out->weight_bytes = net->weight_bytes;
  out->workspace_bytes = net->ws_bytes;
  return MFH_OK;
}

int mfh_net_debug_tensor(mfh_net *net, const char *name, void *out, uint64_t bytes) {
  if (!net || !name || !out)
    return SetError(MFH_ERR_INVALID, "mfh_net_debug_tensor: null argument");
  std::lock_guard<std::mutex> lock(net->mu);
  const size_t B = static_cast<size_t>(net->last_batch);
  const Dims &d = net->d;
  const char *ws_name = nullptr;
  size_t size = 0;
  const std::string n = name;
  if (n == "body") {
    ws_name = "resid";
    size = B * kSquares * d.E * 4;
  } else if (n == "policy_qk") {
    ws_name = "polqk";
    size = B * kSquares * 2 * d.Dp * 2;
  } else if (n == "act" || n == "ctx") {
    ws_name = n == "act" ? "act" : "ctx";
    size = B * kSquares * d.E * 2;
  } else if (n == "qkv") {
    ws_name = "qkv";
    size = B * kSquares * 3 * d.E * 2;
  } else if (n == "hid") {
    ws_name = "hid";
    size = B * kSquares * d.F * 2;
  } else if (n == "pre") {
    ws_name = "pre";
    size = B * kSquares * d.E * 4;
  } else if (d.fp8_act && (n == "act_e4m3" || n == "ctx_e4m3" || n == "hid_e4m3")) {
    ws_name = n == "act_e4m3" ? "act8" : n == "ctx_e4m3" ? "ctx8" : "hid8";
    size = B * kSquares * (n == "hid_e4m3" ? d.F : d.E);
  } else if (d.fp8_act && (n == "act_scale" || n == "ctx_scale" || n == "hid_scale")) {
    ws_name = n == "act_scale" ? "sc_act" : n == "ctx_scale" ? "sc_ctx" : "sc_hid";
    size = B * kSquares * 4;
  } else {
    return SetError(MFH_ERR_INVALID, "unknown debug tensor " + n);
  }
  if (B == 0 || bytes != size)
    return SetError(MFH_ERR_INVALID, "debug tensor size mismatch");
  MFH_HIP_CHECK(hipSetDevice(net->device));
  MFH_HIP_CHECK(hipEventSynchronize(net->last_use));
  MFH_HIP_CHECK(hipMemcpy(out, net->ws + net->ws_off.at(ws_name), size, hipMemcpyDeviceToHost));
  return MFH_OK;
}

int mfh_debug_encoder_layer(mfh_net *net, int batch, int layer, int iterations,
                            const uint16_t *x, const uint16_t *x_lo, float *ms) {
  int rc = CheckBatch(net, batch);
  if (rc != MFH_OK)
    return rc;
  if (layer < 0 || layer >= static_cast<int>(net->layers.size()) || iterations < 1 || !x ||
      !ms || (net->d.split && !x_lo))
    return SetError(MFH_ERR_INVALID, "mfh_debug_encoder_layer: bad arguments");
  std::lock_guard<std::mutex> lock(net->mu);
  MFH_HIP_CHECK(hipSetDevice(net->device));
  const WsView ws = MainWs(net);
  const size_t n = static_cast<size_t>(batch) * kSquares * net->d.E;
  hipStream_t st = net->stream;
  rc = BeginUse(net, st);
  if (rc != MFH_OK)
    return rc;
  // The copies below are synchronous on the null stream, which does not wait
  // for a non-blocking caller stream: wait for the last call's device work
  // on the workspace first.
  MFH_HIP_CHECK(hipEventSynchronize(net->last_use));
  // The layer's input: the residual stream's bf16 planes and, in single
  // precision, its fp32 copy.
  MFH_HIP_CHECK(hipMemcpy(ws.S<std::uint16_t>("act"), x, n * 2, hipMemcpyHostToDevice));
  if (net->d.split) {
    MFH_HIP_CHECK(hipMemcpy(ws.Lo("act"), x_lo, n * 2, hipMemcpyHostToDevice));
    if (net->d.lo8 && batch * kSquares >= kLo8MinRows && ws.Has("act_lo8")) {
      // BF16X2_FP8LO: the lo plane's e4m3 codes (lo * 2^kLo8Shift).
      std::vector<std::uint8_t> codes(n);
      for (size_t i = 0; i < n; ++i) {
        const std::uint32_t u = static_cast<std::uint32_t>(x_lo[i]) << 16;
        float f;
        std::memcpy(&f, &u, 4);
        codes[i] = EncodeE4m3(f * static_cast<float>(1 << mfh::kLo8Shift));
      }
      MFH_HIP_CHECK(hipMemcpy(ws.S<std::uint8_t>("act_lo8"), codes.data(), n,
                              hipMemcpyHostToDevice));
    }
  } else {
    std::vector<float> x32(n);
    for (size_t i = 0; i < n; ++i) {
      const std::uint32_t u = static_cast<std::uint32_t>(x[i]) << 16;
      std::memcpy(&x32[i], &u, 4);
    }
    MFH_HIP_CHECK(hipMemcpy(ws.S<float>("resid"), x32.data(), n * 4, hipMemcpyHostToDevice));
  }
  hipEvent_t a = nullptr, z = nullptr;
  MFH_HIP_CHECK(hipEventCreate(&a));
  MFH_HIP_CHECK(hipEventCreate(&z));
  (void)hipEventRecord(a, st);
  for (int i = 0; i < iterations && rc == MFH_OK; ++i)
    rc = Forward(net, ws, batch, nullptr, nullptr, nullptr, nullptr, nullptr, st, layer);
  (void)hipEventRecord(z, st);
  (void)EndUse(net, st);
  const hipError_t sync = hipEventSynchronize(z);
  float elapsed = 0.f;
  if (rc == MFH_OK && sync == hipSuccess && hipEventElapsedTime(&elapsed, a, z) == hipSuccess)
    *ms = elapsed / static_cast<float>(iterations);
  else if (rc == MFH_OK)
    rc = SetError(MFH_ERR_HIP, "mfh_debug_encoder_layer: timing failed");
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(z);
  if (rc == MFH_OK)
    net->last_batch = batch;
  return rc;
}

int mfh_net_set_graphs(mfh_net *net, int enabled) {
  if (!net)
    return SetError(MFH_ERR_INVALID, "null net");
  std::lock_guard<std::mutex> lock(net->mu);
  MFH_HIP_CHECK(hipSetDevice(net->device));
  MFH_HIP_CHECK(hipDeviceSynchronize());
  DropGraphs(net);
  net->graphs = enabled != 0;
  return MFH_OK;
}

int mfh_net_set_profiling(mfh_net *net, int enabled) {
  if (!net)
    return SetError(MFH_ERR_INVALID, "null net");
  std::lock_guard<std::mutex> lock(net->mu);
  net->profiling = enabled != 0;
  return MFH_OK;
}

int mfh_net_profile_reset(mfh_net *net) {
  if (!net)
    return SetError(MFH_ERR_INVALID, "null net");
  std::lock_guard<std::mutex> lock(net->mu);
  MFH_HIP_CHECK(hipSetDevice(net->device));
  const int rc = CollectProfile(net);
  net->totals.clear();
  return rc;
}

int mfh_net_profile(mfh_net *net, mfh_profile_entry *out, int capacity, int *count) {
  if (!net || !count || (capacity > 0 && !out))
    return SetError(MFH_ERR_INVALID, "mfh_net_profile: bad arguments");
  std::lock_guard<std::mutex> lock(net->mu);
  MFH_HIP_CHECK(hipSetDevice(net->device));
  const int rc = CollectProfile(net);
  if (rc != MFH_OK)
    return rc;
  int n = 0;
  for (const auto &kv : net->totals) {
    if (n < capacity) {
      mfh_profile_entry &e = out[n];
      std::memset(&e, 0, sizeof(e));
      std::snprintf(e.name, sizeof(e.name), "%s", kv.first.c_str());
      e.launches = kv.second.launches;
      e.milliseconds = kv.second.ms;
      e.flops = kv.second.flops;
      e.bytes = kv.second.bytes;
    }
    ++n;
  }
  *count = n;
  return MFH_OK;
}

int mfh_pack_planes(int batch, const float *planes, uint64_t *masks, float *values) {
  if (batch < 0 || (batch > 0 && (!planes || !masks || !values)))
    return SetError(MFH_ERR_INVALID, "mfh_pack_planes: bad arguments");
  PackPlanes(planes, batch, masks, values);
  return MFH_OK;
}

int mfh_debug_unpack_planes(int batch, const uint64_t *masks, const float *values,
                            float *planes) {
  if (batch <= 0 || !masks || !values || !planes)
    return SetError(MFH_ERR_INVALID, "mfh_debug_unpack_planes: bad arguments");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return SetError(MFH_ERR_NO_DEVICE, "no HIP device available");
  const size_t n = static_cast<size_t>(batch) * kPlanes;
  const size_t np = n * kSquares;
  std::uint64_t *dm = nullptr;
  float *dv = nullptr, *dp = nullptr;
  MFH_HIP_CHECK(hipMalloc(&dm, n * 8));
  MFH_HIP_CHECK(hipMalloc(&dv, n * 4));
  MFH_HIP_CHECK(hipMalloc(&dp, np * 4));
  int rc = MFH_OK;
  std::string err;
  if (hipMemcpy(dm, masks, n * 8, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(dv, values, n * 4, hipMemcpyHostToDevice) != hipSuccess)
    rc = SetError(MFH_ERR_HIP, "copy failed");
  else if (mfh::LaunchUnpackPlanes(dm, dv, batch, dp, nullptr, &err) != hipSuccess)
    rc = SetError(MFH_ERR_HIP, err);
  else if (hipMemcpy(planes, dp, np * 4, hipMemcpyDeviceToHost) != hipSuccess)
    rc = SetError(MFH_ERR_HIP, "copy back failed");
  (void)hipFree(dm);
  (void)hipFree(dv);
  (void)hipFree(dp);
  return rc;
}

int mfh_debug_quantize_fp8(int rows, int cols, const float *w, uint8_t *codes, float *scale) {
  if (rows <= 0 || cols <= 0 || !w || !codes || !scale)
    return SetError(MFH_ERR_INVALID, "mfh_debug_quantize_fp8: bad arguments");
  for (int r = 0; r < rows; ++r)
    QuantizeRowE4m3(w + static_cast<size_t>(r) * cols, cols, codes + static_cast<size_t>(r) * cols,
                    scale + r);
  return MFH_OK;
}

// ---- Network files ----------------------------------------------------------

static int WrapWeights(mfh::wf::Weights &&w, mfh_weights **out) {
  auto *h = new (std::nothrow) mfh_weights;
  if (!h)
    return SetError(MFH_ERR_OUT_OF_MEMORY, "out of host memory");
  h->w = std::move(w);
  h->views.reserve(h->w.tensors.size());
  for (const auto &t : h->w.tensors)
    h->views.push_back(mfh_tensor{t.name.c_str(), t.data.data(), t.data.size()});
  *out = h;
  return MFH_OK;
}

int mfh_weights_load(const char *path, mfh_weights **out) {
  if (!path || !out)
    return SetError(MFH_ERR_INVALID, "mfh_weights_load: bad arguments");
  *out = nullptr;
  try {
    return WrapWeights(mfh::wf::LoadFile(path), out);
  } catch (const std::bad_alloc &) {
    return SetError(MFH_ERR_OUT_OF_MEMORY, "out of host memory reading " + std::string(path));
  } catch (const std::exception &e) {
    return SetError(MFH_ERR_INVALID, e.what());
  }
}

int mfh_weights_parse(const void *data, uint64_t bytes, mfh_weights **out) {
  if ((!data && bytes) || !out)
    return SetError(MFH_ERR_INVALID, "mfh_weights_parse: bad arguments");
  *out = nullptr;
  try {
    if (bytes < 2)
      throw std::runtime_error("Invalid weight file: too small");
    return WrapWeights(mfh::wf::Parse(static_cast<const uint8_t *>(data), bytes), out);
  } catch (const std::bad_alloc &) {
    return SetError(MFH_ERR_OUT_OF_MEMORY, "out of host memory");
  } catch (const std::exception &e) {
    return SetError(MFH_ERR_INVALID, e.what());
  }
}

int mfh_weights_describe(const mfh_weights *w, mfh_weights_format *format, mfh_net_desc *desc) {
  if (!w)
    return SetError(MFH_ERR_INVALID, "mfh_weights_describe: null weights");
  const auto &f = w->w.format;
  if (format) {
    format->input = f.input;
    format->output = f.output;
    format->network = f.network;
    format->policy = f.policy;
    format->value = f.value;
    format->moves_left = f.moves_left;
    format->default_activation = f.default_activation;
    format->smolgen_activation = f.smolgen_activation;
    format->ffn_activation = f.ffn_activation;
    format->input_embedding = f.input_embedding;
    format->headcount = static_cast<int>(w->w.headcount);
    format->pol_headcount = static_cast<int>(w->w.pol_headcount);
  }
  if (desc) {
    desc->network = f.network;
    desc->policy = f.policy;
    desc->value = f.value;
    desc->moves_left = f.moves_left;
    desc->input_embedding = f.input_embedding;
    desc->default_activation = f.default_activation;
    desc->ffn_activation = f.ffn_activation;
    desc->smolgen_activation = f.smolgen_activation;
    desc->headcount = static_cast<int>(w->w.headcount);
    desc->pol_headcount = static_cast<int>(w->w.pol_headcount);
  }
  return MFH_OK;
}

int mfh_weights_tensors(const mfh_weights *w, const mfh_tensor **tensors, int *count) {
  if (!w || !tensors || !count)
    return SetError(MFH_ERR_INVALID, "mfh_weights_tensors: bad arguments");
  *tensors = w->views.data();
  *count = static_cast<int>(w->views.size());
  return MFH_OK;
}

int mfh_weights_tensor_dims(const mfh_weights *w, int index, const uint32_t **dims, int *ndims) {
  if (!w || !dims || !ndims || index < 0 || index >= static_cast<int>(w->w.tensors.size()))
    return SetError(MFH_ERR_INVALID, "mfh_weights_tensor_dims: bad arguments");
  *dims = w->w.tensors[index].dims.data();
  *ndims = static_cast<int>(w->w.tensors[index].dims.size());
  return MFH_OK;
}

void mfh_weights_free(mfh_weights *w) { delete w; }

int mfh_debug_gemm_bf16(int M, int N, int K, const uint16_t *A, const uint16_t *W,
                        const float *bias, int act, float *C) {
  if (M <= 0 || N <= 0 || K <= 0 || !A || !W || !C)
    return SetError(MFH_ERR_INVALID, "mfh_debug_gemm_bf16: bad arguments");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return SetError(MFH_ERR_NO_DEVICE, "no HIP device available");
  std::uint16_t *dA = nullptr, *dW = nullptr;
  float *dB = nullptr, *dC = nullptr;
  const size_t na = static_cast<size_t>(M) * K, nw = static_cast<size_t>(N) * K,
               nc = static_cast<size_t>(M) * N;
  MFH_HIP_CHECK(hipMalloc(&dA, na * 2));
  MFH_HIP_CHECK(hipMalloc(&dW, nw * 2));
  MFH_HIP_CHECK(hipMalloc(&dC, nc * 4));
  if (bias)
    MFH_HIP_CHECK(hipMalloc(&dB, static_cast<size_t>(N) * 4));
  int rc = MFH_OK;
  std::string err;
  mfh::GemmParams p;
  p.A = dA;
  p.lda = K;
  p.W = dW;
  p.ldw = K;
  p.M = M;
  p.N = N;
  p.K = K;
  p.bias = dB;
  p.act = ActFromProto(act, mfh::ACT_RELU);
  if (act == MFH_ACTIVATION_NONE || act == MFH_ACTIVATION_DEFAULT)
    p.act = mfh::ACT_NONE;
  p.out_mode = mfh::GEMM_OUT_F32;
  p.C = dC;
  p.ldc = N;
  if (hipMemcpy(dA, A, na * 2, hipMemcpyHostToDevice) != hipSuccess ||
      hipMemcpy(dW, W, nw * 2, hipMemcpyHostToDevice) != hipSuccess ||
      (bias && hipMemcpy(dB, bias, static_cast<size_t>(N) * 4, hipMemcpyHostToDevice) !=
                   hipSuccess))
    rc = SetError(MFH_ERR_HIP, "copy failed");
  else if (mfh::LaunchGemm(p, nullptr, &err) != hipSuccess)
    rc = SetError(MFH_ERR_INVALID, err);
  else if (hipDeviceSynchronize() != hipSuccess ||
           hipMemcpy(C, dC, nc * 4, hipMemcpyDeviceToHost) != hipSuccess)
    rc = SetError(MFH_ERR_HIP, "gemm execution failed");
  (void)hipFree(dA);
  (void)hipFree(dW);
  (void)hipFree(dC);
  if (dB)
    (void)hipFree(dB);
  return rc;
}

}  // extern "C"

// Device copies of host arrays for the debug entry points; frees on exit.
struct DebugBuffers {
  std::vector<void *> ptrs;
  ~DebugBuffers() {
    for (void *q : ptrs)
      (void)hipFree(q);
  }
  // Device buffer of `bytes`, filled from `host` when given; null for a null
  // host array when `keep_null`.
  template <typename T>
  T *Put(const T *host, size_t count, bool keep_null = true) {
    if (!host && keep_null)
      return nullptr;
    void *d = nullptr;
    if (hipMalloc(&d, count * sizeof(T)) != hipSuccess)
      throw std::runtime_error("hipMalloc failed");
    ptrs.push_back(d);
    if (host && hipMemcpy(d, host, count * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
      throw std::runtime_error("copy to device failed");
    return static_cast<T *>(d);
  }
};

int mfh_debug_gemm_fp8(int M, int N, int K, const uint8_t *A8, const float *ascale,
                       const uint8_t *W8, const float *wscale, const float *bias, int act,
                       float *C) {
  if (M <= 0 || N <= 0 || K <= 0 || !A8 || !ascale || !W8 || !wscale || !C)
    return SetError(MFH_ERR_INVALID, "mfh_debug_gemm_fp8: bad arguments");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return SetError(MFH_ERR_NO_DEVICE, "no HIP device available");
  const size_t na = static_cast<size_t>(M) * K, nw = static_cast<size_t>(N) * K,
               nc = static_cast<size_t>(M) * N;
  try {
    DebugBuffers buf;
    mfh::GemmParams p;
    p.A8 = buf.Put(A8, na);
    p.ascale = buf.Put(ascale, M);
    p.lda = K;
    p.W8 = buf.Put(W8, nw);
    p.wscale = buf.Put(wscale, N);
    p.ldw = K;
    p.M = M;
    p.N = N;
    p.K = K;
    p.bias = buf.Put(bias, N);
    p.act = ActFromProto(act, mfh::ACT_RELU);
    if (act == MFH_ACTIVATION_NONE || act == MFH_ACTIVATION_DEFAULT)
      p.act = mfh::ACT_NONE;
    p.out_mode = mfh::GEMM_OUT_F32;
    p.C = buf.Put<float>(nullptr, nc, false);
    p.ldc = N;
    std::string err;
    if (mfh::LaunchGemm(p, nullptr, &err) != hipSuccess)
      return SetError(MFH_ERR_INVALID, err);
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(C, p.C, nc * 4, hipMemcpyDeviceToHost) != hipSuccess)
      return SetError(MFH_ERR_HIP, "fp8 gemm execution failed");
  } catch (const std::exception &e) {
    return SetError(MFH_ERR_HIP, e.what());
  }
  return MFH_OK;
}

int mfh_debug_gemm_lo8(int M, int N, int K, const uint16_t *A, const uint8_t *A_lo8,
                       const uint16_t *W, const uint8_t *W_lo8, const float *wscale,
                       const float *bias, int act, float *C, uint16_t *C_hi, uint8_t *C_lo8) {
  if (M <= 0 || N <= 0 || K <= 0 || !A || !A_lo8 || !W || !W_lo8 || !wscale ||
      (!C && !(C_hi && C_lo8)) || (C && (C_hi || C_lo8)))
    return SetError(MFH_ERR_INVALID, "mfh_debug_gemm_lo8: bad arguments");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return SetError(MFH_ERR_NO_DEVICE, "no HIP device available");
  const size_t na = static_cast<size_t>(M) * K, nw = static_cast<size_t>(N) * K,
               nc = static_cast<size_t>(M) * N;
  try {
    DebugBuffers buf;
    mfh::GemmParams p;
    p.A = buf.Put(A, na);
    p.lda = K;
    p.A_lo8 = buf.Put(A_lo8, na);
    p.lda8 = K;
    p.W = buf.Put(W, nw);
    p.ldw = K;
    p.W_lo8 = buf.Put(W_lo8, nw);
    p.ldw8 = K;
    p.wscale = buf.Put(wscale, N);
    p.M = M;
    p.N = N;
    p.K = K;
    p.bias = buf.Put(bias, N);
    p.act = ActFromProto(act, mfh::ACT_RELU);
    if (act == MFH_ACTIVATION_NONE || act == MFH_ACTIVATION_DEFAULT)
      p.act = mfh::ACT_NONE;
    if (C) {
      p.out_mode = mfh::GEMM_OUT_F32;
      p.C = buf.Put<float>(nullptr, nc, false);
    } else {
      p.out_mode = mfh::GEMM_OUT_BF16;
      p.C = buf.Put<std::uint16_t>(nullptr, nc, false);
      p.C_lo8 = buf.Put<std::uint8_t>(nullptr, nc, false);
      p.ldc8 = N;
    }
    p.ldc = N;
    std::string err;
    if (mfh::LaunchGemm(p, nullptr, &err) != hipSuccess)
      return SetError(MFH_ERR_INVALID, err);
    if (hipDeviceSynchronize() != hipSuccess)
      return SetError(MFH_ERR_HIP, "fp8 lo-correction gemm execution failed");
    if (C ? hipMemcpy(C, p.C, nc * 4, hipMemcpyDeviceToHost) != hipSuccess
          : (hipMemcpy(C_hi, p.C, nc * 2, hipMemcpyDeviceToHost) != hipSuccess ||
             hipMemcpy(C_lo8, p.C_lo8, nc, hipMemcpyDeviceToHost) != hipSuccess))
      return SetError(MFH_ERR_HIP, "copy to host failed");
  } catch (const std::exception &e) {
    return SetError(MFH_ERR_HIP, e.what());
  }
  return MFH_OK;
}

int mfh_debug_quantize_rows_e4m3(int rows, int cols, const uint16_t *x, const uint16_t *x_lo,
                                 uint8_t *codes, float *scales) {
  if (rows <= 0 || cols <= 0 || !x || !codes || !scales)
    return SetError(MFH_ERR_INVALID, "mfh_debug_quantize_rows_e4m3: bad arguments");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return SetError(MFH_ERR_NO_DEVICE, "no HIP device available");
  const size_t n = static_cast<size_t>(rows) * cols;
  try {
    DebugBuffers buf;
    const std::uint16_t *dx = buf.Put(x, n);
    const std::uint16_t *dl = buf.Put(x_lo, n);
    std::uint8_t *dq = buf.Put<std::uint8_t>(nullptr, n, false);
    float *ds = buf.Put<float>(nullptr, rows, false);
    std::string err;
    if (mfh::LaunchQuantizeRowsE4m3(dx, dl, cols, rows, cols, dq, cols, ds, nullptr, &err) !=
        hipSuccess)
      return SetError(MFH_ERR_INVALID, err);
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(codes, dq, n, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(scales, ds, static_cast<size_t>(rows) * 4, hipMemcpyDeviceToHost) != hipSuccess)
      return SetError(MFH_ERR_HIP, "row quantisation failed");
  } catch (const std::exception &e) {
    return SetError(MFH_ERR_HIP, e.what());
  }
  return MFH_OK;
}

int mfh_debug_skinny_gemm(int M, int N, int K, const uint16_t *A, const uint16_t *A_lo,
                          const float *x, int rows_per_src, float eps, const float *gamma,
                          const float *beta, int ln_split, const uint16_t *W, const float *bias,
                          int act, int out_mode, const float *resid32, const uint16_t *resid_hi,
                          const uint16_t *resid_lo, float alpha, void *out, uint16_t *out_lo,
                          float *stats, int *parts, uint16_t *y_hi, uint16_t *y_lo,
                          float *y32) {
  if (M <= 0 || N <= 0 || K <= 0 || (!A && !x) || !W || !out || out_mode < 0 || out_mode > 2 ||
      rows_per_src < 1)
    return SetError(MFH_ERR_INVALID, "mfh_debug_skinny_gemm: bad arguments");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return SetError(MFH_ERR_NO_DEVICE, "no HIP device available");
  const size_t nw = static_cast<size_t>(N) * K, nc = static_cast<size_t>(M) * N;
  const int src_rows = (M + rows_per_src - 1) / rows_per_src;
  const int width = rows_per_src * K;
  try {
    DebugBuffers buf;
    mfh::SkinnyParams p;
    std::vector<float> st;
    if (x) {
      // One statistics part per source row, summed on the host.
      st.resize(2 * static_cast<size_t>(src_rows));
      for (int r = 0; r < src_rows; ++r) {
        float s = 0.f, ss = 0.f;
        for (int c = 0; c < width; ++c) {
          const float v = x[static_cast<size_t>(r) * width + c];
          s += v;
          ss += v * v;
        }
        st[2 * r] = s;
        st[2 * r + 1] = ss;
      }
      p.x = buf.Put(x, static_cast<size_t>(src_rows) * width);
      p.ldx = width;
      p.rows_per_src = rows_per_src;
      p.ln_stats = buf.Put(st.data(), st.size());
      p.ln_parts = 1;
      p.ln_rows = src_rows;
      p.ln_width = width;
      p.ln_eps = eps;
      p.gamma = buf.Put(gamma, width);
      p.beta = buf.Put(beta, width);
      p.ln_split = ln_split != 0;
      p.y16 = y_hi ? buf.Put<std::uint16_t>(nullptr, static_cast<size_t>(M) * K, false) : nullptr;
      p.y16_lo = y_lo ? buf.Put<std::uint16_t>(nullptr, static_cast<size_t>(M) * K, false)
                      : nullptr;
      p.y32 = y32 ? buf.Put<float>(nullptr, static_cast<size_t>(M) * K, false) : nullptr;
      p.ldy = K;
    } else {
      p.a16 = buf.Put(A, static_cast<size_t>(M) * K);
      p.a16_lo = buf.Put(A_lo, static_cast<size_t>(M) * K);
      p.lda = K;
    }
    p.W = buf.Put(W, nw);
    p.ldw = K;
    p.M = M;
    p.N = N;
    p.K = K;
    p.bias = buf.Put(bias, N);
    p.act = ActFromProto(act, mfh::ACT_RELU);
    if (act == MFH_ACTIVATION_NONE || act == MFH_ACTIVATION_DEFAULT)
      p.act = mfh::ACT_NONE;
    p.out_mode = out_mode;
    const size_t out_bytes = out_mode == mfh::SKINNY_OUT_BF16 ? 2 : 4;
    p.C = buf.Put<unsigned char>(nullptr, nc * out_bytes, false);
    p.C_lo = out_lo ? buf.Put<std::uint16_t>(nullptr, nc, false) : nullptr;
    p.ldc = N;
    if (out_mode == mfh::SKINNY_OUT_RESID) {
      p.resid = buf.Put(resid32, nc);
      p.resid16 = buf.Put(resid_hi, nc);
      p.resid16_lo = buf.Put(resid_lo, nc);
      p.ldr = N;
      p.alpha = alpha;
    }
    const int np = mfh::SkinnyGemmParts(N);
    if (parts)
      *parts = np;
    if (stats && out_mode != mfh::SKINNY_OUT_BF16)
      p.stats_out = buf.Put<float>(nullptr, 2 * static_cast<size_t>(np) * M, false);
    std::string err;
    if (mfh::LaunchSkinnyGemm(p, nullptr, &err) != hipSuccess)
      return SetError(MFH_ERR_INVALID, err);
    const size_t ny = static_cast<size_t>(M) * K;
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(out, p.C, nc * out_bytes, hipMemcpyDeviceToHost) != hipSuccess ||
        (p.C_lo && hipMemcpy(out_lo, p.C_lo, nc * 2, hipMemcpyDeviceToHost) != hipSuccess) ||
        (p.stats_out && hipMemcpy(stats, p.stats_out, 8 * static_cast<size_t>(np) * M,
                                  hipMemcpyDeviceToHost) != hipSuccess) ||
        (p.y16 && hipMemcpy(y_hi, p.y16, ny * 2, hipMemcpyDeviceToHost) != hipSuccess) ||
        (p.y16_lo && hipMemcpy(y_lo, p.y16_lo, ny * 2, hipMemcpyDeviceToHost) != hipSuccess) ||
        (p.y32 && hipMemcpy(y32, p.y32, ny * 4, hipMemcpyDeviceToHost) != hipSuccess))
      return SetError(MFH_ERR_HIP, "skinny gemm execution failed");
  } catch (const std::exception &e) {
    return SetError(MFH_ERR_HIP, e.what());
  }
  return MFH_OK;
}

int mfh_debug_panel_gemm(int M, int N, int K, const uint16_t *A, const uint16_t *A_lo,
                         const uint16_t *W, const uint8_t *W8, const float *wscale,
                         const float *bias, int act, int layernorm, const float *resid32,
                         const uint16_t *resid_hi, const uint16_t *resid_lo, float alpha,
                         float eps, const float *gamma, const float *beta, uint16_t *out_hi,
                         uint16_t *out_lo, float *out_f32) {
  if (M <= 0 || N <= 0 || K <= 0 || !A || !out_hi)
    return SetError(MFH_ERR_INVALID, "mfh_debug_panel_gemm: bad arguments");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
    return SetError(MFH_ERR_NO_DEVICE, "no HIP device available");
  const size_t na = static_cast<size_t>(M) * K, nw = static_cast<size_t>(N) * K,
               nc = static_cast<size_t>(M) * N;
  try {
    DebugBuffers buf;
    mfh::PanelGemmParams p;
    p.A = buf.Put(A, na);
    p.A_lo = buf.Put(A_lo, na);
    p.lda = K;
    p.W = buf.Put(W, nw);
    p.W8 = buf.Put(W8, nw);
    p.wscale = buf.Put(wscale, N);
    p.ldw = K;
    p.M = M;
    p.N = N;
    p.K = K;
    p.bias = buf.Put(bias, N);
    p.act = ActFromProto(act, mfh::ACT_RELU);
    if (act == MFH_ACTIVATION_NONE || act == MFH_ACTIVATION_DEFAULT)
      p.act = mfh::ACT_NONE;
    p.out_mode = layernorm ? mfh::PANEL_OUT_LN : mfh::PANEL_OUT_BF16;
    p.C = buf.Put<std::uint16_t>(nullptr, nc, false);
    p.C_lo = out_lo ? buf.Put<std::uint16_t>(nullptr, nc, false) : nullptr;
    p.ldc = N;
    if (layernorm) {
      p.resid = buf.Put(resid32, nc);
      p.resid16 = buf.Put(resid_hi, nc);
      p.resid16_lo = buf.Put(resid_lo, nc);
      p.alpha = alpha;
      p.eps = eps;
      p.gamma = buf.Put(gamma, N);
      p.beta = buf.Put(beta, N);
      p.y_f32 = out_f32 ? buf.Put<float>(nullptr, nc, false) : nullptr;
    }
    std::string err;
    if (mfh::LaunchPanelGemm(p, nullptr, &err) != hipSuccess)
      return SetError(MFH_ERR_INVALID, err);
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(out_hi, p.C, nc * 2, hipMemcpyDeviceToHost) != hipSuccess ||
        (out_lo && hipMemcpy(out_lo, p.C_lo, nc * 2, hipMemcpyDeviceToHost) != hipSuccess) ||
        (p.y_f32 && hipMemcpy(out_f32, p.y_f32, nc * 4, hipMemcpyDeviceToHost) != hipSuccess))
      return SetError(MFH_ERR_HIP, "panel gemm execution failed");
  } catch (const std::exception &e) {
    return SetError(MFH_ERR_HIP, e.what());
  }
  return MFH_OK;
}
