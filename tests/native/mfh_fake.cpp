// CPU fake of the mfhip.h C ABI -- TEST INFRASTRUCTURE ONLY, never shipped.
//
// Lets the C++ HipNetwork adapter run without a GPU, under ThreadSanitizer:
// each position's outputs are a deterministic function of its 112x64 planes
// (an FNV-1a hash of their bits seeding a linear congruential stream), so
// results from concurrent callers can be compared with serial ones bit for
// bit; and the next calls can be made to fail or to return non-finite
// logits, which drives the adapter's retry-then-throw path (reference
// src/nn/cuda/cuda_network.cpp:199-231, 444-458).  Like the real library, an
// eval call holds the net's mutex only while it writes the caller's output
// buffers.
#include "mfhip.h"

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

struct mfh_net {
  std::mutex mu;
  int max_batch = 0;
  int vout = 3;
  bool mlh = false;
};

struct mfh_weights {};

namespace {

thread_local std::string g_err;
std::atomic<int> g_fail_next{0};
std::atomic<int> g_nan_next{0};
std::atomic<int> g_eval_calls{0};

int Err(int code, const char *msg) {
  g_err = msg;
  return code;
}

// Takes one unit from an injection counter; true while it was positive.
bool Take(std::atomic<int> &counter) {
  int v = counter.load();
  while (v > 0)
    if (counter.compare_exchange_weak(v, v - 1))
      return true;
  return false;
}

constexpr int kPlanes = 112, kSquares = 64, kPolicy = 1858;

void Position(const float *planes, float *policy, float *value, int vout, float *moves_left) {
  std::uint32_t h = 2166136261u;
  for (int i = 0; i < kPlanes * kSquares; ++i) {
    std::uint32_t u;
    std::memcpy(&u, planes + i, 4);
    h = (h ^ u) * 16777619u;
  }
  auto next = [&h]() {
    h = h * 1664525u + 1013904223u;
    return static_cast<float>(h >> 8) / 16777216.0f;
  };
  for (int i = 0; i < kPolicy; ++i)
    policy[i] = next() * 8.0f - 4.0f;
  if (vout == 3) {
    const float a = next() + 0.1f, b = next() + 0.1f, c = next() + 0.1f;
    const float s = a + b + c;
    value[0] = a / s;
    value[1] = b / s;
    value[2] = c / s;
  } else {
    value[0] = next() * 2.0f - 1.0f;
  }
  if (moves_left)
    *moves_left = next() * 100.0f;
}

void Unpack(const std::uint64_t *masks, const float *values, float *planes) {
  for (int p = 0; p < kPlanes; ++p)
    for (int sq = 0; sq < kSquares; ++sq)
      planes[p * kSquares + sq] = (masks[p] >> sq) & 1u ? values[p] : 0.0f;
}

}  // namespace

extern "C" {

// Injection controls (fake only): the next n eval calls fail with
// MFH_ERR_HIP, or write a NaN logit; the number of eval calls so far.
void mfh_fake_fail_next(int n) { g_fail_next.store(n); }
void mfh_fake_nan_next(int n) { g_nan_next.store(n); }
int mfh_fake_eval_calls(void) { return g_eval_calls.load(); }

const char *mfh_last_error(void) { return g_err.c_str(); }

int mfh_net_create(const mfh_net_desc *desc, const mfh_tensor *, int, mfh_net **out) {
  if (!desc || !out)
    return Err(MFH_ERR_INVALID, "mfh_net_create: null argument");
  if (desc->max_batch < 1)
    return Err(MFH_ERR_INVALID, "max_batch must be >= 1");
  if (desc->value != MFH_VALUE_WDL && desc->value != MFH_VALUE_CLASSICAL)
    return Err(MFH_ERR_UNSUPPORTED, "value head");
  auto *net = new mfh_net;
  net->max_batch = desc->max_batch;
  net->vout = desc->value == MFH_VALUE_WDL ? 3 : 1;
  net->mlh = desc->moves_left == MFH_MOVES_LEFT_V1;
  *out = net;
  return MFH_OK;
}

void mfh_net_destroy(mfh_net *net) { delete net; }

int mfh_net_set_graphs(mfh_net *net, int) {
  return net ? MFH_OK : Err(MFH_ERR_INVALID, "null net");
}

int mfh_net_eval_planes(mfh_net *net, int batch, const float *planes, float *policy,
                        float *wdl, float *moves_left) {
  if (!net || batch < 1 || batch > net->max_batch || !planes || !policy || !wdl)
    return Err(MFH_ERR_INVALID, "mfh_net_eval_planes: bad arguments");
  std::lock_guard<std::mutex> lock(net->mu);
  g_eval_calls.fetch_add(1);
  if (Take(g_fail_next))
    return Err(MFH_ERR_HIP, "injected device failure");
  for (int b = 0; b < batch; ++b)
    Position(planes + static_cast<std::size_t>(b) * kPlanes * kSquares,
             policy + static_cast<std::size_t>(b) * kPolicy, wdl + b * net->vout, net->vout,
             moves_left ? moves_left + b : nullptr);
  if (Take(g_nan_next))
    policy[static_cast<std::size_t>(batch - 1) * kPolicy + 7] = std::nanf("");
  return MFH_OK;
}

int mfh_pack_planes(int batch, const float *planes, uint64_t *masks, float *values) {
  if (batch < 0 || (batch > 0 && (!planes || !masks || !values)))
    return Err(MFH_ERR_INVALID, "mfh_pack_planes: bad arguments");
  for (int i = 0; i < batch * kPlanes; ++i) {
    const float *plane = planes + static_cast<std::size_t>(i) * kSquares;
    std::uint64_t mask = 0;
    float value = 0.0f;
    for (int sq = 0; sq < kSquares; ++sq)
      if (plane[sq] != 0.0f) {
        if (!mask)
          value = plane[sq];
        mask |= 1ull << sq;
      }
    masks[i] = mask;
    values[i] = value;
  }
  return MFH_OK;
}

int mfh_net_eval_priors(mfh_net *net, int batch, const uint64_t *masks, const float *values,
                        const int32_t *offsets, const int16_t *indices, float softmax_temp,
                        float *priors, float *wdl, float *moves_left) {
  if (!net || batch < 1 || batch > net->max_batch || !masks || !values || !offsets || !wdl)
    return Err(MFH_ERR_INVALID, "mfh_net_eval_priors: bad arguments");
  std::lock_guard<std::mutex> lock(net->mu);
  g_eval_calls.fetch_add(1);
  if (Take(g_fail_next))
    return Err(MFH_ERR_HIP, "injected device failure");
  std::vector<float> planes(kPlanes * kSquares), policy(kPolicy);
  for (int b = 0; b < batch; ++b) {
    Unpack(masks + b * kPlanes, values + b * kPlanes, planes.data());
    Position(planes.data(), policy.data(), wdl + b * net->vout, net->vout,
             moves_left ? moves_left + b : nullptr);
    float mx = -INFINITY, sum = 0.0f;
    for (int i = offsets[b]; i < offsets[b + 1]; ++i)
      mx = std::fmax(mx, policy[indices[i]]);
    for (int i = offsets[b]; i < offsets[b + 1]; ++i)
      sum += priors[i] = std::exp((policy[indices[i]] - mx) / softmax_temp);
    for (int i = offsets[b]; i < offsets[b + 1]; ++i)
      priors[i] /= sum;
  }
  return MFH_OK;
}

int mfh_net_info(const mfh_net *net, char *buf, size_t len) {
  if (!net || !buf || !len)
    return Err(MFH_ERR_INVALID, "mfh_net_info: null argument");
  std::snprintf(buf, len, "CPU fake of the HIP backend, max_batch %d", net->max_batch);
  return MFH_OK;
}

int mfh_net_capabilities(const mfh_net *net, mfh_capabilities *out) {
  if (!net || !out)
    return Err(MFH_ERR_INVALID, "mfh_net_capabilities: null argument");
  std::memset(out, 0, sizeof(*out));
  out->has_wdl = net->vout == 3;
  out->has_moves_left = net->mlh;
  out->max_batch_size = net->max_batch;
  std::snprintf(out->device_name, sizeof(out->device_name), "cpu fake");
  std::snprintf(out->arch_name, sizeof(out->arch_name), "none");
  return MFH_OK;
}

int mfh_weights_load(const char *, mfh_weights **out) {
  if (out)
    *out = nullptr;
  return Err(MFH_ERR_INVALID, "the CPU fake reads no network files");
}
int mfh_weights_describe(const mfh_weights *, mfh_weights_format *, mfh_net_desc *) {
  return Err(MFH_ERR_INVALID, "the CPU fake reads no network files");
}
int mfh_weights_tensors(const mfh_weights *, const mfh_tensor **, int *) {
  return Err(MFH_ERR_INVALID, "the CPU fake reads no network files");
}
void mfh_weights_free(mfh_weights *) {}

}  // extern "C"
