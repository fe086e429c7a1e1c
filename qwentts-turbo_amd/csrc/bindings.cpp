// PyTorch-ROCm extension: the reference's pybind classes over the C ABI of libqwentts_amd.
//
// MegakernelTTSDecoder           -- /root/reference/qwentts_turbo/megakernel_backbone.py:109-332
// MegakernelCodePredictorDecoder -- /root/reference/qwentts_turbo/megakernel_code_predictor.py:86-242
//
// Same constructor arguments, method names and return conventions as the reference (outputs
// are fresh tensors; KV getters alias the internal caches). Differences: shapes, dtypes,
// devices and positions are validated (the reference checks nothing), launch errors raise,
// and extra methods expose the fused head / token-selection / frame entry points.
#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <hip/hip_runtime_api.h>
#include <cmath>
#include <vector>
#include "qwentts_amd.h"

namespace {

constexpr int kHidden = 1024, kKVHeads = 8, kHeadDim = 128, kInter = 3072, kQ = 2048;
constexpr int kMaxStreams = 8;   // streams of one frames_streams() launch (one per XCD)

hipStream_t cur_stream() { return c10::hip::getCurrentHIPStreamMasqueradingAsCUDA().stream(); }

void hip_check(hipError_t e, const char* what) {
  TORCH_CHECK(e == hipSuccess, what, " failed: ", hipGetErrorString(e));
}

void check_bf16(const torch::Tensor& t, std::vector<int64_t> shape, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.scalar_type() == torch::kBFloat16, name, " must be bfloat16, got ", t.scalar_type());
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.sizes().vec() == shape, name, " has shape ", t.sizes(), ", expected ", c10::IntArrayRef(shape));
}

// Layer weights in the reference's struct order (11 per layer).
std::vector<TTSLayerWeights> pack_layers(const std::vector<torch::Tensor>& flat, int num_layers) {
  TORCH_CHECK((int)flat.size() == num_layers * 11, "expected ", num_layers * 11, " layer weights, got ", flat.size());
  const std::vector<std::vector<int64_t>> shapes = {
      {kHidden}, {kQ, kHidden}, {kKVHeads * kHeadDim, kHidden}, {kKVHeads * kHeadDim, kHidden},
      {kHeadDim}, {kHeadDim}, {kHidden, kQ}, {kHidden}, {kInter, kHidden}, {kInter, kHidden}, {kHidden, kInter}};
  std::vector<TTSLayerWeights> out(num_layers);
  for (int i = 0; i < num_layers; ++i) {
    const void** p = reinterpret_cast<const void**>(&out[i]);
    for (int j = 0; j < 11; ++j) {
      const auto& t = flat[i * 11 + j];
      check_bf16(t, shapes[j], "layer weight");
      TORCH_CHECK((reinterpret_cast<uintptr_t>(t.data_ptr()) & 15u) == 0, "layer weights must be 16-byte aligned");
      p[j] = t.data_ptr();
    }
  }
  return out;
}

torch::Tensor upload_struct(const void* data, size_t bytes, const torch::Device& dev) {
  auto t = torch::empty({(int64_t)bytes}, torch::dtype(torch::kUInt8).device(dev));
  hip_check(hipMemcpy(t.data_ptr(), data, bytes, hipMemcpyHostToDevice), "hipMemcpy");
  return t;
}

torch::Tensor make_workspace(const torch::Device& dev) {
  auto ws = torch::zeros({(int64_t)qtts_workspace_bytes()}, torch::dtype(torch::kUInt8).device(dev));
  hip_check(qtts_workspace_init(ws.data_ptr(), dev.index()), "qtts_workspace_init (needs an MI355X: gfx950, 256 CUs)");
  return ws;
}

torch::Tensor as_bf16_vec(torch::Tensor e, const torch::Device& dev) {
  if (e.dim() == 2) e = e.squeeze(0);
  TORCH_CHECK(e.dim() == 1 && e.size(0) == kHidden, "input embedding must be [1024] or [1, 1024], got ", e.sizes());
  TORCH_CHECK(e.device() == dev, "input embedding must be on ", dev);
  return e.to(torch::kBFloat16).contiguous();
}

QttsSampling sampling(bool do_sample, double temperature, int64_t top_k, double top_p, int64_t seed) {
  TORCH_CHECK(!do_sample || temperature > 0.0, "temperature must be > 0");
  QttsSampling s;
  s.do_sample = do_sample ? 1 : 0;
  s.temperature = (float)temperature;
  s.top_k = (int)top_k;
  s.top_p = (float)top_p;
  s.seed = (unsigned long long)seed;
  return s;
}

// the weight-shared launches' workspace, allocated on first use (its first launch zero-fills it)
void ensure_shared_ws(torch::Tensor& ws, const torch::Device& dev) {
  if (ws.defined()) return;
  ws = torch::empty({(int64_t)qtts_shared_workspace_bytes()}, torch::dtype(torch::kUInt8).device(dev));
  hip_check(qtts_workspace_init(ws.data_ptr(), dev.index()), "qtts_workspace_init");
}
void check_shared_error(const torch::Tensor& ws) {
  if (!ws.defined()) return;
  unsigned int code = 0;
  hip_check(qtts_shared_workspace_check(ws.data_ptr(), &code, cur_stream()), "qtts_shared_workspace_check");
  TORCH_CHECK(code == 0, "weight-shared decode kernel reported a device-side wait timeout (error word ", code, ")");
}

void check_device_error(const torch::Tensor& ws) {
  unsigned int code = 0;
  hip_check(qtts_workspace_check(ws.data_ptr(), &code, cur_stream()), "qtts_workspace_check");
  TORCH_CHECK(code == 0, "decode kernel reported a device-side wait timeout (error word ", code, ")");
}

// ---------------------------------------------------------------------------------------
class MegakernelTTSDecoder {
 public:
  MegakernelTTSDecoder(torch::Tensor embed_weight, std::vector<torch::Tensor> layer_weights_flat,
                       torch::Tensor final_norm_weight, torch::Tensor codec_head_weight, torch::Tensor cos_table,
                       torch::Tensor sin_table, int64_t num_layers, int64_t max_seq_len)
      : num_layers_((int)num_layers), max_seq_len_((int)max_seq_len), dev_(embed_weight.device()) {
    TORCH_CHECK(num_layers >= 1, "num_layers must be >= 1");
    TORCH_CHECK(max_seq_len >= 1, "max_seq_len must be >= 1");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev_);
    TORCH_CHECK(embed_weight.dim() == 2 && embed_weight.size(1) == kHidden, "embed_weight must be [vocab, 1024]");
    check_bf16(embed_weight, {embed_weight.size(0), kHidden}, "embed_weight");
    check_bf16(codec_head_weight, {codec_head_weight.size(0), kHidden}, "codec_head_weight");
    check_bf16(final_norm_weight, {kHidden}, "final_norm_weight");
    TORCH_CHECK(cos_table.size(0) >= max_seq_len && sin_table.size(0) >= max_seq_len, "RoPE tables shorter than max_seq_len");
    check_bf16(cos_table, {cos_table.size(0), kHeadDim}, "cos_table");
    check_bf16(sin_table, {sin_table.size(0), kHeadDim}, "sin_table");
    embed_weight_ = embed_weight;
    final_norm_weight_ = final_norm_weight;
    codec_head_weight_ = codec_head_weight;
    cos_table_ = cos_table;
    sin_table_ = sin_table;
    layer_weights_tensors_ = layer_weights_flat;
    auto host = pack_layers(layer_weights_flat, num_layers_);
    d_layer_weights_ = upload_struct(host.data(), host.size() * sizeof(TTSLayerWeights), dev_);
    auto bf = torch::dtype(torch::kBFloat16).device(dev_);
    auto f32 = torch::dtype(torch::kFloat32).device(dev_);
    k_cache_ = torch::zeros({num_layers, kKVHeads, max_seq_len, kHeadDim}, bf);
    v_cache_ = torch::zeros({num_layers, kKVHeads, max_seq_len, kHeadDim}, bf);
    hidden_buffer_ = torch::zeros({kHidden}, bf);
    g_normalized_ = torch::zeros({kHidden}, f32);
    logits_ = torch::zeros({codec_head_weight.size(0)}, f32);
    token_ = torch::zeros({1}, torch::dtype(torch::kInt32).device(dev_));
    ws_ = make_workspace(dev_);
    position_ = 0;
  }
  ~MegakernelTTSDecoder() {
    (void)qtts_workspace_release(ws_.data_ptr(), 1);
    if (ws_streams_.defined()) (void)qtts_workspace_release(ws_streams_.data_ptr(), kMaxStreams);
    if (ws_shared_.defined()) (void)qtts_workspace_release(ws_shared_.data_ptr(), 1);
  }
  MegakernelTTSDecoder(const MegakernelTTSDecoder&) = delete;
  MegakernelTTSDecoder& operator=(const MegakernelTTSDecoder&) = delete;

  torch::Tensor decode_step(int64_t input_token_id) {
    TORCH_CHECK(input_token_id >= 0 && input_token_id < embed_weight_.size(0), "token id out of range");
    run(nullptr, (int)input_token_id, nullptr, false, nullptr, 0, 1.0, -1, false, sampling(false, 1.0, 0, 1.0, 0), 0);
    return g_normalized_.clone();
  }

  int64_t decode_step_with_argmax(int64_t input_token_id) {
    TORCH_CHECK(input_token_id >= 0 && input_token_id < embed_weight_.size(0), "token id out of range");
    run(nullptr, (int)input_token_id, nullptr, true, nullptr, 0, 1.0, -1, false, sampling(false, 1.0, 0, 1.0, 0), 0,
        /*no_mask=*/true);
    return token_.item<int>();
  }

  torch::Tensor decode_step_with_embedding(torch::Tensor input_embedding) {
    auto e = as_bf16_vec(input_embedding, dev_);
    run(e.data_ptr(), 0, nullptr, false, nullptr, 0, 1.0, -1, false, sampling(false, 1.0, 0, 1.0, 0), 0);
    return g_normalized_.clone();
  }

  // Extended: one step with 3D rotary positions (t, h, w); returns the final hidden.
  torch::Tensor decode_step_3d(torch::Tensor input_embedding, std::vector<int64_t> pos3) {
    TORCH_CHECK(pos3.size() == 3, "pos3 must be (t, h, w)");
    auto e = as_bf16_vec(input_embedding, dev_);
    int p3[3] = {(int)pos3[0], (int)pos3[1], (int)pos3[2]};
    run(e.data_ptr(), 0, p3, false, nullptr, 0, 1.0, -1, false, sampling(false, 1.0, 0, 1.0, 0), 0);
    return g_normalized_.clone();
  }

  // Extended: step + fused codec head + on-device selection. Writes the token to
  // out_token (int32 [1] device); keeps hidden / logits in the internal buffers.
  void decode_step_select(torch::Tensor input_embedding, torch::Tensor out_token, torch::Tensor history,
                          int64_t n_history, double repetition_penalty, int64_t eos_id, bool suppress_eos,
                          bool do_sample, double temperature, int64_t top_k, double top_p, int64_t seed,
                          int64_t frame_step, c10::optional<std::vector<int64_t>> pos3, c10::optional<torch::Tensor> skip_if) {
    auto e = as_bf16_vec(input_embedding, dev_);
    TORCH_CHECK(out_token.is_cuda() && out_token.scalar_type() == torch::kInt32 && out_token.numel() >= 1,
                "out_token must be an int32 GPU tensor");
    TORCH_CHECK(history.is_cuda() && history.scalar_type() == torch::kInt32 && history.numel() >= n_history,
                "history must be an int32 GPU tensor with >= n_history entries");
    int p3[3];
    int* p3p = nullptr;
    if (pos3.has_value()) {
      TORCH_CHECK(pos3->size() == 3, "pos3 must be (t, h, w)");
      for (int i = 0; i < 3; ++i) p3[i] = (int)(*pos3)[i];
      p3p = p3;
    }
    const int* skip = nullptr;
    if (skip_if.has_value()) {
      TORCH_CHECK(skip_if->is_cuda() && skip_if->scalar_type() == torch::kInt32, "skip_if must be an int32 GPU tensor");
      skip = skip_if->data_ptr<int>();
    }
    run(e.data_ptr(), 0, p3p, true, history.data_ptr<int>(), (int)n_history, repetition_penalty, (int)eos_id, suppress_eos,
        sampling(do_sample, temperature, top_k, top_p, seed), (int)frame_step, false, out_token.data_ptr<int>(), skip);
  }

  // Extended: prefill of the prompt embeddings [S, 1024] at positions position() .. position() + S - 1
  // in one call (qtts_backbone_prefill: the transformers bf16 forward on MFMA, K/V straight into
  // this decoder's cache). Returns the last token's final-norm hidden (f32 [1024] of bf16 values),
  // also left in hidden_state_buffer(). With out_token, the first group-0 token is selected from
  // the codec head (suppress mask, EOS removed when suppress_eos; generator.py:113-119). pos3:
  // optional int32 [3, S] rotary (t, h, w) rows. The position advances by S.
  torch::Tensor prefill(torch::Tensor embeds, c10::optional<torch::Tensor> out_token, int64_t eos_id, bool suppress_eos,
                        bool do_sample, double temperature, int64_t top_k, double top_p, int64_t seed,
                        c10::optional<torch::Tensor> pos3) {
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev_);
    if (embeds.dim() == 3) embeds = embeds.squeeze(0);
    TORCH_CHECK(embeds.dim() == 2 && embeds.size(1) == kHidden && embeds.size(0) >= 1, "embeds must be [S, 1024], got ",
                embeds.sizes());
    TORCH_CHECK(embeds.device() == dev_, "embeds must be on ", dev_);
    auto e = embeds.to(torch::kBFloat16).contiguous();
    const int S = (int)e.size(0);
    TORCH_CHECK(position_ + S <= max_seq_len_, "prefill of ", S, " tokens at position ", position_, " exceeds max_seq_len ",
                max_seq_len_);
    const int* p3 = nullptr;
    torch::Tensor p3t;
    if (pos3.has_value()) {
      p3t = pos3->to(dev_, torch::kInt32).contiguous();
      TORCH_CHECK(p3t.dim() == 2 && p3t.size(0) == 3 && p3t.size(1) == S, "pos3 must be [3, S]");
      p3 = p3t.data_ptr<int>();
    }
    int* tok = nullptr;
    if (out_token.has_value()) {
      TORCH_CHECK(out_token->is_cuda() && out_token->scalar_type() == torch::kInt32 && out_token->numel() >= 1,
                  "out_token must be an int32 GPU tensor");
      tok = out_token->data_ptr<int>();
    }
    const int vocab = (int)codec_head_weight_.size(0);
    const size_t need = qtts_prefill_workspace_bytes(S, tok ? vocab : 0);
    TORCH_CHECK(need > 0, "prefill workspace size query failed");
    if (!pf_ws_.defined() || (size_t)pf_ws_.numel() < need)
      pf_ws_ = torch::empty({(int64_t)need}, torch::dtype(torch::kUInt8).device(dev_));
    QttsSampling samp = sampling(do_sample, temperature, top_k, top_p, seed);
    hip_check(qtts_backbone_prefill(pf_ws_.data_ptr(), (size_t)pf_ws_.numel(),
                                    reinterpret_cast<const TTSLayerWeights*>(d_layer_weights_.data_ptr()), num_layers_,
                                    final_norm_weight_.data_ptr(), cos_table_.data_ptr(), sin_table_.data_ptr(),
                                    k_cache_.data_ptr(), v_cache_.data_ptr(), max_seq_len_, position_, S, p3, e.data_ptr(),
                                    g_normalized_.data_ptr<float>(), tok ? codec_head_weight_.data_ptr() : nullptr, vocab,
                                    tok ? logits_.data_ptr<float>() : nullptr, tok, 1, (int)eos_id, suppress_eos ? 1 : 0,
                                    &samp, 0, cur_stream()),
              "qtts_backbone_prefill");
    position_ += S;
    return g_normalized_.clone();
  }

  // Extended: decode_step_select for up to 8 independent decoders `decs` (sharing this decoder's
  // weights) in one launch, decoder s on XCD s, each at its own position with its own KV cache.
  // out_tokens[s] gets stream s's token and hidden_out[s] (f32 [n, 1024]) its final-norm hidden;
  // the residual and logits go to each decoder's own buffers. Stream s samples with key seed + s
  // and applies the repetition penalty over history[s][0 : n_history[s]]. Each position advances
  // by one. The launch uses this decoder's block of per-stream workspaces.
  void decode_steps_streams(std::vector<MegakernelTTSDecoder*> decs, torch::Tensor embeds, torch::Tensor out_tokens,
                            torch::Tensor hidden_out, c10::optional<torch::Tensor> history, std::vector<int64_t> n_history,
                            double repetition_penalty, int64_t eos_id, bool suppress_eos, bool do_sample,
                            double temperature, int64_t top_k, double top_p, int64_t seed, int64_t frame_step,
                            c10::optional<torch::Tensor> skip, bool shared) {
    const int64_t n = (int64_t)decs.size();
    TORCH_CHECK(n >= 1 && n <= kMaxStreams, "decode_steps_streams takes 1..", kMaxStreams, " decoders, got ", n);
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev_);
    check_bf16(embeds, {n, kHidden}, "embeds");
    TORCH_CHECK(embeds.device() == dev_, "embeds must be on ", dev_);
    TORCH_CHECK(out_tokens.is_cuda() && out_tokens.scalar_type() == torch::kInt32 && out_tokens.is_contiguous() &&
                    out_tokens.numel() >= n, "out_tokens must be a contiguous int32 GPU tensor with >= ", n, " entries");
    TORCH_CHECK(hidden_out.is_cuda() && hidden_out.scalar_type() == torch::kFloat32 && hidden_out.is_contiguous() &&
                    hidden_out.sizes() == torch::IntArrayRef({n, kHidden}), "hidden_out must be a contiguous f32 [", n, ", 1024] GPU tensor");
    TORCH_CHECK(n_history.empty() || (int64_t)n_history.size() == n, "n_history needs one entry per decoder");
    int64_t hist_stride = 0;
    if (history.has_value()) {
      TORCH_CHECK(history->is_cuda() && history->scalar_type() == torch::kInt32 && history->is_contiguous() &&
                      history->dim() == 2 && history->size(0) >= n, "history must be a contiguous int32 [n, H] GPU tensor");
      hist_stride = history->size(1);
    }
    if (skip.has_value())
      TORCH_CHECK(skip->is_cuda() && skip->scalar_type() == torch::kInt32 && skip->is_contiguous() && skip->numel() >= n,
                  "skip must be a contiguous int32 GPU tensor with >= ", n, " entries");
    std::vector<QttsBackboneStream> io(n);
    for (int64_t st = 0; st < n; ++st) {
      MegakernelTTSDecoder* d = decs[st];
      TORCH_CHECK(d != nullptr, "decoder ", st, " is None");
      TORCH_CHECK(d->dev_ == dev_ && d->num_layers_ == num_layers_ && d->max_seq_len_ == max_seq_len_ &&
                      d->layer_weights_tensors_.size() == layer_weights_tensors_.size() &&
                      d->codec_head_weight_.data_ptr() == codec_head_weight_.data_ptr() &&
                      d->final_norm_weight_.data_ptr() == final_norm_weight_.data_ptr() &&
                      d->cos_table_.data_ptr() == cos_table_.data_ptr() && d->sin_table_.data_ptr() == sin_table_.data_ptr(),
                  "decoder ", st, " does not share this decoder's weights");
      for (size_t j = 0; j < layer_weights_tensors_.size(); ++j)
        TORCH_CHECK(d->layer_weights_tensors_[j].data_ptr() == layer_weights_tensors_[j].data_ptr(),
                    "decoder ", st, " does not share this decoder's layer weights");
      for (int64_t o = 0; o < st; ++o) TORCH_CHECK(decs[o] != d, "decoder ", st, " appears twice");
      TORCH_CHECK(d->position_ < max_seq_len_, "decoder ", st, ": position ", d->position_, " >= max_seq_len ",
                  max_seq_len_, " (KV cache full)");
      const int nh = n_history.empty() ? 0 : (int)n_history[st];
      TORCH_CHECK(nh >= 0 && nh <= hist_stride, "n_history[", st, "] = ", nh, " outside [0, ", hist_stride, "]");
      QttsBackboneStream& q = io[st];
      q.k_cache = d->k_cache_.data_ptr();
      q.v_cache = d->v_cache_.data_ptr();
      q.position = d->position_;
      q.pos3[0] = q.pos3[1] = q.pos3[2] = d->position_;
      q.input_embedding = static_cast<const uint16_t*>(embeds.data_ptr()) + st * kHidden;
      q.out_hidden = hidden_out.data_ptr<float>() + st * kHidden;
      q.out_residual = d->hidden_buffer_.data_ptr();
      q.out_logits = d->logits_.data_ptr<float>();
      q.out_token = out_tokens.data_ptr<int>() + st;
      q.history = nh > 0 ? history->data_ptr<int>() + st * hist_stride : nullptr;
      q.n_history = nh;
      q.seed = (unsigned long long)(seed + st);
      q.skip_if = skip.has_value() ? skip->data_ptr<int>() + st : nullptr;
    }
    QttsSampling samp = sampling(do_sample, temperature, top_k, top_p, seed);
    if (shared) {
      ensure_shared_ws(ws_shared_, dev_);
      hip_check(qtts_backbone_step_shared((int)n, ws_shared_.data_ptr(), reinterpret_cast<const TTSLayerWeights*>(d_layer_weights_.data_ptr()),
                                          num_layers_, final_norm_weight_.data_ptr(), cos_table_.data_ptr(), sin_table_.data_ptr(),
                                          max_seq_len_, io.data(), codec_head_weight_.data_ptr(), (int)codec_head_weight_.size(0),
                                          1, (float)repetition_penalty, (int)eos_id, suppress_eos ? 1 : 0, &samp, (int)frame_step,
                                          cur_stream()),
                "qtts_backbone_step_shared");
      for (auto* d : decs) d->position_++;
      return;
    }
    if (!ws_streams_.defined()) {
      ws_streams_ = torch::zeros({(int64_t)(kMaxStreams * qtts_workspace_bytes())}, torch::dtype(torch::kUInt8).device(dev_));
      hip_check(qtts_workspace_init(ws_streams_.data_ptr(), dev_.index()), "qtts_workspace_init");
    }
    hip_check(qtts_backbone_step_streams((int)n, ws_streams_.data_ptr(), reinterpret_cast<const TTSLayerWeights*>(d_layer_weights_.data_ptr()),
                                         num_layers_, final_norm_weight_.data_ptr(), cos_table_.data_ptr(), sin_table_.data_ptr(),
                                         max_seq_len_, io.data(), codec_head_weight_.data_ptr(), (int)codec_head_weight_.size(0),
                                         1, (float)repetition_penalty, (int)eos_id, suppress_eos ? 1 : 0, &samp, (int)frame_step,
                                         cur_stream()),
              "qtts_backbone_step_streams");
    for (auto* d : decs) d->position_++;
  }
  // the wait-timeout error words of the decode_steps_streams() workspaces
  void check_error_streams() const {
    check_shared_error(ws_shared_);
    if (!ws_streams_.defined()) return;
    for (int st = 0; st < kMaxStreams; ++st) {
      unsigned int code = 0;
      hip_check(qtts_workspace_check(static_cast<uint8_t*>(ws_streams_.data_ptr()) + st * qtts_workspace_bytes(), &code, cur_stream()),
                "qtts_workspace_check");
      TORCH_CHECK(code == 0, "decode kernel reported a device-side wait timeout in stream ", st, " (error word ", code, ")");
    }
  }

  void reset() {
    position_ = 0;
    k_cache_.zero_();
    v_cache_.zero_();
  }
  int64_t position() const { return position_; }
  void set_position(int64_t pos) {
    TORCH_CHECK(pos >= 0 && pos <= max_seq_len_, "position ", pos, " outside [0, ", max_seq_len_, "]");
    position_ = (int)pos;
  }
  torch::Tensor get_hidden_states() const { return g_normalized_.clone(); }
  torch::Tensor get_k_cache() const { return k_cache_; }
  torch::Tensor get_v_cache() const { return v_cache_; }
  torch::Tensor hidden_state_buffer() const { return g_normalized_; }
  torch::Tensor residual_buffer() const { return hidden_buffer_; }
  torch::Tensor logits_buffer() const { return logits_; }
  void check_error() const { check_device_error(ws_); }
  // test hook: pre-sets the workspace's error word (after at least one launch), so that every
  // wait of the next launch gives up at its first check
  void debug_set_error(int64_t code) {
    hip_check(qtts_debug_set_error(ws_.data_ptr(), (unsigned int)code, cur_stream()), "qtts_debug_set_error");
  }

  void set_kv_cache(torch::Tensor k_cache, torch::Tensor v_cache) {
    TORCH_CHECK(k_cache.dim() == 4 && k_cache.sizes() == v_cache.sizes(), "k/v must be [layers, 8, seq, 128]");
    TORCH_CHECK(k_cache.size(0) == num_layers_ && k_cache.size(1) == kKVHeads && k_cache.size(3) == kHeadDim,
                "k/v must be [", num_layers_, ", 8, seq, 128], got ", k_cache.sizes());
    TORCH_CHECK(k_cache.size(2) <= max_seq_len_, "k/v longer than max_seq_len");
    using namespace torch::indexing;
    k_cache_.index_put_({Slice(), Slice(), Slice(0, k_cache.size(2)), Slice()}, k_cache.to(dev_, torch::kBFloat16));
    v_cache_.index_put_({Slice(), Slice(), Slice(0, v_cache.size(2)), Slice()}, v_cache.to(dev_, torch::kBFloat16));
  }

 private:
  void run(const void* emb, int token, const int* pos3, bool with_head, const int* history, int n_history,
           double rep_penalty, int eos_id, bool suppress_eos, QttsSampling samp, int frame_step, bool no_mask = false,
           int* out_token = nullptr, const int* skip = nullptr) {
    TORCH_CHECK(position_ < max_seq_len_, "position ", position_, " >= max_seq_len ", max_seq_len_, " (KV cache full)");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev_);
    const int vocab = (int)codec_head_weight_.size(0);
    int* tok = out_token ? out_token : token_.data_ptr<int>();
    hipError_t e = qtts_backbone_step(
        ws_.data_ptr(), reinterpret_cast<const TTSLayerWeights*>(d_layer_weights_.data_ptr()), num_layers_,
        final_norm_weight_.data_ptr(), cos_table_.data_ptr(), sin_table_.data_ptr(), k_cache_.data_ptr(),
        v_cache_.data_ptr(), max_seq_len_, position_, pos3, emb, emb ? nullptr : embed_weight_.data_ptr(), token,
        g_normalized_.data_ptr<float>(), hidden_buffer_.data_ptr(), with_head ? codec_head_weight_.data_ptr() : nullptr,
        vocab, with_head ? logits_.data_ptr<float>() : nullptr, with_head ? tok : nullptr, no_mask ? 0 : 1, history,
        n_history, (float)rep_penalty, eos_id, suppress_eos ? 1 : 0, &samp, frame_step, skip,
        cur_stream());
    hip_check(e, "qtts_backbone_step");
    position_++;
  }

  int num_layers_, max_seq_len_, position_;
  torch::Device dev_;
  torch::Tensor embed_weight_, final_norm_weight_, codec_head_weight_, cos_table_, sin_table_, d_layer_weights_;
  std::vector<torch::Tensor> layer_weights_tensors_;
  torch::Tensor k_cache_, v_cache_, hidden_buffer_, g_normalized_, logits_, token_, ws_;
  torch::Tensor ws_streams_;   // decode_steps_streams(): per-stream workspaces
  torch::Tensor ws_shared_;    // decode_steps_streams(shared=True): the weight-shared launches' workspace
  torch::Tensor pf_ws_;        // prefill(): activations and split-K partials (grown on demand)
};

// ---------------------------------------------------------------------------------------
class MegakernelCodePredictorDecoder {
 public:
  MegakernelCodePredictorDecoder(std::vector<torch::Tensor> layer_weights_flat, torch::Tensor final_norm_weight,
                                 torch::Tensor cos_table, torch::Tensor sin_table, int64_t num_layers,
                                 int64_t max_seq_len)
      : num_layers_((int)num_layers), max_seq_len_((int)max_seq_len), dev_(final_norm_weight.device()) {
    TORCH_CHECK(num_layers >= 1 && max_seq_len >= 1, "num_layers and max_seq_len must be >= 1");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev_);
    check_bf16(final_norm_weight, {kHidden}, "final_norm_weight");
    TORCH_CHECK(cos_table.size(0) >= max_seq_len && sin_table.size(0) >= max_seq_len, "RoPE tables shorter than max_seq_len");
    check_bf16(cos_table, {cos_table.size(0), kHeadDim}, "cos_table");
    check_bf16(sin_table, {sin_table.size(0), kHeadDim}, "sin_table");
    final_norm_weight_ = final_norm_weight;
    cos_table_ = cos_table;
    sin_table_ = sin_table;
    layer_weights_tensors_ = layer_weights_flat;
    auto host = pack_layers(layer_weights_flat, num_layers_);
    d_layer_weights_ = upload_struct(host.data(), host.size() * sizeof(TTSLayerWeights), dev_);
    auto f32 = torch::dtype(torch::kFloat32).device(dev_);
    k_cache_ = torch::zeros({num_layers, kKVHeads, max_seq_len, kHeadDim}, f32);
    v_cache_ = torch::zeros({num_layers, kKVHeads, max_seq_len, kHeadDim}, f32);
    hidden_buffer_ = torch::zeros({kHidden}, f32);
    g_normalized_ = torch::zeros({kHidden}, f32);
    ws_ = make_workspace(dev_);
    position_ = 0;
  }
  ~MegakernelCodePredictorDecoder() {
    (void)qtts_workspace_release(ws_.data_ptr(), 1);
    if (ws_streams_.defined()) (void)qtts_workspace_release(ws_streams_.data_ptr(), kMaxStreams);
    if (ws_shared_.defined()) (void)qtts_workspace_release(ws_shared_.data_ptr(), 1);
  }
  MegakernelCodePredictorDecoder(const MegakernelCodePredictorDecoder&) = delete;
  MegakernelCodePredictorDecoder& operator=(const MegakernelCodePredictorDecoder&) = delete;

  torch::Tensor decode_step_with_embedding(torch::Tensor input_embedding) {
    TORCH_CHECK(position_ < max_seq_len_, "position ", position_, " >= max_seq_len ", max_seq_len_, " (KV cache full)");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev_);
    auto e = as_bf16_vec(input_embedding, dev_);
    hip_check(qtts_cp_step(ws_.data_ptr(), reinterpret_cast<const CPLayerWeights*>(d_layer_weights_.data_ptr()),
                           num_layers_, final_norm_weight_.data_ptr(), cos_table_.data_ptr(), sin_table_.data_ptr(),
                           k_cache_.data_ptr(), v_cache_.data_ptr(), max_seq_len_, position_, e.data_ptr(),
                           g_normalized_.data_ptr<float>(), hidden_buffer_.data_ptr<float>(),
                           cur_stream()),
              "qtts_cp_step");
    position_++;
    return g_normalized_.clone();
  }

  // Extended: bind the 15 lm-heads, the 15 codebook embedding tables and the backbone codec
  // embedding used by frame().
  void set_heads(std::vector<torch::Tensor> lm_heads, std::vector<torch::Tensor> embeddings, torch::Tensor bb_embedding) {
    TORCH_CHECK(!lm_heads.empty() && lm_heads.size() == embeddings.size(), "need as many lm-heads as embedding tables");
    const int64_t v = lm_heads[0].size(0);
    std::vector<const void*> hp, ep;
    for (size_t g = 0; g < lm_heads.size(); ++g) {
      check_bf16(lm_heads[g], {v, kHidden}, "lm_head");
      check_bf16(embeddings[g], {embeddings[g].size(0), kHidden}, "codec embedding");
      TORCH_CHECK(embeddings[g].size(0) >= v, "codec embedding ", g, " has fewer rows than the lm-head vocabulary");
      hp.push_back(lm_heads[g].data_ptr());
      ep.push_back(embeddings[g].data_ptr());
    }
    check_bf16(bb_embedding, {bb_embedding.size(0), kHidden}, "backbone codec embedding");
    bb_vocab_ = bb_embedding.size(0);
    heads_ = lm_heads;
    embs_ = embeddings;
    bb_emb_ = bb_embedding;
    cp_vocab_ = (int)v;
    d_heads_ = upload_struct(hp.data(), hp.size() * sizeof(void*), dev_);
    d_embs_ = upload_struct(ep.data(), ep.size() * sizeof(void*), dev_);
  }

  // Extended: one whole frame (2-token prefill + 14 decode steps + 15 heads + combine).
  void frame(torch::Tensor bb_hidden, torch::Tensor g0, c10::optional<torch::Tensor> text_row, torch::Tensor out_tokens,
             torch::Tensor out_combined, int64_t eos_id, torch::Tensor done, bool do_sample, double temperature,
             int64_t top_k, double top_p, int64_t seed, int64_t frame_step, c10::optional<torch::Tensor> history_slot) {
    TORCH_CHECK(!heads_.empty(), "call set_heads() before frame()");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev_);
    TORCH_CHECK(bb_hidden.is_cuda() && bb_hidden.scalar_type() == torch::kFloat32 && bb_hidden.numel() == kHidden &&
                    bb_hidden.is_contiguous(), "bb_hidden must be a contiguous f32 GPU tensor of 1024 values");
    TORCH_CHECK(g0.is_cuda() && g0.scalar_type() == torch::kInt32, "g0 must be an int32 GPU tensor");
    TORCH_CHECK(out_tokens.is_cuda() && out_tokens.scalar_type() == torch::kInt32 &&
                    out_tokens.numel() >= (int64_t)heads_.size() + 1, "out_tokens must be int32 GPU with >= groups+1 entries");
    TORCH_CHECK(out_combined.is_cuda() && out_combined.scalar_type() == torch::kBFloat16 && out_combined.numel() == kHidden,
                "out_combined must be a bf16 GPU tensor of 1024 values");
    TORCH_CHECK(done.is_cuda() && done.scalar_type() == torch::kInt32, "done must be an int32 GPU tensor");
    TORCH_CHECK((int)heads_.size() + 1 <= max_seq_len_, "max_seq_len too small for a frame");
    const void* tr = nullptr;
    if (text_row.has_value()) {
      TORCH_CHECK(text_row->is_cuda() && text_row->scalar_type() == torch::kBFloat16 && text_row->numel() == kHidden &&
                      text_row->is_contiguous(), "text_row must be a contiguous bf16 GPU tensor of 1024 values");
      tr = text_row->data_ptr();
    }
    int* hs = nullptr;
    if (history_slot.has_value()) {
      TORCH_CHECK(history_slot->is_cuda() && history_slot->scalar_type() == torch::kInt32 && history_slot->numel() >= 1,
                  "history_slot must be an int32 GPU tensor");
      hs = history_slot->data_ptr<int>();
    }
    QttsSampling s = sampling(do_sample, temperature, top_k, top_p, seed);
    hip_check(qtts_cp_frame(ws_.data_ptr(), reinterpret_cast<const CPLayerWeights*>(d_layer_weights_.data_ptr()),
                            num_layers_, final_norm_weight_.data_ptr(), cos_table_.data_ptr(), sin_table_.data_ptr(),
                            k_cache_.data_ptr(), v_cache_.data_ptr(), max_seq_len_, bb_hidden.data_ptr<float>(),
                            g0.data_ptr<int>(), bb_emb_.data_ptr(), reinterpret_cast<const void* const*>(d_heads_.data_ptr()),
                            reinterpret_cast<const void* const*>(d_embs_.data_ptr()), (int)heads_.size(), cp_vocab_, tr,
                            out_tokens.data_ptr<int>(), out_combined.data_ptr(), hs, (int)eos_id, done.data_ptr<int>(), &s,
                            (int)frame_step, cur_stream()),
              "qtts_cp_frame");
  }

  // Extended: frames of n (1..8) independent streams in one launch, stream s on XCD s (its own
  // workspace and KV cache, allocated on first use); row s of each argument belongs to stream s.
  void frames_streams(torch::Tensor bb_hidden, torch::Tensor g0, c10::optional<torch::Tensor> text_rows,
                      torch::Tensor out_tokens, torch::Tensor out_combined, int64_t eos_id, torch::Tensor done,
                      bool do_sample, double temperature, int64_t top_k, double top_p, int64_t seed, int64_t frame_step,
                      bool shared) {
    TORCH_CHECK(!heads_.empty(), "call set_heads() before frames_streams()");
    c10::hip::HIPGuardMasqueradingAsCUDA guard(dev_);
    const int64_t n = bb_hidden.size(0);
    const int64_t groups = (int64_t)heads_.size();
    TORCH_CHECK(n >= 1 && n <= kMaxStreams, "1..", kMaxStreams, " streams per launch, got ", n);
    TORCH_CHECK(bb_hidden.is_cuda() && bb_hidden.scalar_type() == torch::kFloat32 && bb_hidden.dim() == 2 &&
                    bb_hidden.size(1) == kHidden && bb_hidden.is_contiguous(), "bb_hidden must be contiguous f32 [n, 1024]");
    TORCH_CHECK(g0.is_cuda() && g0.scalar_type() == torch::kInt32 && g0.numel() == n && g0.is_contiguous(), "g0 must be int32 [n]");
    TORCH_CHECK(out_tokens.is_cuda() && out_tokens.scalar_type() == torch::kInt32 && out_tokens.dim() == 2 &&
                    out_tokens.size(0) == n && out_tokens.size(1) == groups + 1 && out_tokens.is_contiguous(),
                "out_tokens must be contiguous int32 [n, groups + 1]");
    TORCH_CHECK(out_combined.is_cuda() && out_combined.scalar_type() == torch::kBFloat16 && out_combined.dim() == 2 &&
                    out_combined.size(0) == n && out_combined.size(1) == kHidden && out_combined.is_contiguous(),
                "out_combined must be contiguous bf16 [n, 1024]");
    TORCH_CHECK(done.is_cuda() && done.scalar_type() == torch::kInt32 && done.numel() == n && done.is_contiguous(), "done must be int32 [n]");
    const void* tr = nullptr;
    if (text_rows.has_value()) {
      TORCH_CHECK(text_rows->is_cuda() && text_rows->scalar_type() == torch::kBFloat16 && text_rows->dim() == 2 &&
                      text_rows->size(0) == n && text_rows->size(1) == kHidden && text_rows->is_contiguous(),
                  "text_rows must be contiguous bf16 [n, 1024]");
      tr = text_rows->data_ptr();
    }
    if (!k_streams_.defined()) {
      auto f32 = torch::dtype(torch::kFloat32).device(dev_);
      k_streams_ = torch::zeros({kMaxStreams, num_layers_, kKVHeads, max_seq_len_, kHeadDim}, f32);
      v_streams_ = torch::zeros({kMaxStreams, num_layers_, kKVHeads, max_seq_len_, kHeadDim}, f32);
    }
    QttsSampling smp = sampling(do_sample, temperature, top_k, top_p, seed);
    if (shared) {
      ensure_shared_ws(ws_shared_, dev_);
      hip_check(qtts_cp_frame_shared((int)n, ws_shared_.data_ptr(), reinterpret_cast<const CPLayerWeights*>(d_layer_weights_.data_ptr()),
                                     num_layers_, final_norm_weight_.data_ptr(), cos_table_.data_ptr(), sin_table_.data_ptr(),
                                     k_streams_.data_ptr(), v_streams_.data_ptr(), max_seq_len_, bb_hidden.data_ptr<float>(),
                                     g0.data_ptr<int>(), bb_emb_.data_ptr(), reinterpret_cast<const void* const*>(d_heads_.data_ptr()),
                                     reinterpret_cast<const void* const*>(d_embs_.data_ptr()), (int)groups, cp_vocab_, tr,
                                     out_tokens.data_ptr<int>(), out_combined.data_ptr(), (int)eos_id, done.data_ptr<int>(), &smp,
                                     (int)frame_step, cur_stream()),
                "qtts_cp_frame_shared");
      return;
    }
    if (!ws_streams_.defined()) {
      ws_streams_ = torch::zeros({(int64_t)(kMaxStreams * qtts_workspace_bytes())}, torch::dtype(torch::kUInt8).device(dev_));
      hip_check(qtts_workspace_init(ws_streams_.data_ptr(), dev_.index()), "qtts_workspace_init");
    }
    hip_check(qtts_cp_frame_streams((int)n, ws_streams_.data_ptr(), reinterpret_cast<const CPLayerWeights*>(d_layer_weights_.data_ptr()),
                                    num_layers_, final_norm_weight_.data_ptr(), cos_table_.data_ptr(), sin_table_.data_ptr(),
                                    k_streams_.data_ptr(), v_streams_.data_ptr(), max_seq_len_, bb_hidden.data_ptr<float>(),
                                    g0.data_ptr<int>(), bb_emb_.data_ptr(), reinterpret_cast<const void* const*>(d_heads_.data_ptr()),
                                    reinterpret_cast<const void* const*>(d_embs_.data_ptr()), (int)groups, cp_vocab_, tr,
                                    out_tokens.data_ptr<int>(), out_combined.data_ptr(), (int)eos_id, done.data_ptr<int>(), &smp,
                                    (int)frame_step, cur_stream()),
              "qtts_cp_frame_streams");
  }
  void check_error_streams() const {
    check_shared_error(ws_shared_);
    if (!ws_streams_.defined()) return;
    for (int st = 0; st < kMaxStreams; ++st) {
      unsigned int code = 0;
      hip_check(qtts_workspace_check(static_cast<uint8_t*>(ws_streams_.data_ptr()) + st * qtts_workspace_bytes(), &code, cur_stream()),
                "qtts_workspace_check");
      TORCH_CHECK(code == 0, "stream ", st, ": decode kernel reported a device-side wait timeout (error word ", code, ")");
    }
  }


  void reset() {
    position_ = 0;
    k_cache_.zero_();
    v_cache_.zero_();
  }
  int64_t position() const { return position_; }
  void set_position(int64_t pos) {
    TORCH_CHECK(pos >= 0 && pos <= max_seq_len_, "position ", pos, " outside [0, ", max_seq_len_, "]");
    position_ = (int)pos;
  }
  torch::Tensor get_hidden_states() const { return g_normalized_.clone(); }
  torch::Tensor get_k_cache() const { return k_cache_; }
  torch::Tensor get_v_cache() const { return v_cache_; }
  void check_error() const { check_device_error(ws_); }
  // test hook: pre-sets the workspace's error word (after at least one launch), so that every
  // wait of the next launch gives up at its first check
  void debug_set_error(int64_t code) {
    hip_check(qtts_debug_set_error(ws_.data_ptr(), (unsigned int)code, cur_stream()), "qtts_debug_set_error");
  }

  void set_kv_cache(torch::Tensor k_cache, torch::Tensor v_cache) {
    TORCH_CHECK(k_cache.dim() == 4 && k_cache.sizes() == v_cache.sizes(), "k/v must be [layers, 8, seq, 128]");
    TORCH_CHECK(k_cache.size(0) == num_layers_ && k_cache.size(1) == kKVHeads && k_cache.size(3) == kHeadDim,
                "k/v must be [", num_layers_, ", 8, seq, 128], got ", k_cache.sizes());
    TORCH_CHECK(k_cache.size(2) <= max_seq_len_, "k/v longer than max_seq_len");
    using namespace torch::indexing;
    k_cache_.index_put_({Slice(), Slice(), Slice(0, k_cache.size(2)), Slice()}, k_cache.to(dev_, torch::kFloat32));
    v_cache_.index_put_({Slice(), Slice(), Slice(0, v_cache.size(2)), Slice()}, v_cache.to(dev_, torch::kFloat32));
  }

 private:
  int num_layers_, max_seq_len_, position_, cp_vocab_ = 0;
  int64_t bb_vocab_ = 0;
  torch::Device dev_;
  torch::Tensor final_norm_weight_, cos_table_, sin_table_, d_layer_weights_;
  std::vector<torch::Tensor> layer_weights_tensors_, heads_, embs_;
  torch::Tensor bb_emb_, d_heads_, d_embs_;
  torch::Tensor k_cache_, v_cache_, hidden_buffer_, g_normalized_, ws_;
  torch::Tensor ws_streams_, k_streams_, v_streams_;   // frames_streams(): per-stream workspaces and KV caches
  torch::Tensor ws_shared_;                            // frames_streams(shared=True): the weight-shared launches' workspace
};

}  // namespace

PYBIND11_MODULE(_qwentts_amd_C, m) {
  m.doc() = "MI355X decode kernels for Qwen3-TTS (backbone + code predictor)";
  m.def("workspace_bytes", []() { return (int64_t)qtts_workspace_bytes(); });
  m.def("shutdown", []() { hip_check(qtts_shutdown(), "qtts_shutdown"); },
        "Free the library-owned workspaces (synchronises their devices); registered with atexit by the loader.");
  m.def("set_trace", [](c10::optional<torch::Tensor> buf) {
    if (!buf.has_value()) { hip_check(qtts_debug_trace(nullptr, 0), "qtts_debug_trace"); return; }
    TORCH_CHECK(buf->is_cuda() && buf->is_contiguous(), "trace buffer must be a contiguous GPU tensor");
    hip_check(qtts_debug_trace(buf->data_ptr(), (size_t)buf->numel() * buf->element_size()), "qtts_debug_trace");
  }, py::arg("buffer") = py::none());
  m.def("set_trace_shared", [](c10::optional<torch::Tensor> buf) {
    if (!buf.has_value()) { hip_check(qtts_debug_trace_shared(nullptr, 0), "qtts_debug_trace_shared"); return; }
    TORCH_CHECK(buf->is_cuda() && buf->is_contiguous(), "trace buffer must be a contiguous GPU tensor");
    hip_check(qtts_debug_trace_shared(buf->data_ptr(), (size_t)buf->numel() * buf->element_size()), "qtts_debug_trace_shared");
  }, py::arg("buffer") = py::none());
  py::class_<MegakernelTTSDecoder>(m, "MegakernelTTSDecoder")
      .def(py::init<torch::Tensor, std::vector<torch::Tensor>, torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor,
                    int64_t, int64_t>())
      .def("decode_step", &MegakernelTTSDecoder::decode_step)
      .def("decode_step_with_argmax", &MegakernelTTSDecoder::decode_step_with_argmax)
      .def("decode_step_with_embedding", &MegakernelTTSDecoder::decode_step_with_embedding)
      .def("decode_step_3d", &MegakernelTTSDecoder::decode_step_3d)
      .def("decode_step_select", &MegakernelTTSDecoder::decode_step_select, py::arg("input_embedding"),
           py::arg("out_token"), py::arg("history"), py::arg("n_history"), py::arg("repetition_penalty"),
           py::arg("eos_id"), py::arg("suppress_eos"), py::arg("do_sample"), py::arg("temperature"), py::arg("top_k"),
           py::arg("top_p"), py::arg("seed"), py::arg("frame_step"), py::arg("pos3") = py::none(),
           py::arg("skip_if") = py::none())
      .def("reset", &MegakernelTTSDecoder::reset)
      .def("position", &MegakernelTTSDecoder::position)
      .def("set_position", &MegakernelTTSDecoder::set_position)
      .def("get_hidden_states", &MegakernelTTSDecoder::get_hidden_states)
      .def("get_k_cache", &MegakernelTTSDecoder::get_k_cache)
      .def("get_v_cache", &MegakernelTTSDecoder::get_v_cache)
      .def("set_kv_cache", &MegakernelTTSDecoder::set_kv_cache)
      .def("hidden_state_buffer", &MegakernelTTSDecoder::hidden_state_buffer)
      .def("residual_buffer", &MegakernelTTSDecoder::residual_buffer)
      .def("logits_buffer", &MegakernelTTSDecoder::logits_buffer)
      .def("prefill", &MegakernelTTSDecoder::prefill, py::arg("embeds"), py::arg("out_token") = py::none(),
           py::arg("eos_id") = -1, py::arg("suppress_eos") = false, py::arg("do_sample") = false,
           py::arg("temperature") = 1.0, py::arg("top_k") = 0, py::arg("top_p") = 1.0, py::arg("seed") = 0,
           py::arg("pos3") = py::none())
      .def("decode_steps_streams", &MegakernelTTSDecoder::decode_steps_streams, py::arg("decoders"), py::arg("embeds"),
           py::arg("out_tokens"), py::arg("hidden_out"), py::arg("history"), py::arg("n_history"),
           py::arg("repetition_penalty"), py::arg("eos_id"), py::arg("suppress_eos"), py::arg("do_sample"),
           py::arg("temperature"), py::arg("top_k"), py::arg("top_p"), py::arg("seed"), py::arg("frame_step"),
           py::arg("skip") = py::none(), py::arg("shared") = false)
      .def("check_error_streams", &MegakernelTTSDecoder::check_error_streams)
      .def("debug_set_error", &MegakernelTTSDecoder::debug_set_error)
      .def("check_error", &MegakernelTTSDecoder::check_error);
  py::class_<MegakernelCodePredictorDecoder>(m, "MegakernelCodePredictorDecoder")
      .def(py::init<std::vector<torch::Tensor>, torch::Tensor, torch::Tensor, torch::Tensor, int64_t, int64_t>())
      .def("decode_step_with_embedding", &MegakernelCodePredictorDecoder::decode_step_with_embedding)
      .def("set_heads", &MegakernelCodePredictorDecoder::set_heads)
      .def("frames_streams", &MegakernelCodePredictorDecoder::frames_streams, py::arg("bb_hidden"), py::arg("g0"),
           py::arg("text_rows"), py::arg("out_tokens"), py::arg("out_combined"), py::arg("eos_id"), py::arg("done"),
           py::arg("do_sample"), py::arg("temperature"), py::arg("top_k"), py::arg("top_p"), py::arg("seed"),
           py::arg("frame_step"), py::arg("shared") = false)
      .def("check_error_streams", &MegakernelCodePredictorDecoder::check_error_streams)
      .def("frame", &MegakernelCodePredictorDecoder::frame, py::arg("bb_hidden"), py::arg("g0"), py::arg("text_row"),
           py::arg("out_tokens"), py::arg("out_combined"), py::arg("eos_id"), py::arg("done"), py::arg("do_sample"),
           py::arg("temperature"), py::arg("top_k"), py::arg("top_p"), py::arg("seed"), py::arg("frame_step"),
           py::arg("history_slot") = py::none())
      .def("reset", &MegakernelCodePredictorDecoder::reset)
      .def("position", &MegakernelCodePredictorDecoder::position)
      .def("set_position", &MegakernelCodePredictorDecoder::set_position)
      .def("get_hidden_states", &MegakernelCodePredictorDecoder::get_hidden_states)
      .def("get_k_cache", &MegakernelCodePredictorDecoder::get_k_cache)
      .def("get_v_cache", &MegakernelCodePredictorDecoder::get_v_cache)
      .def("set_kv_cache", &MegakernelCodePredictorDecoder::set_kv_cache)
      .def("debug_set_error", &MegakernelCodePredictorDecoder::debug_set_error)
      .def("check_error", &MegakernelCodePredictorDecoder::check_error);
}
