// Model: the vision encoder and the decoder loaded by checkpoint names.

#include "model/rocm/model.h"

#include <algorithm>
#include <stdexcept>
#include <string>
#include <utility>

#include "backend/rocm/ops.h"

namespace uocr::rocm {
namespace {

std::int64_t count_of(const HostTensor& t) {
  std::int64_t n = 1;
  for (std::int64_t d : t.shape) n *= d;
  return n;
}

std::string layer(const char* root, std::int64_t i) { return std::string(root) + std::to_string(i) + "."; }

}  // namespace

std::vector<float> Model::host(const std::string& name, std::int64_t n) const {
  HostTensor t = src_.get(name);
  if (count_of(t) != n || static_cast<std::int64_t>(t.data.size()) != n) {
    throw std::invalid_argument("Model: " + name + " holds " + std::to_string(t.data.size()) + " values, expected " +
                                std::to_string(n));
  }
  return std::move(t.data);
}

const float* Model::vector(const std::string& name, std::int64_t n) {
  const std::vector<float> v = host(name, n);
  owned_.emplace_back(ctx_, DType::kF32, n);
  owned_.back().upload(v.data(), n);
  return owned_.back().f32();
}

const std::uint16_t* Model::matrix(const std::string& name, std::int64_t rows, std::int64_t cols) {
  HostTensor t = src_.get(name);
  if (t.shape.empty() || t.shape[0] != rows || count_of(t) != rows * cols ||
      static_cast<std::int64_t>(t.data.size()) != rows * cols) {
    throw std::invalid_argument("Model: " + name + " is not [" + std::to_string(rows) + ", " + std::to_string(cols) +
                                "]");
  }
  owned_.emplace_back(ctx_, DType::kBF16, rows * cols);
  owned_.back().upload(t.data.data(), rows * cols);  // nearest even
  return owned_.back().bf16();
}

// Matrices of `rows` rows each, one after another in one bf16 array (the
// reference's stacked expert weights, cuda_decoder.cpp:73-85).
const std::uint16_t* Model::stacked(const std::vector<std::string>& names, std::int64_t rows, std::int64_t cols) {
  const auto n = static_cast<std::int64_t>(names.size());
  owned_.emplace_back(ctx_, DType::kBF16, n * rows * cols);
  Array& a = owned_.back();
  for (std::int64_t i = 0; i < n; ++i) {
    const std::vector<float> v = host(names[static_cast<std::size_t>(i)], rows * cols);
    a.upload(v.data(), rows * cols, i * rows * cols);
  }
  return a.bf16();
}

Model::Model(const Context& ctx, const TensorSource& weights, const ModelDims& dims)
    : ctx_(ctx), src_(weights), dims_(dims) {
  // ---- vision (cuda_vision.cpp:54-115) ----
  const SamDims& s = dims.vision.sam;
  const ClipDims& c = dims.vision.clip;
  const std::int64_t pg = s.image / s.patch, hd = s.width / s.heads, H = dims.decoder.hidden;
  VisionWeights vw;
  const std::string sam = "model.sam_model.";
  vw.patch = matrix(sam + "patch_embed.proj.weight", s.width, 3 * s.patch * s.patch);
  vw.patch_b = vector(sam + "patch_embed.proj.bias", s.width);
  vw.sam_pos = host(sam + "pos_embed", pg * pg * s.width);
  for (std::int64_t i = 0; i < s.layers; ++i) {
    const std::string p = layer("model.sam_model.blocks.", i);
    const bool global = std::find(s.global_layers.begin(), s.global_layers.end(), i) != s.global_layers.end();
    const std::int64_t span = global ? pg : s.window;
    SamBlockWeights b;
    b.norm1_w = vector(p + "norm1.weight", s.width);
    b.norm1_b = vector(p + "norm1.bias", s.width);
    b.qkv = matrix(p + "attn.qkv.weight", 3 * s.width, s.width);
    b.qkv_b = vector(p + "attn.qkv.bias", 3 * s.width);
    b.proj = matrix(p + "attn.proj.weight", s.width, s.width);
    b.proj_b = vector(p + "attn.proj.bias", s.width);
    b.rel_h = host(p + "attn.rel_pos_h", (2 * span - 1) * hd);
    b.rel_w = host(p + "attn.rel_pos_w", (2 * span - 1) * hd);
    b.norm2_w = vector(p + "norm2.weight", s.width);
    b.norm2_b = vector(p + "norm2.bias", s.width);
    b.lin1 = matrix(p + "mlp.lin1.weight", s.mlp, s.width);
    b.lin1_b = vector(p + "mlp.lin1.bias", s.mlp);
    b.lin2 = matrix(p + "mlp.lin2.weight", s.width, s.mlp);
    b.lin2_b = vector(p + "mlp.lin2.bias", s.width);
    vw.sam_blocks.push_back(std::move(b));
  }
  vw.neck0 = matrix(sam + "neck.0.weight", s.neck, s.width);
  vw.neck1_w = vector(sam + "neck.1.weight", s.neck);
  vw.neck1_b = vector(sam + "neck.1.bias", s.neck);
  vw.neck2 = matrix(sam + "neck.2.weight", s.neck, s.neck * 9);
  vw.neck3_w = vector(sam + "neck.3.weight", s.neck);
  vw.neck3_b = vector(sam + "neck.3.bias", s.neck);
  vw.net2 = matrix(sam + "net_2.weight", s.net2, s.neck * 9);
  vw.net3 = matrix(sam + "net_3.weight", s.net3, s.net2 * 9);
  const std::string clip = "model.vision_model.";
  vw.class_embedding = vector(clip + "embeddings.class_embedding", c.width);
  vw.clip_pos = host(clip + "embeddings.position_embedding.weight", c.positions * c.width);
  vw.pre_ln_w = vector(clip + "pre_layrnorm.weight", c.width);  // upstream's spelling
  vw.pre_ln_b = vector(clip + "pre_layrnorm.bias", c.width);
  for (std::int64_t i = 0; i < c.layers; ++i) {
    const std::string p = layer("model.vision_model.transformer.layers.", i);
    ClipLayerWeights l;
    l.ln1_w = vector(p + "layer_norm1.weight", c.width);
    l.ln1_b = vector(p + "layer_norm1.bias", c.width);
    l.qkv = matrix(p + "self_attn.qkv_proj.weight", 3 * c.width, c.width);
    l.qkv_b = vector(p + "self_attn.qkv_proj.bias", 3 * c.width);
    l.out = matrix(p + "self_attn.out_proj.weight", c.width, c.width);
    l.out_b = vector(p + "self_attn.out_proj.bias", c.width);
    l.ln2_w = vector(p + "layer_norm2.weight", c.width);
    l.ln2_b = vector(p + "layer_norm2.bias", c.width);
    l.fc1 = matrix(p + "mlp.fc1.weight", c.mlp, c.width);
    l.fc1_b = vector(p + "mlp.fc1.bias", c.mlp);
    l.fc2 = matrix(p + "mlp.fc2.weight", c.width, c.mlp);
    l.fc2_b = vector(p + "mlp.fc2.bias", c.width);
    vw.clip_layers.push_back(std::move(l));
  }
  vw.projector = matrix("model.projector.layers.weight", H, c.width + s.net3);
  vw.projector_b = vector("model.projector.layers.bias", H);
  vw.newline = host("model.image_newline", H);
  vw.separator = host("model.view_seperator", H);  // upstream's spelling
  VisionDims vd = dims.vision;
  vd.hidden = H;
  vision_ = std::make_unique<VisionEncoder>(ctx, vd, std::move(vw));

  // ---- decoder (cuda_decoder.cpp:33-71) ----
  const DecoderDims& d = dims.decoder;
  const std::int64_t W = d.heads * d.head_dim, D = d.index_dim;
  embed_ = matrix("model.embed_tokens.weight", d.vocab, H);
  std::vector<LayerWeights> layers;
  for (std::int64_t i = 0; i < dims.layers; ++i) {
    const std::string p = layer("model.layers.", i);
    const std::string r = p + "self_attn.dash_router.";
    LayerWeights l;
    l.input_norm = vector(p + "input_layernorm.weight", H);
    l.post_norm = vector(p + "post_attention_layernorm.weight", H);
    // [Wq; Wk; Wv; router Wq; router Wk]: the decode step's one stacked GEMV
    owned_.emplace_back(ctx, DType::kBF16, (3 * W + 2 * D) * H);
    Array& qkv = owned_.back();
    std::int64_t at = 0;
    for (const auto& [name, rows] : {std::pair<std::string, std::int64_t>{p + "self_attn.q_proj.weight", W},
                                     {p + "self_attn.k_proj.weight", W},
                                     {p + "self_attn.v_proj.weight", W},
                                     {r + "q_proj.weight", D},
                                     {r + "k_proj.weight", D}}) {
      const std::vector<float> v = host(name, rows * H);
      qkv.upload(v.data(), rows * H, at);
      at += rows * H;
    }
    l.qkv = qkv.bf16();
    l.o = matrix(p + "self_attn.o_proj.weight", H, W);
    l.router_q_norm = vector(r + "q_norm.weight", D);
    l.router_k_norm = vector(r + "k_norm.weight", D);
    l.head_cls = vector(r + "head_cls", D);
    if (i < dims.first_moe_layer) {
      l.gate = matrix(p + "mlp.gate_proj.weight", dims.dense_ffn, H);
      l.up = matrix(p + "mlp.up_proj.weight", dims.dense_ffn, H);
      l.down = matrix(p + "mlp.down_proj.weight", H, dims.dense_ffn);
      l.ffn = dims.dense_ffn;
    } else {
      auto m = std::make_unique<MoeWeights>();
      const std::int64_t E = dims.routed_experts, F = dims.expert_ffn, SF = dims.shared_experts * F;
      m->gate = vector(p + "mlp.gate.weight", E * H);  // fp32: expert choice unperturbed by bf16
      auto names = [&](const char* proj) {
        std::vector<std::string> out;
        for (std::int64_t e = 0; e < E; ++e) out.push_back(p + "mlp.experts." + std::to_string(e) + "." + proj);
        return out;
      };
      m->gate_stack = stacked(names("gate_proj.weight"), F, H);
      m->up_stack = stacked(names("up_proj.weight"), F, H);
      m->down_stack = stacked(names("down_proj.weight"), H, F);
      m->experts = E;
      m->top_k = dims.experts_per_token;
      m->expert_ffn = F;
      m->shared_gate = matrix(p + "mlp.shared_experts.gate_proj.weight", SF, H);
      m->shared_up = matrix(p + "mlp.shared_experts.up_proj.weight", SF, H);
      m->shared_down = matrix(p + "mlp.shared_experts.down_proj.weight", H, SF);
      m->shared_ffn = SF;
      l.moe = m.get();
      moe_.push_back(std::move(m));
    }
    layers.push_back(l);
  }
  const float* final_norm = vector("model.norm.weight", H);
  const std::uint16_t* lm_head = matrix("lm_head.weight", d.vocab, H);
  decoder_ = std::make_unique<DecodeStep>(ctx, d, embed_, std::move(layers), final_norm, lm_head);
  session_ = std::make_unique<Decoder>(ctx, *decoder_, embed_, d.vocab, H);
}

Model::~Model() = default;

std::vector<float> Model::encode_page(const View& global, const std::vector<View>& tiles, std::int64_t tiles_wide,
                                      std::int64_t tiles_high) const {
  return vision_->encode_page(global, tiles, tiles_wide, tiles_high);
}

std::vector<float> Model::embed(const std::vector<std::int64_t>& ids) const { return session_->embed(ids); }

}  // namespace uocr::rocm
