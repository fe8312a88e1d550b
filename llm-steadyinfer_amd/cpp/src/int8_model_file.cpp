// INT8 model file loader (see model/int8_model_file.h for the reference lines each step follows).
#include "model/int8_model_file.h"
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#include <cstdio>
#include <cstdlib>

namespace model {

RawModelDataInt8::~RawModelDataInt8() {
  if (data != nullptr && data != MAP_FAILED) munmap(data, file_size);
  if (fd != -1) close(fd);
}

namespace {

// Bytes one quantised block occupies in the file: int8 values then fp32 scales.
size_t block_bytes(int64_t rows, int64_t cols, int32_t group_size) {
  const int64_t n = rows * cols;
  return static_cast<size_t>(n) + static_cast<size_t>(n / group_size) * sizeof(float);
}

}  // namespace

base::Status Int8ModelFile::open(const std::string& path) {
  FILE* file = std::fopen(path.c_str(), "rb");
  if (!file) return base::error::PathNotValid("Failed to open the model file " + path);
  ModelConfig header;
  const bool ok_header = std::fread(&header, sizeof(ModelConfig), 1, file) == 1;
  const bool ok_group = ok_header && std::fread(&group_size_, sizeof(int32_t), 1, file) == 1;
  std::fclose(file);
  if (!ok_header) return base::error::ModelParseError("Failed to read the model configuration");
  if (!ok_group) return base::error::ModelParseError("Failed to read the group size");
  if (header.dim <= 0 || header.hidden_dim <= 0 || header.layer_num <= 0 || header.head_num <= 0 ||
      header.kv_head_num <= 0 || header.vocab_size == 0 || group_size_ <= 0)
    return base::error::ModelParseError("Invalid model configuration in " + path);

  config_ = TransformerConfig{};
  config_.dim_ = header.dim;
  config_.hidden_dim_ = header.hidden_dim;
  config_.layer_num_ = header.layer_num;
  config_.head_num_ = header.head_num;
  config_.kv_head_num_ = header.kv_head_num;
  config_.seq_len_ = header.seq_len;
  config_.kv_dim_ = (header.dim * header.kv_head_num) / header.head_num;
  config_.kv_mul_ = header.head_num / header.kv_head_num;
  config_.head_size_ = header.dim / header.head_num;
  config_.immediate_dim_ = header.immediate_dim_;
  config_.rope_theta_ = header.rope_theta_;
  config_.is_shared_weight_ = header.vocab_size > 0;
  config_.vocab_size_ = std::abs(header.vocab_size);

  // Cursor over the weights, as create_quant_layers walks them.
  const int64_t d = config_.dim_, h = config_.hidden_dim_, kv = config_.kv_dim_, L = config_.layer_num_;
  const int64_t vocab = config_.vocab_size_;
  if ((d * d) % group_size_ || (kv * d) % group_size_ || (h * d) % group_size_ ||
      (vocab * d) % group_size_)
    return base::error::ModelParseError("Projection sizes are not multiples of the group size");
  size_t pos = L * (2 * block_bytes(d, d, group_size_) + 2 * block_bytes(kv, d, group_size_) +
                    3 * block_bytes(h, d, group_size_));
  if (!config_.is_shared_weight_) pos += block_bytes(vocab, d, group_size_);
  pos += static_cast<size_t>(vocab * d) * sizeof(float);
  pos += static_cast<size_t>((2 * L + 1) * d) * sizeof(float);
  weights_end_ = pos;

  auto raw = std::make_shared<RawModelDataInt8>();
  raw->fd = ::open(path.c_str(), O_RDONLY);
  if (raw->fd == -1) return base::error::PathNotValid("Failed to open the model file " + path);
  struct stat sb;
  if (fstat(raw->fd, &sb) == -1) return base::error::ModelParseError("Failed to stat " + path);
  raw->file_size = static_cast<size_t>(sb.st_size);
  const size_t head = sizeof(ModelConfig) + sizeof(int32_t);
  if (raw->file_size < head + weights_end_)
    return base::error::ModelParseError("Model file " + path + " is shorter than its layout");
  raw->data = mmap(nullptr, raw->file_size, PROT_READ, MAP_PRIVATE, raw->fd, 0);
  if (raw->data == MAP_FAILED || raw->data == nullptr)
    return base::error::ModelParseError("Failed to map the weight file " + path + " into memory.");
  raw->weight_data = static_cast<int8_t*>(raw->data) + head;
  raw_ = std::move(raw);
  return base::error::Success();
}

base::Status Int8ModelFile::create_quant_layers(base::DeviceType device_type,
                                                QuantLayers* layers) const {
  if (!raw_) return base::error::InternalError("Model file not opened");
  if (!layers) return base::error::InvalidArgument("Null layer table");
  const auto cpu = base::DeviceType::kDeviceCPU;
  const int32_t d = config_.dim_, h = config_.hidden_dim_, kv = config_.kv_dim_;
  size_t pos = 0;
  auto bind = [&](int32_t rows, int32_t cols,
                  std::vector<std::shared_ptr<op::MatmulLayer>>& dst) -> base::Status {
    for (int32_t i = 0; i < config_.layer_num_; ++i) {
      auto layer = std::make_shared<op::MatmulLayer>(device_type, rows, cols, true);
      layer->set_group_size(group_size_);
      base::Status st = layer->set_weight(0, {rows, cols}, raw_->weight(pos), cpu);
      if (!st) return st;
      dst.push_back(layer);
      pos += static_cast<size_t>(rows) * cols + layer->get_scale_num() * sizeof(float);
    }
    return base::error::Success();
  };
  base::Status st;
  if (!(st = bind(d, d, layers->wq))) return st;
  if (!(st = bind(kv, d, layers->wk))) return st;
  if (!(st = bind(kv, d, layers->wv))) return st;
  if (!(st = bind(d, d, layers->wo))) return st;
  if (!(st = bind(h, d, layers->w1))) return st;
  if (!(st = bind(d, h, layers->w2))) return st;
  if (!(st = bind(h, d, layers->w3))) return st;

  const int32_t vocab = config_.vocab_size_;
  layers->cls = std::make_shared<op::MatmulLayer>(device_type, vocab, d, true);
  layers->cls->set_group_size(group_size_);
  if (!(st = layers->cls->set_weight(0, {vocab, d}, raw_->weight(pos), cpu))) return st;
  // A positive header vocab_size marks a shared classifier: the cursor is not advanced, so the
  // classifier is bound at the start of the fp32 embedding (llama3.cpp:268-277).
  if (!config_.is_shared_weight_)
    pos += static_cast<size_t>(vocab) * d + layers->cls->get_scale_num() * sizeof(float);

  const float* fp = static_cast<const float*>(raw_->weight(pos));
  layers->embedding = fp;
  fp += static_cast<size_t>(vocab) * d;
  layers->rmsnorm.clear();
  for (int32_t i = 0; i < 2 * config_.layer_num_ + 1; ++i) {
    layers->rmsnorm.push_back(fp);
    fp += d;
  }
  return base::error::Success();
}

}  // namespace model
