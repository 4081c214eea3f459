// Offline IDX reader for MNIST (src/dataset.rs:116-161): big-endian u32
// header fields, u8 payload; images are scaled to f32 in [0, 1] by /255 and
// shaped [count, 784]. There is no download path (dataset.rs:170-196 fetches
// and gunzips with ureq/flate2): files must already be unpacked on disk.
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "tensor.hpp"

namespace fg {

namespace {

struct File {
  std::FILE* f = nullptr;
  explicit File(const std::string& path) : f(std::fopen(path.c_str(), "rb")) {
    if (!f) fail("io: " + path + ": " + std::strerror(errno));
  }
  ~File() {
    if (f) std::fclose(f);
  }
  void read_exact(void* dst, size_t n, const std::string& path) {
    if (std::fread(dst, 1, n, f) != n) fail("io: " + path + ": failed to fill whole buffer");
  }
  uint32_t read_u32(const std::string& path) {  // dataset.rs:163-167
    unsigned char b[4];
    read_exact(b, 4, path);
    return (uint32_t(b[0]) << 24) | (uint32_t(b[1]) << 16) | (uint32_t(b[2]) << 8) | uint32_t(b[3]);
  }
};

}  // namespace

// dataset.rs:116-142
Tensor idx_images(const std::string& path, DeviceId dev) {
  File file(path);
  uint32_t magic = file.read_u32(path);
  if (magic != 2051) fail("bad IDX format: expected IDX image magic 2051, got " + std::to_string(magic));
  size_t count = file.read_u32(path), rows = file.read_u32(path), cols = file.read_u32(path);
  if (rows != 28 || cols != 28)
    fail("bad IDX format: expected 28x28 images, got " + std::to_string(rows) + "x" + std::to_string(cols));
  std::vector<unsigned char> pixels(count * rows * cols);
  file.read_exact(pixels.data(), pixels.size(), path);
  std::vector<float> data(pixels.size());
  for (size_t i = 0; i < pixels.size(); i++) data[i] = static_cast<float>(pixels[i]) / 255.0f;
  return Tensor::new_f32(data, Shape{count, 784}, dev);
}

// dataset.rs:144-157
std::vector<uint8_t> idx_labels(const std::string& path) {
  File file(path);
  uint32_t magic = file.read_u32(path);
  if (magic != 2049) fail("bad IDX format: expected IDX label magic 2049, got " + std::to_string(magic));
  size_t count = file.read_u32(path);
  std::vector<uint8_t> labels(count);
  file.read_exact(labels.data(), count, path);
  return labels;
}

}  // namespace fg
