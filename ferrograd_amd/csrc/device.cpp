// Device registry, buffer identity and program cache (src/device.rs:96-360).
#include "device.hpp"

#include <atomic>
#include <cstdlib>
#include <cstring>

namespace fg {

void Device::copy_to_host_into(const Buffer& b, void* dst, size_t nbytes) {
  std::vector<uint8_t> v = copy_to_host(b);
  FG_CHECK(v.size() == nbytes, "copy_to_host: expected " + std::to_string(v.size()) + " bytes, got " +
                                   std::to_string(nbytes));
  if (nbytes) std::memcpy(dst, v.data(), nbytes);
}

size_t next_buffer_id() {  // device.rs:230-234
  static std::atomic<size_t> next{0};
  return next.fetch_add(1);
}

void BufferInner::ensure_allocated() {  // device.rs:191-213
  if (realized) return;
  get_device(device).realize_storage(*this, true);
}

BufferInner::~BufferInner() {
  if (realized && has_device(device)) get_device(device).release(*this);
}

Buffer Device::reserve_buffer(DType dtype, size_t numel) {
  auto b = std::make_shared<BufferInner>();
  b->id = next_buffer_id();
  b->device = id();
  b->dtype = dtype;
  b->numel = numel;
  return b;
}

std::shared_ptr<Program> Device::cached_program(const UOp& sink) {
  auto it = programs_.find(sink);
  return it == programs_.end() ? nullptr : it->second;
}

void Device::insert_program(const UOp& sink, std::shared_ptr<Program> p) { programs_[sink] = std::move(p); }

void Device::clear_for_tests() { programs_.clear(); }

void Device::read_async(const Buffer& b, int slot) {
  std::vector<uint8_t> bytes = copy_to_host(b);
  for (auto& s : read_slots_)
    if (s.first == slot) {
      s.second = std::move(bytes);
      return;
    }
  read_slots_.emplace_back(slot, std::move(bytes));
}

std::vector<uint8_t> Device::read_wait(int slot) {
  for (auto it = read_slots_.begin(); it != read_slots_.end(); ++it)
    if (it->first == slot) {
      std::vector<uint8_t> out = std::move(it->second);
      read_slots_.erase(it);
      return out;
    }
  fail("read_wait: no read queued in slot " + std::to_string(slot));
}

namespace {
Device* g_devices[2] = {nullptr, nullptr};
}

bool has_device(DeviceId id) {
  int i = static_cast<int>(id);
  if (!g_devices[i] && id == DeviceId::Hip) g_devices[i] = make_hip_device();
  return g_devices[i] != nullptr;
}

Device& get_device(DeviceId id) {
  int i = static_cast<int>(id);
  if (!g_devices[i] && id == DeviceId::Hip) g_devices[i] = make_hip_device();
  FG_CHECK(g_devices[i] != nullptr,
           std::string("device '") + device_name(id) +
               "' is not registered (the CPU device is provided by the oracle test harness)");
  return *g_devices[i];
}

void register_device(DeviceId id, Device* dev) { g_devices[static_cast<int>(id)] = dev; }

DeviceId default_device() {
  static const std::string raw = [] {
    const char* e = std::getenv("DEVICE");
    return std::string(e ? e : "");
  }();
  if (raw.empty() || raw == "hip") return DeviceId::Hip;
  if (raw == "cpu") return DeviceId::Cpu;
  FG_CHECK(false, "DEVICE must be 'hip' or 'cpu'; got '" + raw + "'");
  return DeviceId::Hip;
}

}  // namespace fg
