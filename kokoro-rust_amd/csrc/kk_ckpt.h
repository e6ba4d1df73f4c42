// kk_ckpt.h -- PyTorch zip checkpoints (torch.save) read on the host: the model file (a dict of
// state dicts) and the voice packs (one tensor).  Internal to the library; the C ABI is in
// include/kokoro_hip.h.
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace kk {

struct HostTensor {
    std::vector<int64_t> shape;
    std::vector<float> data;  // row-major, contiguous
};

// Parses a torch.save zip archive (STORED entries only) and interprets its data.pkl with a
// restricted pickle machine (no code runs: only the opcodes torch.save emits for f32 tensors in
// (ordered) dicts, and the globals collections.OrderedDict, torch._utils._rebuild_tensor_v2 and
// torch.FloatStorage).  Throws std::runtime_error with a message on anything else.
// Model file: {submodule: state_dict} -> "submodule.param", a leading "module." of a parameter
// name stripped (src/torchpt.rs:311-327).
std::map<std::string, HostTensor> read_model_checkpoint(const std::string& path);
// Voice pack: a single tensor of shape [rows, 1, 256] (src/torchpt.rs:329-335).
HostTensor read_voice_pack(const std::string& path);
// The same from an archive already in memory (`path` names it in messages).
std::map<std::string, HostTensor> read_model_checkpoint_bytes(std::vector<uint8_t> data, const std::string& path);
HostTensor read_voice_pack_bytes(std::vector<uint8_t> data, const std::string& path);

// torch._weight_norm(v, g, dim = 0): w = v * (g / ||v||), the norm over all but the first dim,
// summed in f64 (src/ops.rs:9-23).
void weight_norm(const float* v, const float* g, int64_t rows, int64_t per_row, float* w);

}  // namespace kk
