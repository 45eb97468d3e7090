// Host-side driver for the safetensors tests (no GPU calls): the Python test
// writes files with the `safetensors` package and HF model classes, runs one
// of these modes, and reads the output back with `safetensors`.
//
//   convert <in> <out> <transpose 0|1>      every tensor through read_host
//                                           (2-D ones transposed if asked),
//                                           written with write_safetensors,
//                                           metadata copied
//   mapping <gpt2|qwen|gemma> <n_layer>     "internal<TAB>hf" lines
//   load_mapped <arch> <n_layer> <in> <out> <transpose 0|1>
//                                           read_mapped_host under the
//                                           arch's mapping, written out
//                                           under the internal names
//   header <in>                             parse_header only
// Errors print "error: <what>" and exit 1.
#include <cstdio>
#include <cstdlib>
#include <map>
#include <stdexcept>
#include <string>

#include "finetune_ops/graph/safetensors_loader.h"

using namespace ops;

namespace {

std::unordered_map<std::string, std::string> mapping_for(const std::string& arch, int n) {
  if (arch == "gpt2") return GPT2KeyMapper::generate_gpt2_mapping(n);
  if (arch == "qwen") return QwenKeyMapper::generate_qwen_mapping(n);
  if (arch == "gemma") return GemmaKeyMapper::generate_gemma_mapping(n);
  throw std::invalid_argument("unknown arch " + arch);
}

void write_host(const std::string& out, const std::vector<HostTensor>& ts, const std::map<std::string, std::string>& md) {
  std::vector<SafeTensorsEntry> entries;
  for (const auto& h : ts)
    entries.push_back({h.name, h.dtype == kFloat16 ? "F16" : "F32", h.shape, h.bytes.data(), h.bytes.size()});
  write_safetensors(out, entries, md);
}

int run(int argc, char** argv) {
  if (argc < 2) throw std::invalid_argument("mode expected");
  const std::string mode = argv[1];
  if (mode == "convert" && argc == 5) {
    SafeTensorsReader r(argv[2]);
    r.parse_header();
    std::vector<HostTensor> ts;
    for (const auto& name : r.get_tensor_names())
      ts.push_back(r.read_host(name, std::atoi(argv[4]) && r.tensor_info(name).shape.size() == 2));
    write_host(argv[3], ts, r.metadata());
    return 0;
  }
  if (mode == "mapping" && argc == 4) {
    for (const auto& kv : mapping_for(argv[2], std::atoi(argv[3]))) std::printf("%s\t%s\n", kv.first.c_str(), kv.second.c_str());
    return 0;
  }
  if (mode == "load_mapped" && argc == 7) {
    SafeTensorsReader r(argv[4]);
    r.parse_header();
    SafeTensorsLoadOptions opts;
    opts.transpose_linear = std::atoi(argv[6]) != 0;
    opts.verbose = false;
    write_host(argv[5], r.read_mapped_host(mapping_for(argv[2], std::atoi(argv[3])), opts), {});
    return 0;
  }
  if (mode == "header" && argc == 3) {
    SafeTensorsReader r(argv[2]);
    r.parse_header();
    std::printf("%zu tensors\n", r.get_tensor_names().size());
    return 0;
  }
  throw std::invalid_argument("bad arguments for mode " + mode);
}

}  // namespace

int main(int argc, char** argv) {
  try {
    return run(argc, argv);
  } catch (const std::exception& e) {
    std::printf("error: %s\n", e.what());
    return 1;
  }
}
