// A C++ program on the C++ LOAD surface (include/foundry/CUDAGraph.h), as a
// caller of the reference's include/CUDAGraph.h would write it:
//
//   cudagraph_caller CODE_OBJECT_DIR SAVED_BASE SIZE WEIGHTS ORDER PATH...
//
// registers the code objects, sets the allocation region at SAVED_BASE,
// allocates WEIGHTS bytes in it (the model's allocations before the graphs),
// loads the graphs with start_graph_builds + finish_graph_loads, then for
// each graph index of ORDER (comma-separated) zeroes the output buffer,
// replays that graph and prints what it wrote.  One JSON object per line; the
// test that runs it checks the values.
#include <foundry/CUDAGraph.h>

#include <ATen/ATen.h>
#include <hip/hip_runtime_api.h>

#include <ATen/CPUGeneratorImpl.h>
#include <unistd.h>

#include <chrono>
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <future>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

constexpr int64_t kBufBytes = 16384;  // the graphs' buffer; the output tensor is its first 16 words

std::vector<int> parse_order(const std::string& s) {
  std::vector<int> out;
  std::stringstream ss(s);
  std::string item;
  while (std::getline(ss, item, ',')) out.push_back(std::stoi(item));
  return out;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 7) {
    std::fprintf(stderr, "usage: %s CODE_OBJECT_DIR SAVED_BASE SIZE WEIGHTS ORDER PATH...\n", argv[0]);
    return 2;
  }
  try {
    const std::string co_dir = argv[1];
    const uint64_t saved_base = std::strtoull(argv[2], nullptr, 0);
    const uint64_t size = std::strtoull(argv[3], nullptr, 0);
    const uint64_t weights = std::strtoull(argv[4], nullptr, 0);
    const std::vector<int> order = parse_order(argv[5]);
    std::vector<std::string> paths(argv + 6, argv + argc);

    std::printf("{\"code_objects\": %d}\n", foundry::load_cuda_modules_and_libraries(co_dir));
    foundry::preallocate_cublas_workspaces();
    foundry::set_allocation_region(saved_base, size);
    const uint64_t w = foundry::region_alloc(weights);
    std::printf("{\"weights\": %" PRIu64 "}\n", w);

    // A corrupt archive: start returns, the worker's error surfaces in the
    // finish calls (every one of them).
    {
      const std::string bad = "/tmp/cudagraph_caller_bad_" + std::to_string((long)getpid());
      if (FILE* f = std::fopen((bad + ".cugraph").c_str(), "wb")) {
        std::fputs("CUGRAPH", f);
        std::fclose(f);
      }
      if (FILE* f = std::fopen((bad + ".json").c_str(), "wb")) {
        std::fputs("{not json", f);
        std::fclose(f);
      }
      auto broken = foundry::CUDAGraph::start_graph_builds({bad + ".json"});
      int raised = 0;
      for (int k = 0; k < 2; ++k) {
        try {
          foundry::CUDAGraph::finish_graph_loads(broken);
        } catch (const c10::Error&) {
          ++raised;
        }
      }
      try {
        foundry::CUDAGraph::finish_one_graph_load(broken, 0);
      } catch (const c10::Error&) {
        ++raised;
      }
      std::printf("{\"corrupt_raised_in_finish\": %d}\n", raised);
      std::remove((bad + ".cugraph").c_str());
      std::remove((bad + ".json").c_str());
    }

    auto pending = foundry::CUDAGraph::start_graph_builds(paths);
    const bool ready_at_return =
        pending->build_complete_.wait_for(std::chrono::seconds(0)) == std::future_status::ready;
    std::printf("{\"ready_at_return\": %d}\n", ready_at_return ? 1 : 0);

    bool out_of_range = false;
    try {
      foundry::CUDAGraph::finish_one_graph_load(pending, paths.size());
    } catch (const std::out_of_range&) {
      out_of_range = true;
    }
    std::printf("{\"out_of_range_throws\": %d}\n", out_of_range ? 1 : 0);

    std::vector<foundry::GraphLoadResult> results = foundry::CUDAGraph::finish_graph_loads(pending);
    std::printf("{\"used_manifest\": %d, \"template_of\": [", pending->used_manifest ? 1 : 0);
    for (size_t i = 0; i < pending->template_of.size(); ++i)
      std::printf("%s%u", i ? ", " : "", pending->template_of[i]);
    std::printf("]}\n");

    // Typed generator state (include/CUDAGraph.h:59-76 of the reference):
    // graph 0 reads state 77's words; two replays write seed and offset and
    // advance the offset by the increment rounded up to 4 each time.
    auto& reg = foundry::global_generator_state_registry();
    c10::intrusive_ptr<at::CUDAGeneratorState> st = reg.get_state_from_id(77, 1234);
    const bool same_state = reg.get_state_from_id(77, 999).get() == st.get();
    results[0].graph->register_generator_state(st, 5);
    bool generator_refused = false;
    try {
      results[0].graph->register_generator_state(at::detail::getDefaultCPUGenerator());
    } catch (const c10::Error&) {
      generator_refused = true;
    }
    std::printf("{\"state_id\": %" PRIu64 ", \"same_state\": %d, \"seed_ptr\": %" PRIu64
                ", \"offset_ptr\": %" PRIu64 ", \"torch_generator_refused\": %d}\n",
                reg.query_state_id(st.get()), same_state ? 1 : 0, (uint64_t)(uintptr_t)st->seed_extragraph_.data_ptr(),
                (uint64_t)(uintptr_t)st->offset_extragraph_.data_ptr(), generator_refused ? 1 : 0);
    std::vector<at::Tensor> outs;
    for (auto& r : results) {
      if (r.output_type != foundry::OutputTensorType::Single) throw std::runtime_error("expected one output tensor");
      outs.push_back(std::get<at::Tensor>(r.outputs));
    }
    const at::Tensor& o0 = outs[0];
    std::printf("{\"out_ptr\": %" PRIu64 ", \"numel\": %" PRId64 ", \"dtype_long\": %d, \"same_exec\": %d}\n",
                (uint64_t)(uintptr_t)o0.data_ptr(), o0.numel(), o0.scalar_type() == at::kLong ? 1 : 0,
                results.size() > 1 && results[0].graph->raw_cuda_graph_exec() == results[1].graph->raw_cuda_graph_exec()
                    ? 1
                    : 0);
    bool keep_graph_refused = false;
    try {
      results[0].graph->raw_cuda_graph();
    } catch (const c10::Error&) {
      keep_graph_refused = true;
    }
    std::printf("{\"raw_graph_needs_keep_graph\": %d}\n", keep_graph_refused ? 1 : 0);

    at::Tensor whole = at::from_blob(o0.data_ptr(), {kBufBytes / 8}, o0.options());
    for (int g : order) {
      whole.zero_();
      results.at((size_t)g).graph->replay();
      if (hipDeviceSynchronize() != hipSuccess) throw std::runtime_error("replay failed");
      at::Tensor host = whole.cpu();
      const uint64_t* v = reinterpret_cast<const uint64_t*>(host.data_ptr());
      std::printf("{\"graph\": %d, \"words\": [", g);
      for (int64_t i = 0; i < kBufBytes / 8; ++i) std::printf("%s\"%" PRIu64 "\"", i ? ", " : "", v[i]);
      std::printf("]}\n");
    }
    {
      at::Tensor seed = at::Tensor(st->seed_extragraph_).cpu(), off = at::Tensor(st->offset_extragraph_).cpu();
      std::printf("{\"rng_seed\": %" PRId64 ", \"rng_offset\": %" PRId64 ", \"philox_offset\": %" PRIu64 "}\n",
                  seed.item<int64_t>(), off.item<int64_t>(), st->philox_offset_per_thread_);
    }
    results[0].graph->reset();
    std::printf("{\"words_released\": %d}\n", st->seed_extragraph_.defined() ? 0 : 1);
    results.clear();
    outs.clear();
    whole = at::Tensor();
    pending.reset();
    std::printf("{\"done\": 1}\n");
    std::fflush(stdout);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "cudagraph_caller: %s\n", e.what());
    return 1;
  }
  return 0;
}
