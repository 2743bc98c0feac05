// directional.hip -- directional (LSH / PQ) path.
#include "directional.hpp"
#include "directional_api.hpp"

#include <stdexcept>

namespace jasper_amd {

LshArtifacts::~LshArtifacts() {
  if (rows) (void)hipFree(rows);
}

PqArtifacts::~PqArtifacts() {
  if (centroids) (void)hipFree(centroids);
  if (codes) (void)hipFree(codes);
}

void check_directional_dim(bool small_dim, int64_t dim) {
  if (small_dim ? dim > 128 : dim <= 128)
    throw std::invalid_argument("dim " + std::to_string(dim) + " does not match the config's dim bucket");
}

static void not_yet(const char* what) {
  throw std::runtime_error(std::string(what) + " is not available in this build yet");
}

std::unique_ptr<Graph> construct_directional(uint32_t, int, uint32_t, bool, const void*, int64_t, int64_t, double,
                                             int64_t, bool, bool, uint64_t, hipStream_t, BuildStats*) {
  not_yet("construct_directional");
  return nullptr;
}
void build_lsh(Graph&, int64_t, uint64_t) { not_yet("build_lsh"); }
void build_pq(Graph&, int64_t, int64_t, uint64_t) { not_yet("build_pq"); }
void directional_search(Graph&, bool, const void*, int64_t, int64_t, int32_t*, float*, int64_t, int64_t, int64_t,
                        bool, hipStream_t) {
  not_yet("directional_search");
}
void save_directional_file(const Graph&, const std::string&) { not_yet("save_directional"); }
std::unique_ptr<Graph> load_directional_file(const std::string&, uint32_t, uint32_t, int, uint32_t, bool, bool, bool,
                                             uint64_t) {
  not_yet("load_directional");
  return nullptr;
}

}  // namespace jasper_amd
