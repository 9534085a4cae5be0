// checkpoint.hip -- reader of the reference's weight files, so the HIP MoE
// and block engines run on trained weights.
//
// Format (crates/prichs-model/src/model.rs:1648-1670 writes it, 1673-1736
// reads it), little endian:
//   "PRICHS02" | step u64 | loss f32 | count u64 |
//   count x ( len u64 | len x f32 )
// in the order of Model::get_parameter_tensors (model.rs:312-338): wte,
// final_norm, then per block input_norm, q_proj, k_proj, v_proj, out_proj,
// post_attn_norm, router, the shared expert's gate/up/down and every routed
// expert's gate/up/down, so block l starts at 2 + l * (10 + 3E)
// (model.rs:557-562, 1083-1087).  The legacy "PRICHS_W" files hold only the
// embedding table and optionally the final norm, sized by the model config
// (model.rs:1707-1729); none of that is on the MoE path, so they open with no
// indexed parameters.
//
// Opening indexes the parameters (length and file offset of each payload)
// without reading payloads; each parameter is then read with one pread into
// the caller's buffer.  Every length is checked against the file size, so a
// truncated or corrupt file fails at open instead of mid-upload.
#include <cerrno>
#include <cstring>
#include <string>
#include <vector>

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include "common.hpp"

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__,
              "the file format is little endian and is read in place");

struct prichs_checkpoint {
  int fd = -1;
  int format = 0;  // 2: PRICHS02, 1: legacy PRICHS_W
  uint64_t step = 0;
  float loss = 0.f;
  uint64_t size = 0;
  std::vector<uint64_t> len;  // elements of each parameter
  std::vector<uint64_t> off;  // byte offset of each payload
};

namespace prichs {
namespace {

// pread of exactly n bytes (retries short reads and EINTR).
bool read_at(int fd, uint64_t off, void *dst, size_t n) {
  char *p = static_cast<char *>(dst);
  while (n > 0) {
    const ssize_t r = ::pread(fd, p, n, (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    p += r;
    off += (uint64_t)r;
    n -= (size_t)r;
  }
  return true;
}

}  // namespace

int checkpoint_read_vec(const prichs_checkpoint *ck, size_t index, size_t want,
                        std::vector<float> &out, const char *what, size_t layer) {
  if (index >= ck->len.size())
    return fail(PRICHS_ERR_INVALID_ARGUMENT,
                "checkpoint: %s of block %zu is parameter %zu, but the file has %zu", what,
                layer, index, ck->len.size());
  if (ck->len[index] != (uint64_t)want)
    return fail(PRICHS_ERR_INVALID_ARGUMENT,
                "checkpoint: %s of block %zu (parameter %zu) has %llu elements, the engine "
                "expects %zu",
                what, layer, index, (unsigned long long)ck->len[index], want);
  out.resize(want);
  if (want && !read_at(ck->fd, ck->off[index], out.data(), 4 * want))
    return fail(PRICHS_ERR_INVALID_ARGUMENT, "checkpoint: reading %s of block %zu failed: %s",
                what, layer, std::strerror(errno));
  return PRICHS_OK;
}

int checkpoint_moe_weights(const prichs_checkpoint *ck, size_t layer, size_t d, size_t f,
                           size_t E, CheckpointMoe &w) {
  static const char *kNames[3] = {"gate_proj", "up_proj", "down_proj"};
  const size_t G = E + 1;
  w.gate.assign(G, {});
  w.up.assign(G, {});
  w.down.assign(G, {});
  int rc = checkpoint_read_vec(ck, prichs_checkpoint_block_param(layer, E, PRICHS_CKPT_ROUTER),
                               d * E, w.router, "moe.router", layer);
  // Shared expert (slots 7..9), then routed experts 0..E-1 (slots 10 + 3e ..).
  for (size_t g = 0; g < G && rc == PRICHS_OK; ++g) {
    const size_t first = g == 0 ? PRICHS_CKPT_SHARED_GATE : PRICHS_CKPT_EXPERT0 + 3 * (g - 1);
    std::vector<float> *dst[3] = {&w.gate[g], &w.up[g], &w.down[g]};
    const size_t want[3] = {d * f, d * f, f * d};
    for (int p = 0; p < 3 && rc == PRICHS_OK; ++p) {
      std::string what = g == 0 ? std::string("moe.shared_expert.") + kNames[p]
                                : "moe.experts[" + std::to_string(g - 1) + "]." + kNames[p];
      rc = checkpoint_read_vec(ck, prichs_checkpoint_block_param(layer, E, first + p), want[p],
                               *dst[p], what.c_str(), layer);
    }
  }
  if (rc) return rc;
  w.pg.resize(G);
  w.pu.resize(G);
  w.pd.resize(G);
  for (size_t g = 0; g < G; ++g) {
    w.pg[g] = w.gate[g].data();
    w.pu[g] = w.up[g].data();
    w.pd[g] = w.down[g].data();
  }
  return PRICHS_OK;
}

}  // namespace prichs

using namespace prichs;

extern "C" int prichs_checkpoint_open(const char *path, prichs_checkpoint **out) {
  PRICHS_REQUIRE(out != nullptr && path != nullptr, "checkpoint_open: null pointer argument");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0)
    return fail(PRICHS_ERR_INVALID_ARGUMENT, "checkpoint_open: cannot open %s: %s", path,
                std::strerror(errno));
  prichs_checkpoint *ck = new (std::nothrow) prichs_checkpoint();
  if (!ck) {
    ::close(fd);
    return fail(PRICHS_ERR_CAPACITY, "checkpoint_open: out of host memory");
  }
  ck->fd = fd;
  struct stat st;
  int rc = PRICHS_OK;
  char magic[8];
  if (::fstat(fd, &st) != 0) {
    rc = fail(PRICHS_ERR_INVALID_ARGUMENT, "checkpoint_open: cannot stat %s", path);
  } else {
    ck->size = (uint64_t)st.st_size;
    // Header common to both formats: magic, step u64, loss f32 (model.rs:1677-1688).
    if (ck->size < 20 || !read_at(fd, 0, magic, 8) || !read_at(fd, 8, &ck->step, 8) ||
        !read_at(fd, 16, &ck->loss, 4))
      rc = fail(PRICHS_ERR_INVALID_ARGUMENT, "checkpoint_open: %s: truncated header", path);
  }
  if (rc == PRICHS_OK && std::memcmp(magic, "PRICHS02", 8) == 0) {
    ck->format = 2;
    uint64_t n = 0;
    if (ck->size < 28 || !read_at(fd, 20, &n, 8)) {
      rc = fail(PRICHS_ERR_INVALID_ARGUMENT, "checkpoint_open: %s: truncated header", path);
    } else if (n > (ck->size - 28) / 8) {
      // Every parameter needs at least its 8-byte length field.
      rc = fail(PRICHS_ERR_INVALID_ARGUMENT,
                "checkpoint_open: %s: %llu parameters cannot fit in %llu bytes", path,
                (unsigned long long)n, (unsigned long long)ck->size);
    } else {
      ck->len.reserve(n);
      ck->off.reserve(n);
      uint64_t pos = 28;
      for (uint64_t i = 0; i < n && rc == PRICHS_OK; ++i) {
        uint64_t len = 0;
        if (ck->size - pos < 8 || !read_at(fd, pos, &len, 8)) {
          rc = fail(PRICHS_ERR_INVALID_ARGUMENT,
                    "checkpoint_open: %s: truncated before the length of parameter %llu", path,
                    (unsigned long long)i);
          break;
        }
        const uint64_t payload = pos + 8;
        if (len > (ck->size - payload) / 4) {
          rc = fail(PRICHS_ERR_INVALID_ARGUMENT,
                    "checkpoint_open: %s: parameter %llu claims %llu floats past the end of "
                    "the file",
                    path, (unsigned long long)i, (unsigned long long)len);
          break;
        }
        ck->len.push_back(len);
        ck->off.push_back(payload);
        pos = payload + 4 * len;
      }
    }
  } else if (rc == PRICHS_OK && std::memcmp(magic, "PRICHS_W", 8) == 0) {
    ck->format = 1;  // embedding / final norm only: nothing indexed
  } else if (rc == PRICHS_OK) {
    rc = fail(PRICHS_ERR_INVALID_ARGUMENT, "checkpoint_open: %s: invalid magic", path);
  }
  if (rc != PRICHS_OK) {
    prichs_checkpoint_close(ck);
    return rc;
  }
  *out = ck;
  return PRICHS_OK;
}

extern "C" int prichs_checkpoint_close(prichs_checkpoint *ck) {
  if (!ck) return PRICHS_OK;
  if (ck->fd >= 0) ::close(ck->fd);
  delete ck;
  return PRICHS_OK;
}

extern "C" int prichs_checkpoint_info(const prichs_checkpoint *ck, uint64_t *step, float *loss,
                                      size_t *n_params, int *format) {
  PRICHS_REQUIRE(ck != nullptr, "checkpoint_info: null checkpoint");
  if (step) *step = ck->step;
  if (loss) *loss = ck->loss;
  if (n_params) *n_params = ck->len.size();
  if (format) *format = ck->format;
  return PRICHS_OK;
}

extern "C" int prichs_checkpoint_param_len(const prichs_checkpoint *ck, size_t index,
                                           size_t *len) {
  PRICHS_REQUIRE(ck != nullptr && len != nullptr, "checkpoint_param_len: null pointer argument");
  PRICHS_REQUIRE(index < ck->len.size(), "checkpoint_param_len: index %zu >= %zu parameters",
                 index, ck->len.size());
  *len = (size_t)ck->len[index];
  return PRICHS_OK;
}

extern "C" int prichs_checkpoint_read(const prichs_checkpoint *ck, size_t index, float *dst,
                                      size_t len) {
  PRICHS_REQUIRE(ck != nullptr, "checkpoint_read: null checkpoint");
  PRICHS_REQUIRE(index < ck->len.size(), "checkpoint_read: index %zu >= %zu parameters", index,
                 ck->len.size());
  PRICHS_REQUIRE(len == ck->len[index],
                 "checkpoint_read: parameter %zu has %llu elements, not %zu", index,
                 (unsigned long long)ck->len[index], len);
  if (len == 0) return PRICHS_OK;
  PRICHS_REQUIRE(dst != nullptr, "checkpoint_read: null destination");
  if (!read_at(ck->fd, ck->off[index], dst, 4 * len))
    return fail(PRICHS_ERR_INVALID_ARGUMENT, "checkpoint_read: reading parameter %zu failed: %s",
                index, std::strerror(errno));
  return PRICHS_OK;
}

extern "C" size_t prichs_checkpoint_block_param(size_t layer, size_t E, size_t slot) {
  const size_t per_block = 10 + 3 * E;
  if (slot >= per_block) return (size_t)-1;
  return 2 + layer * per_block + slot;
}
