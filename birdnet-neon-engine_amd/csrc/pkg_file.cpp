// The .bnpk file: a read-only mapping of the package, checked stage by stage before anything else may look at it,
// plus the metadata index and the tensor / path tables the runtime reads.
//
// Format (python/bnneon/compiler/pkgfmt.py:1-22 documents it; src/rt_pkg.c:30-102 is the reference reader, whose
// acceptance rules and refusal messages this reader keeps so that hosts see the same outcome for the same file):
//   bytes  0..63  header: magic "BNNPKG01", u32 byte-order mark, u16 format version, u16 oldest reader version,
//                 u32 counts {metadata, tensors, paths, reserved}, u64 offsets {metadata, tensors, paths, file size}
//   metadata      records {u16 key bytes, u16 type (0 text, 1 i64, 2 f64, 3 bytes), u32 value bytes, key, value},
//                 each padded to 8 bytes
//   tensor table  96-byte rt_tensor records; blobs 64-byte aligned with >= 64 readable bytes after each
//   path table    72-byte rt_pathdesc records, each naming its 40-byte buffer descriptors and its op records
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string_view>
#include <vector>

#include "rt.h"

namespace {

// the fixed 64-byte header, field by field at its file offsets
struct FileHeader {
  char magic[8];
  uint32_t byte_order;
  uint16_t format_version, min_reader;
  uint32_t n_meta, n_tensors, n_paths, reserved;
  uint64_t meta_at, tensors_at, paths_at, file_bytes;
};
static_assert(sizeof(FileHeader) == 64, "the .bnpk header is 64 bytes");

constexpr uint32_t kByteOrderMark = 0x01020304u;
constexpr uint32_t kMaxMeta = 4096, kMaxTensors = 65536, kMaxPaths = 8, kMaxPathBufs = 4096, kMaxPathOps = 4096;
constexpr uint64_t kBlobSlack = 64;  // readable bytes the file holds after every tensor blob
constexpr uint32_t kNoEmbedding = 0xffffffffu;

// the refusal texts of the reference reader (a host may match on them); %s first is always the file path
constexpr const char *kMsgTooSmall =
    "%s: %lld bytes, smaller than a package header (64); hint: incomplete download or the wrong file";
constexpr const char *kMsgNoMap = "%s: mmap of %zu bytes failed (%s); hint: memory or a filesystem that cannot map files";
constexpr const char *kMsgMagic =
    "%s: not a .bnpk package (magic '%.8s', expected BNNPKG01); hint: the file is not a compiled model package: "
    "compile the model with bnc, or check the download (sha256)";
constexpr const char *kMsgByteOrder = "%s: byte-order mark 0x%08x, expected 0x01020304 (little endian); hint: corrupt file";
constexpr const char *kMsgReader =
    "%s: the package needs reader version %u, this library reads format version %u; hint: update libbnneon_hip, or "
    "recompile the model with the compiler that matches this library";
constexpr const char *kMsgTruncated =
    "%s: package truncated (size %zu, header says %llu); hint: incomplete download or copy; compare the sha256";
constexpr const char *kMsgCounts =
    "%s: corrupt header (%u metadata records, %u tensors, %u paths; limits 4096 / 65536 / 1..8); hint: corrupt file or "
    "not a package";
constexpr const char *kMsgTables =
    "%s: table offsets outside the file (meta %llu, tensors %llu, paths %llu, size %zu); hint: corrupt file";
constexpr const char *kMsgTensor =
    "%s: tensor %u (%.48s) lies outside the file (offset %llu, %llu bytes, file %zu); hint: truncated or corrupt file";
constexpr const char *kMsgPath =
    "%s: path %u (%.24s) has corrupt tables (%u buffers, %u ops, in %u out %u emb %u); hint: corrupt file";

// whether [at, at + len) lies inside a file of `size` bytes (no overflow for any 64-bit inputs)
bool inside(uint64_t at, uint64_t len, uint64_t size) { return at <= size && len <= size - at; }

// a metadata record as found in the file
struct MetaEntry {
  std::string_view key;
  uint16_t type;
  const uint8_t *value;
  uint32_t bytes;
};

}  // namespace

struct rt_pkg {
  const uint8_t *bytes = nullptr;  // the mapping
  size_t size = 0;
  FileHeader hdr{};
  std::vector<rt_tensor> tensors;  // aligned copies of the tables
  std::vector<rt_pathdesc> paths;
  std::vector<MetaEntry> meta;     // records in file order, up to the first one that does not fit

  ~rt_pkg() {
    if (bytes) munmap((void *)bytes, size);
  }
};

namespace {

// Opens and checks a package, one stage after the other; a stage that refuses the file writes its message and
// stops the open.
class Loader {
 public:
  Loader(const char *path, char *err, size_t errlen) : path_(path), err_(err), errlen_(errlen) {}

  rt_pkg *open() {
    pkg_ = new (std::nothrow) rt_pkg;
    if (!pkg_) { say("out of memory"); return nullptr; }
    const bool ok = map() && check_identity() && check_extent() && load_tables() && check_tensor_blobs() &&
                    check_path_tables();
    if (!ok) { delete pkg_; return nullptr; }
    index_meta();
    return pkg_;
  }

 private:
  bool say(const char *fmt, ...) __attribute__((format(printf, 2, 3))) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err_, errlen_, fmt, ap);
    va_end(ap);
    return false;
  }

  bool map() {
    const int fd = ::open(path_, O_RDONLY);
    if (fd < 0) return say("cannot open %s (%s)", path_, strerror(errno));
    struct stat st;
    const bool have_size = fstat(fd, &st) == 0;
    if (!have_size || st.st_size < (off_t)sizeof(FileHeader)) {
      ::close(fd);
      return say(kMsgTooSmall, path_, have_size ? (long long)st.st_size : -1LL);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    const int map_errno = errno;
    ::close(fd);
    if (m == MAP_FAILED) return say(kMsgNoMap, path_, (size_t)st.st_size, strerror(map_errno));
    pkg_->bytes = (const uint8_t *)m;
    pkg_->size = (size_t)st.st_size;
    memcpy(&pkg_->hdr, pkg_->bytes, sizeof(FileHeader));
    return true;
  }

  // what the file is and whether this reader may read it
  bool check_identity() {
    const FileHeader &h = pkg_->hdr;
    if (memcmp(h.magic, "BNNPKG01", 8)) return say(kMsgMagic, path_, h.magic);
    if (h.byte_order != kByteOrderMark) return say(kMsgByteOrder, path_, h.byte_order);
    if (h.min_reader > RT_READER_VERSION) return say(kMsgReader, path_, h.min_reader, RT_READER_VERSION);
    return true;
  }

  // the header's view of the file's size, counts and table positions
  bool check_extent() {
    const FileHeader &h = pkg_->hdr;
    const uint64_t size = pkg_->size;
    if (h.file_bytes != size) return say(kMsgTruncated, path_, pkg_->size, (unsigned long long)h.file_bytes);
    if (h.n_tensors > kMaxTensors || h.n_paths < 1 || h.n_paths > kMaxPaths || h.n_meta > kMaxMeta)
      return say(kMsgCounts, path_, h.n_meta, h.n_tensors, h.n_paths);
    const bool placed = h.meta_at <= size && h.tensors_at <= size && h.paths_at <= size && h.meta_at <= h.tensors_at &&
                        inside(h.tensors_at, (uint64_t)h.n_tensors * sizeof(rt_tensor), size) &&
                        inside(h.paths_at, (uint64_t)h.n_paths * sizeof(rt_pathdesc), size);
    if (!placed)
      return say(kMsgTables, path_, (unsigned long long)h.meta_at, (unsigned long long)h.tensors_at,
                 (unsigned long long)h.paths_at, pkg_->size);
    return true;
  }

  bool load_tables() {
    const FileHeader &h = pkg_->hdr;
    pkg_->tensors.resize(h.n_tensors);
    pkg_->paths.resize(h.n_paths);
    if (h.n_tensors) memcpy(pkg_->tensors.data(), pkg_->bytes + h.tensors_at, sizeof(rt_tensor) * h.n_tensors);
    memcpy(pkg_->paths.data(), pkg_->bytes + h.paths_at, sizeof(rt_pathdesc) * h.n_paths);
    return true;
  }

  // every blob 64-byte aligned, inside the file, and followed by the slack the kernels' read-ahead may touch
  bool check_tensor_blobs() {
    const uint64_t size = pkg_->size;
    for (uint32_t i = 0; i < (uint32_t)pkg_->tensors.size(); i++) {
      const rt_tensor &t = pkg_->tensors[i];
      const bool ok = t.offset % 64 == 0 && inside(t.offset, t.nbytes, size) && t.offset + t.nbytes + kBlobSlack <= size;
      if (!ok)
        return say(kMsgTensor, path_, i, t.name, (unsigned long long)t.offset, (unsigned long long)t.nbytes, pkg_->size);
    }
    return true;
  }

  // each path's buffer and op tables inside the file, 8-byte aligned, and its input / output / embedding buffers
  // among its buffers
  bool check_path_tables() {
    const uint64_t size = pkg_->size;
    for (uint32_t i = 0; i < (uint32_t)pkg_->paths.size(); i++) {
      const rt_pathdesc &d = pkg_->paths[i];
      const bool counts = d.n_buf >= 1 && d.n_buf <= kMaxPathBufs && d.n_ops >= 1 && d.n_ops <= kMaxPathOps;
      const bool placed = d.buf_off % 8 == 0 && d.ops_off % 8 == 0 &&
                          d.buf_off + (uint64_t)d.n_buf * sizeof(rt_bufdesc) <= size && d.ops_off + d.ops_bytes <= size;
      const bool roles = d.in_buf < d.n_buf && d.out_buf < d.n_buf && (d.emb_buf == kNoEmbedding || d.emb_buf < d.n_buf);
      if (!(counts && placed && roles))
        return say(kMsgPath, path_, i, d.name, d.n_buf, d.n_ops, d.in_buf, d.out_buf, d.emb_buf);
    }
    return true;
  }

  // the metadata records in file order; a record that runs past the metadata area ends the index there
  void index_meta() {
    const FileHeader &h = pkg_->hdr;
    const uint8_t *at = pkg_->bytes + h.meta_at, *end = pkg_->bytes + h.tensors_at;
    for (uint32_t i = 0; i < h.n_meta && end - at >= 8; i++) {
      uint16_t key_bytes, type;
      uint32_t value_bytes;
      memcpy(&key_bytes, at, 2);
      memcpy(&type, at + 2, 2);
      memcpy(&value_bytes, at + 4, 4);
      const size_t record = (8 + (size_t)key_bytes + value_bytes + 7) / 8 * 8;
      if ((size_t)(end - at) < record) break;
      pkg_->meta.push_back({std::string_view((const char *)at + 8, key_bytes), type, at + 8 + key_bytes, value_bytes});
      at += record;
    }
  }

  const char *path_;
  char *err_;
  size_t errlen_;
  rt_pkg *pkg_ = nullptr;
};

const MetaEntry *find_meta(const rt_pkg *p, const char *key) {
  const std::string_view k(key);
  for (const MetaEntry &e : p->meta)
    if (e.key == k) return &e;
  return nullptr;
}

}  // namespace

rt_pkg *rt_pkg_open(const char *path, char *err, size_t errlen) { return Loader(path, err, errlen).open(); }

void rt_pkg_close(rt_pkg *p) { delete p; }

const uint8_t *rt_meta_raw(const rt_pkg *p, const char *key, uint16_t *type, uint32_t *bytes) {
  const MetaEntry *e = find_meta(p, key);
  if (!e) return nullptr;
  *type = e->type;
  *bytes = e->bytes;
  return e->value;
}

int rt_meta_str(const rt_pkg *p, const char *key, char *buf, size_t n) {
  const MetaEntry *e = find_meta(p, key);
  if (!e) return -1;
  // numbers answer as decimal text: integers exactly, doubles with 17 significant digits (they read back equal)
  char text[64];
  const char *v = (const char *)e->value;
  size_t len = e->bytes;
  if ((e->type == 1 || e->type == 2) && e->bytes == 8) {
    int64_t i;
    double d;
    memcpy(&i, e->value, 8);
    memcpy(&d, e->value, 8);
    len = (size_t)(e->type == 1 ? snprintf(text, sizeof text, "%lld", (long long)i) : snprintf(text, sizeof text, "%.17g", d));
    v = text;
  }
  if (buf && n) {
    const size_t k = len < n - 1 ? len : n - 1;
    memcpy(buf, v, k);
    buf[k] = 0;
  }
  return (int)len;
}

static bool meta_word(const rt_pkg *p, const char *key, uint16_t type, void *out) {
  const MetaEntry *e = find_meta(p, key);
  if (!e || e->type != type || e->bytes != 8) return false;
  memcpy(out, e->value, 8);
  return true;
}
int rt_meta_i64(const rt_pkg *p, const char *key, int64_t *v) { return meta_word(p, key, 1, v) ? 0 : -1; }
int rt_meta_f64(const rt_pkg *p, const char *key, double *v) { return meta_word(p, key, 2, v) ? 0 : -1; }

int rt_n_paths(const rt_pkg *p) { return (int)p->paths.size(); }
int rt_n_tensors(const rt_pkg *p) { return (int)p->tensors.size(); }
int rt_format_version(const rt_pkg *p) { return p->hdr.format_version; }
const uint8_t *rt_pkg_bytes(const rt_pkg *p) { return p->bytes; }
const rt_pathdesc *rt_path(const rt_pkg *p, int i) {
  return i >= 0 && (size_t)i < p->paths.size() ? &p->paths[(size_t)i] : nullptr;
}
const rt_tensor *rt_tensor_at(const rt_pkg *p, int i, const void **data) {
  if (i < 0 || (size_t)i >= p->tensors.size()) return nullptr;
  const rt_tensor *t = &p->tensors[(size_t)i];
  if (data) *data = p->bytes + t->offset;
  return t;
}
