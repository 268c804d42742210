// Serialized executables (include/iree_mi355x_executable_format.h): the
// dispatch library's ELF with its export table in one versioned, checksummed
// container, and a loader that dlopens the ELF from an anonymous file the way
// the reference's DSP runtime dlopens the .so written out of its module
// (RT/dsp/executable.c:92-147).
#include <dlfcn.h>
#include <sys/mman.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/iree_mi355x_executable_format.h"
#include "../../include/iree_mi355x_kernels.h"

namespace ihp {
int fail(int status, const char *fmt, ...);
}

using ihp::fail;

struct iree_mi355x_loaded_executable_t {
  void *handle = nullptr;  // dlopen handle
  int fd = -1;             // the anonymous file holding the ELF
  const iree_mi355x_executable_library_t *library = nullptr;
};

namespace {

constexpr const char kArch[] = "gfx950";

uint64_t fnv1a64(const unsigned char *p, size_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

// This library's own file (the object that holds this function).
std::string own_path() {
  Dl_info info;
  if (!dladdr((const void *)&iree_mi355x_executable_serialize, &info) ||
      !info.dli_fname)
    return std::string();
  return info.dli_fname;
}

bool read_file(const std::string &path, std::vector<unsigned char> *out) {
  FILE *f = fopen(path.c_str(), "rb");
  if (!f)
    return false;
  unsigned char buf[1 << 16];
  size_t n;
  while ((n = fread(buf, 1, sizeof(buf), f)) > 0)
    out->insert(out->end(), buf, buf + n);
  const bool ok = !ferror(f);
  fclose(f);
  return ok;
}

// dlopen an ELF image from memory through an anonymous file. *fd keeps the
// file open for the life of the mapping.
void *open_image(const unsigned char *elf, size_t bytes, int *fd) {
  *fd = memfd_create("iree_mi355x_executable", MFD_CLOEXEC);
  if (*fd < 0)
    return nullptr;
  size_t done = 0;
  while (done < bytes) {
    const ssize_t w = write(*fd, elf + done, bytes - done);
    if (w <= 0) {
      close(*fd);
      *fd = -1;
      return nullptr;
    }
    done += (size_t)w;
  }
  char path[64];
  snprintf(path, sizeof(path), "/proc/self/fd/%d", *fd);
  void *h = dlopen(path, RTLD_NOW | RTLD_LOCAL);
  if (!h) {
    close(*fd);
    *fd = -1;
  }
  return h;
}

const iree_mi355x_executable_library_t *query(void *handle) {
  typedef const iree_mi355x_executable_library_header_t **(*QueryFn)(
      iree_mi355x_executable_library_version_t,
      const iree_mi355x_executable_environment_t *);
  QueryFn q =
      (QueryFn)dlsym(handle, IREE_MI355X_EXECUTABLE_LIBRARY_EXPORT_NAME);
  if (!q)
    return nullptr;
  return (const iree_mi355x_executable_library_t *)q(
      IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST, nullptr);
}

void put_u64(std::vector<unsigned char> *v, uint64_t x) {
  for (int i = 0; i < 8; ++i)
    v->push_back((unsigned char)(x >> (8 * i)));
}

}  // namespace

extern "C" {

size_t iree_mi355x_executable_serialize(const char *library_path, void *out,
                                        size_t capacity) {
  const std::string path = library_path ? library_path : own_path();
  std::vector<unsigned char> elf;
  if (path.empty() || !read_file(path, &elf) || elf.size() < 4 ||
      memcmp(elf.data(), "\x7f" "ELF", 4) != 0) {
    fail(IREE_MI355X_INVALID_ARGUMENT, "serialize: no ELF at '%s'",
         path.c_str());
    return 0;
  }
  // The export table as the library itself reports it (this library's own
  // table directly; another file's from a private copy of it).
  int fd = -1;
  void *h = nullptr;
  const iree_mi355x_executable_library_t *lib;
  if (library_path) {
    h = open_image(elf.data(), elf.size(), &fd);
    lib = h ? query(h) : nullptr;
  } else {
    lib = (const iree_mi355x_executable_library_t *)
        iree_mi355x_executable_library_query(
            IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST, nullptr);
  }
  if (!lib || !lib->header ||
      lib->header->version != IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST) {
    if (h)
      dlclose(h);
    if (fd >= 0)
      close(fd);
    fail(IREE_MI355X_UNSUPPORTED,
         "serialize: '%s' has no library of version 0x%x", path.c_str(),
         IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST);
    return 0;
  }
  std::vector<unsigned char> table;
  const uint32_t count = lib->exports.count;
  for (uint32_t i = 0; i < count; ++i) {
    const iree_mi355x_executable_dispatch_attrs_t a =
        lib->exports.attrs ? lib->exports.attrs[i]
                           : iree_mi355x_executable_dispatch_attrs_t{0, 0, 0};
    put_u64(&table, a.flags);
    put_u64(&table, a.lds_bytes);
    put_u64(&table, a.threads);
  }
  for (uint32_t i = 0; i < count; ++i) {
    const char *name = lib->exports.names[i];
    table.insert(table.end(), name, name + strlen(name) + 1);
  }
  const uint32_t library_version = lib->header->version;
  if (h)
    dlclose(h);
  if (fd >= 0)
    close(fd);
  while (table.size() % 8)
    table.push_back(0);

  iree_mi355x_executable_header_t hdr;
  memset(&hdr, 0, sizeof(hdr));
  memcpy(hdr.magic, IREE_MI355X_EXECUTABLE_MAGIC, 8);
  hdr.format_version = IREE_MI355X_EXECUTABLE_FORMAT_VERSION;
  hdr.library_version = library_version;
  memcpy(hdr.arch, kArch, sizeof(kArch));
  memcpy(hdr.mime, IREE_MI355X_EXECUTABLE_MIME,
         sizeof(IREE_MI355X_EXECUTABLE_MIME));
  hdr.export_count = count;
  hdr.table_offset = sizeof(hdr);
  hdr.table_bytes = table.size();
  hdr.library_offset = hdr.table_offset + hdr.table_bytes;
  hdr.library_bytes = elf.size();
  const size_t total = (size_t)(hdr.library_offset + hdr.library_bytes);
  if (!out || capacity < total)
    return total;
  unsigned char *o = (unsigned char *)out;
  memcpy(o + hdr.table_offset, table.data(), table.size());
  memcpy(o + hdr.library_offset, elf.data(), elf.size());
  hdr.checksum = fnv1a64(o + sizeof(hdr), total - sizeof(hdr));
  memcpy(o, &hdr, sizeof(hdr));
  return total;
}

int iree_mi355x_executable_verify(const void *data, size_t size) {
  const unsigned char *p = (const unsigned char *)data;
  iree_mi355x_executable_header_t h;
  if (!p || size < sizeof(h))
    return fail(IREE_MI355X_INVALID_ARGUMENT, "executable: %zu bytes is "
                "smaller than its header", size);
  memcpy(&h, p, sizeof(h));
  if (memcmp(h.magic, IREE_MI355X_EXECUTABLE_MAGIC, 8) != 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "executable: bad magic");
  if (h.format_version != IREE_MI355X_EXECUTABLE_FORMAT_VERSION ||
      h.library_version != IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST)
    return fail(IREE_MI355X_UNSUPPORTED,
                "executable: format %u / library 0x%x, this runtime reads "
                "format %u / library 0x%x",
                h.format_version, h.library_version,
                IREE_MI355X_EXECUTABLE_FORMAT_VERSION,
                IREE_MI355X_EXECUTABLE_LIBRARY_VERSION_LATEST);
  if (strncmp(h.arch, kArch, sizeof(h.arch)) != 0)
    return fail(IREE_MI355X_UNSUPPORTED, "executable: built for '%.16s', not "
                "%s", h.arch, kArch);
  if (strncmp(h.mime, IREE_MI355X_EXECUTABLE_MIME, sizeof(h.mime)) != 0)
    return fail(IREE_MI355X_UNSUPPORTED, "executable: payload '%.24s'",
                h.mime);
  if (h.table_offset != sizeof(h) || h.table_bytes > size ||
      h.library_offset != h.table_offset + h.table_bytes ||
      h.library_bytes > size || h.library_offset + h.library_bytes != size ||
      h.table_bytes < (uint64_t)h.export_count * 24 || h.library_bytes < 4)
    return fail(IREE_MI355X_INVALID_ARGUMENT,
                "executable: sections do not tile the %zu bytes", size);
  if (fnv1a64(p + sizeof(h), size - sizeof(h)) != h.checksum)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "executable: checksum mismatch");
  if (memcmp(p + h.library_offset, "\x7f" "ELF", 4) != 0)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "executable: payload is not ELF");
  // names: export_count NUL-terminated strings inside the table
  size_t at = (size_t)h.table_offset + (size_t)h.export_count * 24;
  const size_t end = (size_t)(h.table_offset + h.table_bytes);
  for (uint32_t i = 0; i < h.export_count; ++i) {
    const void *nul = memchr(p + at, 0, end - at);
    if (!nul)
      return fail(IREE_MI355X_INVALID_ARGUMENT,
                  "executable: export name %u unterminated", i);
    at = (const unsigned char *)nul - p + 1;
  }
  return IREE_MI355X_OK;
}

int iree_mi355x_executable_load(const void *data, size_t size,
                                iree_mi355x_loaded_executable_t **out) {
  if (!out)
    return fail(IREE_MI355X_INVALID_ARGUMENT, "load: null output");
  *out = nullptr;
  int st = iree_mi355x_executable_verify(data, size);
  if (st != IREE_MI355X_OK)
    return st;
  const unsigned char *p = (const unsigned char *)data;
  iree_mi355x_executable_header_t h;
  memcpy(&h, p, sizeof(h));
  iree_mi355x_loaded_executable_t *e = new iree_mi355x_loaded_executable_t();
  e->handle = open_image(p + h.library_offset, (size_t)h.library_bytes, &e->fd);
  if (!e->handle) {
    const char *why = dlerror();
    delete e;
    return fail(IREE_MI355X_UNSUPPORTED, "load: dlopen failed: %s",
                why ? why : "?");
  }
  e->library = query(e->handle);
  const char *problem = nullptr;
  if (!e->library || !e->library->header)
    problem = "no library at the latest version";
  else if (e->library->header->version != h.library_version)
    problem = "library version differs from the container";
  else if (e->library->imports.count != 0)
    problem = "declares imports (only self-contained libraries load)";
  else if (e->library->exports.count != h.export_count)
    problem = "export count differs from the container";
  if (!problem) {
    // Every export, in order, named as the container says.
    const char *name = (const char *)p + h.table_offset + h.export_count * 24;
    for (uint32_t i = 0; i < h.export_count && !problem; ++i) {
      if (strcmp(name, e->library->exports.names[i]) != 0)
        problem = "export names differ from the container";
      name += strlen(name) + 1;
    }
  }
  if (problem) {
    iree_mi355x_loaded_executable_release(e);
    return fail(IREE_MI355X_UNSUPPORTED, "load: %s", problem);
  }
  *out = e;
  return IREE_MI355X_OK;
}

const iree_mi355x_executable_library_t *iree_mi355x_loaded_executable_library(
    const iree_mi355x_loaded_executable_t *executable) {
  return executable ? executable->library : nullptr;
}

void iree_mi355x_loaded_executable_release(
    iree_mi355x_loaded_executable_t *executable) {
  if (!executable)
    return;
  if (executable->handle)
    dlclose(executable->handle);
  if (executable->fd >= 0)
    close(executable->fd);
  delete executable;
}

}  // extern "C"
