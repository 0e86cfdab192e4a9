// Host-side sparse matrix formats of the benchmark harness: the Matrix Market
// coordinate reader, the SWCSR001 / SWCOO001 / SWBSR001 little-endian binary
// files, and COO -> padded BSR conversion.  Behaviour (accepted headers,
// entry checks, ordering, coalescing, limits, messages) follows
// benchmark/benchmark_utils.py:56-379 (reader, writers, convert_to_bsr) and
// benchmark/SparseBenchmarkUtils.cpp:37-185 (binary readers).  Readers also
// check the index structure, so a loaded matrix is safe to hand to the GPU
// kernels.
#include "sw_internal.h"

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <new>
#include <numeric>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

constexpr char kCsrMagic[8] = {'S', 'W', 'C', 'S', 'R', '0', '0', '1'};
constexpr char kCooMagic[8] = {'S', 'W', 'C', 'O', 'O', '0', '0', '1'};
constexpr char kBsrMagic[8] = {'S', 'W', 'B', 'S', 'R', '0', '0', '1'};
constexpr int64_t kI32Max = std::numeric_limits<int32_t>::max();
constexpr uint64_t kI64Max = (uint64_t)std::numeric_limits<int64_t>::max();

template <typename T> T *dup_array(const std::vector<T> &v) {
  T *p = static_cast<T *>(std::malloc(std::max<size_t>(v.size(), 1) * sizeof(T)));
  if (p && !v.empty())
    std::memcpy(p, v.data(), v.size() * sizeof(T));
  return p;
}

struct File {
  std::FILE *f = nullptr;
  ~File() {
    if (f)
      std::fclose(f);
  }
};

// ---- Matrix Market ---------------------------------------------------------

std::vector<std::string> split_ws(const std::string &s) {
  std::vector<std::string> out;
  size_t i = 0;
  while (i < s.size()) {
    while (i < s.size() && std::isspace((unsigned char)s[i]))
      ++i;
    size_t j = i;
    while (j < s.size() && !std::isspace((unsigned char)s[j]))
      ++j;
    if (j > i)
      out.emplace_back(s.substr(i, j - i));
    i = j;
  }
  return out;
}

bool read_line(std::FILE *f, std::string &line) {
  line.clear();
  int c;
  bool any = false;
  while ((c = std::fgetc(f)) != EOF) {
    any = true;
    if (c == '\n')
      return true;
    line.push_back((char)c);
  }
  return any;
}

// Base-10 integer token with an optional sign (Python int() on a token).
bool parse_int(const std::string &t, int64_t *v) {
  if (t.empty())
    return false;
  errno = 0;
  char *end = nullptr;
  long long x = std::strtoll(t.c_str(), &end, 10);
  if (errno || end != t.c_str() + t.size())
    return false;
  *v = x;
  return true;
}

// Decimal floating-point token (Python float(): decimal, inf, nan; no hex).
bool parse_real(const std::string &t, double *v) {
  if (t.empty() || t.find_first_of("xX") != std::string::npos)
    return false;
  errno = 0;
  char *end = nullptr;
  double x = std::strtod(t.c_str(), &end);
  if (end != t.c_str() + t.size())
    return false;
  *v = x; // overflow gives +-inf, rejected by the finiteness check
  return true;
}

// An integer-field value: sign and digits, converted with rounding as
// float(int(token)) does.
bool parse_integer_value(const std::string &t, double *v) {
  size_t i = (t[0] == '+' || t[0] == '-') ? 1 : 0;
  if (i == t.size())
    return false;
  for (size_t j = i; j < t.size(); ++j)
    if (t[j] < '0' || t[j] > '9')
      return false;
  *v = std::strtod(t.c_str(), nullptr);
  return true;
}

struct Entry {
  int32_t row, col;
  double val;
};

void fill_stats(sw_host_matrix *m) {
  std::vector<int64_t> len(m->rows, 0);
  for (int64_t p = 0; p < m->nnz; ++p)
    ++len[m->row_indices[p]];
  int64_t mn = m->rows ? INT64_MAX : 0, mx = 0;
  for (int64_t l : len) {
    mn = std::min(mn, l);
    mx = std::max(mx, l);
  }
  m->min_row_nnz = mn;
  m->max_row_nnz = mx;
  m->mean_row_nnz = m->rows ? (double)m->nnz / (double)m->rows : 0.0;
}

// CSR arrays + row indices from entries sorted by (row, column).
int finish_matrix(std::vector<Entry> &e, int64_t rows, int64_t cols,
                  sw_host_matrix **out) {
  std::stable_sort(e.begin(), e.end(), [](const Entry &a, const Entry &b) {
    return a.row != b.row ? a.row < b.row : a.col < b.col;
  });
  if ((int64_t)e.size() > kI32Max)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "%zu entries exceed the i32 index range", e.size());
  auto *m = static_cast<sw_host_matrix *>(std::calloc(1, sizeof(sw_host_matrix)));
  if (!m)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  m->rows = rows;
  m->columns = cols;
  m->nnz = (int64_t)e.size();
  std::vector<int32_t> ro(rows + 1, 0), ri(e.size()), ci(e.size());
  std::vector<double> val(e.size());
  for (size_t i = 0; i < e.size(); ++i) {
    ++ro[e[i].row + 1];
    ri[i] = e[i].row;
    ci[i] = e[i].col;
    val[i] = e[i].val;
  }
  for (int64_t r = 0; r < rows; ++r)
    ro[r + 1] += ro[r];
  m->row_offsets = dup_array(ro);
  m->row_indices = dup_array(ri);
  m->column_indices = dup_array(ci);
  m->values = dup_array(val);
  m->has_row_offsets = 1;
  if (!m->row_offsets || !m->row_indices || !m->column_indices || !m->values) {
    sw_host_matrix_free(m);
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  }
  fill_stats(m);
  *out = m;
  return SW_OK;
}

// ---- binary files ----------------------------------------------------------

bool write_all(std::FILE *f, const void *p, size_t bytes) {
  return bytes == 0 || std::fwrite(p, 1, bytes, f) == bytes;
}

bool write_u64s(std::FILE *f, std::initializer_list<uint64_t> v) {
  for (uint64_t x : v) // little-endian host (x86-64 / gfx950 hosts)
    if (!write_all(f, &x, 8))
      return false;
  return true;
}

template <typename T>
bool write_as(std::FILE *f, const T *p, int64_t n) {
  return write_all(f, p, (size_t)n * sizeof(T));
}

bool write_f32(std::FILE *f, const double *p, int64_t n, bool *overflow) {
  std::vector<float> buf;
  const int64_t chunk = 1 << 20;
  for (int64_t i = 0; i < n; i += chunk) {
    const int64_t m = std::min(chunk, n - i);
    buf.resize(m);
    for (int64_t j = 0; j < m; ++j) {
      buf[j] = (float)p[i + j];
      if (std::isinf(buf[j]) && !std::isinf(p[i + j]))
        *overflow = true;
    }
    if (*overflow || !write_all(f, buf.data(), m * sizeof(float)))
      return false;
  }
  return true;
}

int read_header(std::FILE *f, const char *magic, const char *format,
                uint64_t *dims, int count) {
  char m[8];
  if (std::fread(m, 1, 8, f) != 8 || std::memcmp(m, magic, 8) != 0)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "invalid %s binary header",
                    format);
  static const char *names[] = {"row count", "column count", "NNZ count",
                                "block size", "original row count",
                                "original column count", "original NNZ count"};
  for (int i = 0; i < count; ++i)
    if (std::fread(&dims[i], 8, 1, f) != 1)
      return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not read %s", names[i]);
  for (int i = 0; i < 3; ++i)
    if (dims[i] > kI64Max)
      return sw::fail(SW_ERR_INVALID_SHAPE,
                      "%s dimensions exceed the runner limits", format);
  return SW_OK;
}

template <typename T>
int read_array(std::FILE *f, uint64_t n, const char *name, T **out) {
  if (n > kI64Max / sizeof(T))
    return sw::fail(SW_ERR_INVALID_SHAPE, "%s exceeds the runner limits",
                    name);
  T *p = static_cast<T *>(std::malloc(std::max<uint64_t>(n, 1) * sizeof(T)));
  if (!p)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory for %s", name);
  if (n && std::fread(p, sizeof(T), n, f) != n) {
    std::free(p);
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not read %s", name);
  }
  *out = p;
  return SW_OK;
}

int read_f32_as_f64(std::FILE *f, uint64_t n, const char *name, double **out) {
  float *tmp = nullptr;
  int rc = read_array(f, n, name, &tmp);
  if (rc)
    return rc;
  double *p = static_cast<double *>(std::malloc(std::max<uint64_t>(n, 1) * 8));
  if (!p) {
    std::free(tmp);
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory for %s", name);
  }
  for (uint64_t i = 0; i < n; ++i)
    p[i] = tmp[i];
  std::free(tmp);
  *out = p;
  return SW_OK;
}

// Index structure of a CSR: offsets from 0 to nnz, non-decreasing, columns
// in range.
int check_csr_structure(const int32_t *ro, int64_t rows, const int32_t *col,
                        int64_t nnz, int64_t cols, const char *what) {
  if (ro[0] != 0 || ro[rows] != nnz)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "%s row offsets must run from 0 to %lld", what,
                    (long long)nnz);
  for (int64_t r = 0; r < rows; ++r)
    if (ro[r + 1] < ro[r])
      return sw::fail(SW_ERR_INVALID_SHAPE,
                      "%s row offsets decrease at row %lld", what,
                      (long long)r);
  for (int64_t p = 0; p < nnz; ++p)
    if (col[p] < 0 || col[p] >= cols)
      return sw::fail(SW_ERR_INVALID_SHAPE,
                      "%s column index %d at position %lld is out of bounds",
                      what, col[p], (long long)p);
  return SW_OK;
}

// Host allocations of the format code report failure instead of throwing
// through the C ABI.
template <typename F> int guarded(F &&f) {
  try {
    return f();
  } catch (const std::bad_alloc &) {
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  } catch (const std::length_error &) {
    return sw::fail(SW_ERR_INVALID_SHAPE, "matrix too large for host memory");
  }
}

} // namespace

extern "C" {

void sw_host_matrix_free(sw_host_matrix *m) {
  if (!m)
    return;
  std::free(m->row_offsets);
  std::free(m->row_indices);
  std::free(m->column_indices);
  std::free(m->values);
  std::free(m);
}

void sw_host_bsr_free(sw_host_bsr *b) {
  if (!b)
    return;
  std::free(b->block_row_offsets);
  std::free(b->block_column_indices);
  std::free(b->block_values);
  std::free(b->input_row_indices);
  std::free(b->input_column_indices);
  std::free(b->input_values);
  std::free(b);
}

static int matrix_market_read_impl(const char *path, sw_host_matrix **out) {
  sw::clear_error();
  if (!path || !out)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null path or output");
  *out = nullptr;
  File file;
  file.f = std::fopen(path, "rb");
  if (!file.f)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not open %s", path);
  std::string line;
  read_line(file.f, line);
  auto header = split_ws(line);
  if (header.size() != 5 || header[0] != "%%MatrixMarket" ||
      header[1] != "matrix" || header[2] != "coordinate")
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    "%s: expected a Matrix Market coordinate matrix", path);
  std::string field = header[3], symmetry = header[4];
  for (auto &c : field)
    c = (char)std::tolower((unsigned char)c);
  for (auto &c : symmetry)
    c = (char)std::tolower((unsigned char)c);
  if (field != "real" && field != "integer" && field != "pattern")
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    "%s: unsupported Matrix Market field '%s'", path,
                    field.c_str());
  if (symmetry != "general" && symmetry != "symmetric")
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    "%s: unsupported Matrix Market symmetry '%s'", path,
                    symmetry.c_str());
  int64_t line_no = 1;
  bool have_size = false;
  std::vector<std::string> size;
  while (read_line(file.f, line)) {
    ++line_no;
    auto t = split_ws(line);
    if (t.empty() || t[0][0] == '%')
      continue;
    size = t;
    have_size = true;
    break;
  }
  if (!have_size)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "%s: missing matrix dimensions",
                    path);
  int64_t rows, cols, stored;
  if (size.size() != 3 || !parse_int(size[0], &rows) ||
      !parse_int(size[1], &cols) || !parse_int(size[2], &stored))
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "%s: invalid matrix dimensions",
                    path);
  if (rows <= 0 || cols <= 0 || stored < 0)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "%s: matrix dimensions must be nonnegative", path);
  const bool sym = symmetry == "symmetric";
  if (sym && rows != cols)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "%s: a symmetric matrix must be square", path);
  if (rows > kI32Max || cols > kI32Max)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "%s: dimensions exceed the i32 index range", path);
  const bool pattern = field == "pattern", integer = field == "integer";
  const size_t want = pattern ? 2 : 3;
  std::vector<Entry> entries;
  entries.reserve((size_t)std::min<int64_t>(stored, 1 << 26) * (sym ? 2 : 1));
  int64_t read_entries = 0;
  while (read_line(file.f, line)) {
    ++line_no;
    auto t = split_ws(line);
    if (t.empty() || t[0][0] == '%')
      continue;
    if (t.size() != want)
      return sw::fail(SW_ERR_INVALID_ARGUMENT, "%s:%lld: expected %zu fields",
                      path, (long long)line_no, want);
    int64_t r, c;
    double v = 1.0;
    if (!parse_int(t[0], &r) || !parse_int(t[1], &c) ||
        (integer && !parse_integer_value(t[2], &v)) ||
        (!pattern && !integer && !parse_real(t[2], &v)))
      return sw::fail(SW_ERR_INVALID_ARGUMENT,
                      "%s:%lld: invalid matrix entry", path,
                      (long long)line_no);
    --r;
    --c;
    if (r < 0 || r >= rows || c < 0 || c >= cols)
      return sw::fail(SW_ERR_INVALID_SHAPE,
                      "%s:%lld: matrix index is out of bounds", path,
                      (long long)line_no);
    if (!std::isfinite(v))
      return sw::fail(SW_ERR_INVALID_ARGUMENT,
                      "%s:%lld: matrix value must be finite", path,
                      (long long)line_no);
    if (std::isinf((float)v))
      return sw::fail(SW_ERR_INVALID_ARGUMENT,
                      "%s:%lld: matrix value must fit in f32", path,
                      (long long)line_no);
    entries.push_back({(int32_t)r, (int32_t)c, v});
    ++read_entries;
    if (sym && r != c)
      entries.push_back({(int32_t)c, (int32_t)r, v});
  }
  if (read_entries != stored)
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    "%s: header declares %lld entries, but the file contains "
                    "%lld",
                    path, (long long)stored, (long long)read_entries);
  int rc = finish_matrix(entries, rows, cols, out);
  if (rc)
    return rc;
  std::snprintf((*out)->field, sizeof((*out)->field), "%s", field.c_str());
  std::snprintf((*out)->symmetry, sizeof((*out)->symmetry), "%s",
                symmetry.c_str());
  return SW_OK;
}

static int csr_binary_write_impl(const char *path, const sw_host_matrix *m) {
  sw::clear_error();
  if (!path || !m)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null path or matrix");
  if (m->rows > kI32Max || m->nnz > kI32Max)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "matrix rows and NNZ must fit in the i32 CSR type");
  File file;
  file.f = std::fopen(path, "wb");
  if (!file.f)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not open %s", path);
  bool overflow = false;
  if (!write_all(file.f, kCsrMagic, 8) ||
      !write_u64s(file.f, {(uint64_t)m->rows, (uint64_t)m->columns,
                           (uint64_t)m->nnz}) ||
      !write_as(file.f, m->row_offsets, m->rows + 1) ||
      !write_as(file.f, m->column_indices, m->nnz) ||
      !write_f32(file.f, m->values, m->nnz, &overflow))
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    overflow ? "matrix values must fit in f32"
                             : "could not write %s",
                    path);
  return SW_OK;
}

static int coo_binary_write_impl(const char *path, const sw_host_matrix *m) {
  sw::clear_error();
  if (!path || !m)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null path or matrix");
  if (m->rows > kI32Max || m->columns > kI32Max || m->nnz > kI32Max)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "matrix dimensions and NNZ must fit in the i32 COO type");
  File file;
  file.f = std::fopen(path, "wb");
  if (!file.f)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not open %s", path);
  bool overflow = false;
  if (!write_all(file.f, kCooMagic, 8) ||
      !write_u64s(file.f, {(uint64_t)m->rows, (uint64_t)m->columns,
                           (uint64_t)m->nnz}) ||
      !write_as(file.f, m->row_indices, m->nnz) ||
      !write_as(file.f, m->column_indices, m->nnz) ||
      !write_f32(file.f, m->values, m->nnz, &overflow))
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    overflow ? "matrix values must fit in f32"
                             : "could not write %s",
                    path);
  return SW_OK;
}

static int csr_binary_read_impl(const char *path, sw_host_matrix **out) {
  sw::clear_error();
  if (!path || !out)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null path or output");
  *out = nullptr;
  File file;
  file.f = std::fopen(path, "rb");
  if (!file.f)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not open %s", path);
  uint64_t d[3];
  int rc = read_header(file.f, kCsrMagic, "CSR", d, 3);
  if (rc)
    return rc;
  if (d[0] >= (uint64_t)kI32Max || d[1] > (uint64_t)kI32Max ||
      d[2] > (uint64_t)kI32Max)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "CSR dimensions exceed the i32 index range");
  auto *m = static_cast<sw_host_matrix *>(std::calloc(1, sizeof(sw_host_matrix)));
  if (!m)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  m->rows = (int64_t)d[0];
  m->columns = (int64_t)d[1];
  m->nnz = (int64_t)d[2];
  if ((rc = read_array(file.f, d[0] + 1, "row offsets", &m->row_offsets)) ||
      (rc = read_array(file.f, d[2], "column indices", &m->column_indices)) ||
      (rc = read_f32_as_f64(file.f, d[2], "values", &m->values)) ||
      (rc = check_csr_structure(m->row_offsets, m->rows, m->column_indices,
                                m->nnz, m->columns, "CSR"))) {
    sw_host_matrix_free(m);
    return rc;
  }
  std::vector<int32_t> ri(m->nnz);
  for (int64_t r = 0; r < m->rows; ++r)
    for (int32_t p = m->row_offsets[r]; p < m->row_offsets[r + 1]; ++p)
      ri[p] = (int32_t)r;
  m->row_indices = dup_array(ri);
  m->has_row_offsets = 1;
  if (!m->row_indices) {
    sw_host_matrix_free(m);
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  }
  fill_stats(m);
  return (*out = m), SW_OK;
}

static int coo_binary_read_impl(const char *path, sw_host_matrix **out) {
  sw::clear_error();
  if (!path || !out)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null path or output");
  *out = nullptr;
  File file;
  file.f = std::fopen(path, "rb");
  if (!file.f)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not open %s", path);
  uint64_t d[3];
  int rc = read_header(file.f, kCooMagic, "COO", d, 3);
  if (rc)
    return rc;
  if (d[0] > (uint64_t)kI32Max || d[1] > (uint64_t)kI32Max ||
      d[2] > (uint64_t)kI32Max)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "COO dimensions exceed the i32 index range");
  int32_t *ri = nullptr, *ci = nullptr;
  double *val = nullptr;
  if ((rc = read_array(file.f, d[2], "row indices", &ri)) ||
      (rc = read_array(file.f, d[2], "column indices", &ci)) ||
      (rc = read_f32_as_f64(file.f, d[2], "values", &val))) {
    std::free(ri);
    std::free(ci);
    std::free(val);
    return rc;
  }
  // The arrays stay in file order (duplicates preserved).  When that order
  // is by (row, column) -- as the writer produces from a Matrix Market file
  // -- the row offsets are derived as well.
  auto *m = static_cast<sw_host_matrix *>(std::calloc(1, sizeof(sw_host_matrix)));
  if (!m) {
    std::free(ri);
    std::free(ci);
    std::free(val);
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  }
  m->rows = (int64_t)d[0];
  m->columns = (int64_t)d[1];
  m->nnz = (int64_t)d[2];
  m->row_indices = ri;
  m->column_indices = ci;
  m->values = val;
  bool sorted = true;
  for (uint64_t p = 0; p < d[2]; ++p) {
    if (ri[p] < 0 || (uint64_t)ri[p] >= d[0] || ci[p] < 0 ||
        (uint64_t)ci[p] >= d[1]) {
      sw_host_matrix_free(m);
      return sw::fail(SW_ERR_INVALID_SHAPE, "COO coordinate is out of bounds");
    }
    if (p && (ri[p] < ri[p - 1] || (ri[p] == ri[p - 1] && ci[p] < ci[p - 1])))
      sorted = false;
  }
  if (sorted) {
    std::vector<int32_t> ro(d[0] + 1, 0);
    for (uint64_t p = 0; p < d[2]; ++p)
      ++ro[ri[p] + 1];
    for (uint64_t r = 0; r < d[0]; ++r)
      ro[r + 1] += ro[r];
    m->row_offsets = dup_array(ro);
    if (!m->row_offsets) {
      sw_host_matrix_free(m);
      return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
    }
    m->has_row_offsets = 1;
  }
  fill_stats(m);
  *out = m;
  return SW_OK;
}

static int convert_to_bsr_impl(const sw_host_matrix *m, int64_t block_size,
                               sw_host_bsr **out) {
  sw::clear_error();
  if (!m || !out)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null matrix or output");
  *out = nullptr;
  if (block_size <= 0)
    return sw::fail(SW_ERR_INVALID_SHAPE, "BSR block size must be positive");
  const int64_t b = block_size;
  const int64_t prow = sw::ceil_div(m->rows, b) * b;
  const int64_t pcol = sw::ceil_div(m->columns, b) * b;
  const int64_t nbr = prow / b, nbc = pcol / b;
  // entries ordered by (block row, block column), storage order within a
  // block kept, so repeated coordinates add up in the order they are stored
  std::vector<int64_t> order(m->nnz);
  std::iota(order.begin(), order.end(), 0);
  auto key = [&](int64_t p) {
    return (int64_t)(m->row_indices[p] / b) * nbc + m->column_indices[p] / b;
  };
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t a, int64_t c) { return key(a) < key(c); });
  std::vector<int32_t> bro(nbr + 1, 0), bcol;
  std::vector<double> acc;
  int64_t last = -1;
  for (int64_t p : order) {
    const int64_t k = key(p);
    if (k != last) {
      bcol.push_back((int32_t)(k % nbc));
      ++bro[k / nbc + 1];
      acc.resize(acc.size() + (size_t)(b * b), 0.0);
      last = k;
    }
    const int64_t local =
        (m->row_indices[p] % b) * b + m->column_indices[p] % b;
    acc[acc.size() - (size_t)(b * b) + (size_t)local] += m->values[p];
  }
  for (int64_t r = 0; r < nbr; ++r)
    bro[r + 1] += bro[r];
  // distinct occupied coordinates
  std::vector<int64_t> coords(m->nnz);
  for (int64_t p = 0; p < m->nnz; ++p)
    coords[p] = (int64_t)m->row_indices[p] * m->columns + m->column_indices[p];
  std::sort(coords.begin(), coords.end());
  const int64_t occupied =
      (int64_t)(std::unique(coords.begin(), coords.end()) - coords.begin());

  auto *o = static_cast<sw_host_bsr *>(std::calloc(1, sizeof(sw_host_bsr)));
  if (!o)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  o->rows = prow;
  o->columns = pcol;
  o->original_rows = m->rows;
  o->original_columns = m->columns;
  o->nnz = m->nnz;
  o->block_size = b;
  o->nnzb = (int64_t)bcol.size();
  o->block_row_offsets = dup_array(bro);
  o->block_column_indices = dup_array(bcol);
  o->block_values = dup_array(acc);
  std::vector<int32_t> ri(m->row_indices, m->row_indices + m->nnz);
  std::vector<int32_t> ci(m->column_indices, m->column_indices + m->nnz);
  std::vector<double> iv(m->values, m->values + m->nnz);
  o->input_row_indices = dup_array(ri);
  o->input_column_indices = dup_array(ci);
  o->input_values = dup_array(iv);
  if (!o->block_row_offsets || !o->block_column_indices || !o->block_values ||
      !o->input_row_indices || !o->input_column_indices || !o->input_values) {
    sw_host_bsr_free(o);
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  }
  const double slots = (double)o->nnzb * (double)(b * b);
  o->block_density = (nbr && nbc) ? (double)o->nnzb / ((double)nbr * nbc) : 0;
  o->internal_zero_fraction = slots ? 1.0 - (double)occupied / slots : 0.0;
  o->storage_overhead = occupied ? slots / (double)occupied : 0.0;
  *out = o;
  return SW_OK;
}

static int bsr_binary_write_impl(const char *path, const sw_host_bsr *m) {
  sw::clear_error();
  if (!path || !m)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null path or matrix");
  if (m->rows > kI32Max || m->columns > kI32Max || m->nnzb > kI32Max ||
      m->original_rows > kI32Max || m->original_columns > kI32Max ||
      m->nnz > kI32Max)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "BSR dimensions and NNZ blocks must fit in i32");
  File file;
  file.f = std::fopen(path, "wb");
  if (!file.f)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not open %s", path);
  const int64_t bb = m->block_size * m->block_size;
  bool overflow = false;
  bool ok =
      write_all(file.f, kBsrMagic, 8) &&
      write_u64s(file.f, {(uint64_t)m->rows, (uint64_t)m->columns,
                          (uint64_t)m->nnzb, (uint64_t)m->block_size,
                          (uint64_t)m->original_rows,
                          (uint64_t)m->original_columns, (uint64_t)m->nnz}) &&
      write_as(file.f, m->block_row_offsets, m->rows / m->block_size + 1) &&
      write_as(file.f, m->block_column_indices, m->nnzb) &&
      write_f32(file.f, m->block_values, m->nnzb * bb, &overflow);
  if (!ok)
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    overflow ? "coalesced BSR values must fit in f32"
                             : "could not write %s",
                    path);
  ok = write_as(file.f, m->input_row_indices, m->nnz) &&
       write_as(file.f, m->input_column_indices, m->nnz) &&
       write_f32(file.f, m->input_values, m->nnz, &overflow);
  if (!ok)
    return sw::fail(SW_ERR_INVALID_ARGUMENT,
                    overflow ? "matrix values must fit in f32"
                             : "could not write %s",
                    path);
  return SW_OK;
}

static int bsr_binary_read_impl(const char *path, sw_host_bsr **out) {
  sw::clear_error();
  if (!path || !out)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "null path or output");
  *out = nullptr;
  File file;
  file.f = std::fopen(path, "rb");
  if (!file.f)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "could not open %s", path);
  uint64_t d[7];
  int rc = read_header(file.f, kBsrMagic, "BSR", d, 7);
  if (rc)
    return rc;
  const uint64_t rows = d[0], cols = d[1], nnzb = d[2], b = d[3];
  if (b == 0 || rows % b != 0 || cols % b != 0)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "BSR dimensions must be divisible by a positive block "
                    "size");
  if (d[4] > rows || d[5] > cols)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "original BSR dimensions exceed the padded dimensions");
  if (b > kI64Max || nnzb > kI64Max / b / b)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "BSR block values exceed the runner limits");
  if (rows > (uint64_t)kI32Max || cols > (uint64_t)kI32Max ||
      nnzb > (uint64_t)kI32Max || d[6] > (uint64_t)kI32Max)
    return sw::fail(SW_ERR_INVALID_SHAPE,
                    "BSR dimensions exceed the i32 index range");
  auto *o = static_cast<sw_host_bsr *>(std::calloc(1, sizeof(sw_host_bsr)));
  if (!o)
    return sw::fail(SW_ERR_INVALID_ARGUMENT, "out of host memory");
  o->rows = (int64_t)rows;
  o->columns = (int64_t)cols;
  o->nnzb = (int64_t)nnzb;
  o->block_size = (int64_t)b;
  o->original_rows = (int64_t)d[4];
  o->original_columns = (int64_t)d[5];
  o->nnz = (int64_t)d[6];
  if ((rc = read_array(file.f, rows / b + 1, "block-row offsets",
                       &o->block_row_offsets)) ||
      (rc = read_array(file.f, nnzb, "block-column indices",
                       &o->block_column_indices)) ||
      (rc = read_f32_as_f64(file.f, nnzb * b * b, "block values",
                            &o->block_values)) ||
      (rc = read_array(file.f, d[6], "input row indices",
                       &o->input_row_indices)) ||
      (rc = read_array(file.f, d[6], "input column indices",
                       &o->input_column_indices)) ||
      (rc = read_f32_as_f64(file.f, d[6], "input values", &o->input_values)) ||
      (rc = check_csr_structure(o->block_row_offsets, (int64_t)(rows / b),
                                o->block_column_indices, (int64_t)nnzb,
                                (int64_t)(cols / b), "BSR block"))) {
    sw_host_bsr_free(o);
    return rc;
  }
  for (int64_t p = 0; p < o->nnz; ++p)
    if (o->input_row_indices[p] < 0 ||
        o->input_row_indices[p] >= o->original_rows ||
        o->input_column_indices[p] < 0 ||
        o->input_column_indices[p] >= o->original_columns) {
      sw_host_bsr_free(o);
      return sw::fail(SW_ERR_INVALID_SHAPE,
                      "original BSR input coordinate is out of bounds");
    }
  const int64_t slots = o->nnzb * o->block_size * o->block_size;
  std::vector<int64_t> coords(o->nnz);
  for (int64_t p = 0; p < o->nnz; ++p)
    coords[p] = (int64_t)o->input_row_indices[p] * o->original_columns +
                o->input_column_indices[p];
  std::sort(coords.begin(), coords.end());
  const int64_t occupied =
      (int64_t)(std::unique(coords.begin(), coords.end()) - coords.begin());
  const int64_t nbr = o->rows / o->block_size, nbc = o->columns / o->block_size;
  o->block_density = (nbr && nbc) ? (double)o->nnzb / ((double)nbr * nbc) : 0;
  o->internal_zero_fraction = slots ? 1.0 - (double)occupied / slots : 0.0;
  o->storage_overhead = occupied ? (double)slots / occupied : 0.0;
  *out = o;
  return SW_OK;
}

int sw_matrix_market_read(const char *path, sw_host_matrix **out) {
  return guarded([&] { return matrix_market_read_impl(path, out); });
}

int sw_csr_binary_write(const char *path, const sw_host_matrix *m) {
  return guarded([&] { return csr_binary_write_impl(path, m); });
}

int sw_coo_binary_write(const char *path, const sw_host_matrix *m) {
  return guarded([&] { return coo_binary_write_impl(path, m); });
}

int sw_csr_binary_read(const char *path, sw_host_matrix **out) {
  return guarded([&] { return csr_binary_read_impl(path, out); });
}

int sw_coo_binary_read(const char *path, sw_host_matrix **out) {
  return guarded([&] { return coo_binary_read_impl(path, out); });
}

int sw_convert_to_bsr(const sw_host_matrix *m, int64_t block_size,
                      sw_host_bsr **out) {
  return guarded([&] { return convert_to_bsr_impl(m, block_size, out); });
}

int sw_bsr_binary_write(const char *path, const sw_host_bsr *m) {
  return guarded([&] { return bsr_binary_write_impl(path, m); });
}

int sw_bsr_binary_read(const char *path, sw_host_bsr **out) {
  return guarded([&] { return bsr_binary_read_impl(path, out); });
}

} // extern "C"
