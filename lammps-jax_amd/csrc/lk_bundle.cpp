// Model bundles for `pair_coeff * * bundle.json`: the contract the pair style checks and the model
// section this library runs (host code, no device work).
//
// Reference interface: lammps_jax::load_bundle_file (cpp/lammps_jax_model.cpp:212-315). The
// bundle is the exporter's JSON with sorted keys, read by first-match key lookup: "contract"
// sorts before every other section, so a key's first occurrence is the contract's. The contract
// keys, their defaults for older bundles and the validation messages are the reference's. The
// reference's bundles carry StableHLO programs for PJRT; a bundle for this library carries a
// "model" section instead, whose keys are prefixed so that they never collide with the
// contract's under first-match lookup:
//   "model_kind": "eam/alloy" with "eam_setfl" (a DYNAMO setfl file, path relative to the bundle,
//                 optionally gzipped), or "lj/cut" with "lj_epsilon", "lj_sigma", "lj_cutoff"
//                 and "lj_edge_energy_scale"; optional "model_accumulation":
//                 "plain" | "half" | "onesided".
// The setfl tables become PairEAM::interpolate coefficients (eam.py:115-135, 174-227).

#include <zlib.h>

#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/lk_hip.h"

struct lk_bundle {
  std::string format;
  std::string unit_style;
  // contract (lammps_jax_model.h:43-76)
  std::string input_layout, precision, force_output, newton, edge_pairing;
  int max_atoms = 0, max_edges = 0, max_neighbors = 0, n_hops = 1, n_species = 0, max_owned = 0;
  double cutoff = 0.0;
  bool uses_box = false, pair_sum = false, half_edges = false;
  std::vector<int> comm_widths;
  // model section
  int kind = 0;  // 1 eam/alloy, 2 lj/cut
  int accumulation = -1;
  int n_el = 0, nrho = 0, nr = 0;
  double drho = 0, dr = 0, eam_cutoff = 0;
  std::vector<double> emb, dens, pair;  // [n_el][nrho][4], [n_el][nr][4], [npair][nr][4]
  std::vector<std::string> elements;
  std::vector<double> masses;
  lk_lj_params lj{};
};

namespace {

std::string read_text(const std::string &path, const char *what)
{
  gzFile g = gzopen(path.c_str(), "rb");  // plain files read through unchanged
  if (!g) throw std::runtime_error(std::string("Could not open ") + what + ": " + path);
  std::string out;
  char buf[1 << 16];
  for (;;) {
    const int n = gzread(g, buf, sizeof(buf));
    if (n < 0) {
      gzclose(g);
      throw std::runtime_error("Could not read " + path);
    }
    if (n == 0) break;
    out.append(buf, static_cast<size_t>(n));
  }
  gzclose(g);
  return out;
}

// Position just past "key": (first occurrence).
size_t value_pos(const std::string &json, const std::string &key)
{
  const std::string quoted = "\"" + key + "\"";
  const size_t at = json.find(quoted);
  if (at == std::string::npos) throw std::runtime_error("Missing key in bundle: " + key);
  size_t pos = json.find(':', at + quoted.size());
  if (pos == std::string::npos) throw std::runtime_error("Malformed key in bundle: " + key);
  ++pos;
  while (pos < json.size() && std::isspace(static_cast<unsigned char>(json[pos]))) ++pos;
  return pos;
}

bool has_key(const std::string &json, const std::string &key)
{
  return json.find("\"" + key + "\"") != std::string::npos;
}

std::string str(const std::string &json, const std::string &key)
{
  size_t pos = value_pos(json, key);
  if (pos >= json.size() || json[pos] != '"') throw std::runtime_error("Expected JSON string");
  std::string out;
  for (++pos; pos < json.size(); ++pos) {
    const char c = json[pos];
    if (c == '"') return out;
    if (c != '\\') {
      out.push_back(c);
      continue;
    }
    if (++pos >= json.size()) break;
    const char e = json[pos];
    const char *plain = "\"\\/";
    if (std::strchr(plain, e)) out.push_back(e);
    else if (e == 'n') out.push_back('\n');
    else if (e == 't') out.push_back('\t');
    else if (e == 'r') out.push_back('\r');
    else if (e == 'b') out.push_back('\b');
    else if (e == 'f') out.push_back('\f');
    else throw std::runtime_error("Unsupported JSON escape in model bundle");
  }
  throw std::runtime_error("Unterminated JSON string");
}

double num(const std::string &json, const std::string &key)
{
  const size_t pos = value_pos(json, key);
  const size_t end = json.find_first_of(",}]\n\r\t ", pos);
  return std::stod(json.substr(pos, end - pos));
}

int int_or(const std::string &json, const std::string &key, int fallback)
{
  return has_key(json, key) ? static_cast<int>(num(json, key)) : fallback;
}

bool boolean(const std::string &json, const std::string &key)
{
  const size_t pos = value_pos(json, key);
  if (json.compare(pos, 4, "true") == 0) return true;
  if (json.compare(pos, 5, "false") == 0) return false;
  throw std::runtime_error("Expected boolean for key: " + key);
}

bool bool_or(const std::string &json, const std::string &key, bool fallback)
{
  return has_key(json, key) ? boolean(json, key) : fallback;
}

std::vector<int> ints_or(const std::string &json, const std::string &key)
{
  std::vector<int> out;
  if (!has_key(json, key)) return out;
  size_t pos = value_pos(json, key);
  if (pos >= json.size() || json[pos] != '[')
    throw std::runtime_error("Expected JSON array for key: " + key);
  ++pos;
  for (;;) {
    while (pos < json.size() && std::isspace(static_cast<unsigned char>(json[pos]))) ++pos;
    if (pos >= json.size()) throw std::runtime_error("Unterminated JSON array for key: " + key);
    if (json[pos] == ']') return out;
    const size_t end = json.find_first_of(",]", pos);
    if (end == std::string::npos) throw std::runtime_error("Unterminated JSON array for key: " + key);
    out.push_back(std::stoi(json.substr(pos, end - pos)));
    pos = json[end] == ',' ? end + 1 : end;
  }
}

// PairEAM::interpolate (eam.py:115-135): 5-point interior slopes, one-sided ends, the last row
// c2 = c3 = 0. Built with -ffp-contract=off: every product is rounded before its sum, as in the
// numpy restatement, so the coefficients agree bit for bit.
void interpolate(const double *f, int n, double *coef)
{
  std::vector<double> d(static_cast<size_t>(n));
  d[0] = f[1] - f[0];
  d[1] = 0.5 * (f[2] - f[0]);
  d[n - 2] = 0.5 * (f[n - 1] - f[n - 3]);
  d[n - 1] = f[n - 1] - f[n - 2];
  for (int m = 2; m < n - 2; ++m) d[m] = ((f[m - 2] - f[m + 2]) + 8.0 * (f[m + 1] - f[m - 1])) / 12.0;
  for (int m = 0; m < n; ++m) {
    double *c = coef + 4L * m;
    c[0] = f[m];
    c[1] = d[m];
    c[2] = 0.0;
    c[3] = 0.0;
    if (m + 1 < n) {
      const double step = f[m + 1] - f[m];
      c[2] = 3.0 * step - 2.0 * d[m] - d[m + 1];
      c[3] = d[m] + d[m + 1] - 2.0 * step;
    }
  }
}

// DYNAMO setfl (eam.py:174-227): 3 comment lines, then whitespace-separated tokens: element
// count and names, the grid (nrho drho nr dr cutoff), per element a 4-token header (Z, mass,
// lattice constant, lattice) with F(rho) and rho(r), then r*phi for pairs (i, j <= i). `path`
// names the source in messages.
void parse_setfl(lk_bundle &b, const std::string &text, const std::string &path)
{
  size_t pos = 0;
  for (int line = 0; line < 3; ++line) {
    pos = text.find('\n', pos);
    if (pos == std::string::npos) throw std::runtime_error(path + ": truncated setfl header");
    ++pos;
  }
  std::istringstream in(text.substr(pos));
  std::vector<std::string> tok;
  for (std::string t; in >> t;) tok.push_back(std::move(t));
  size_t k = 0;
  auto need = [&](size_t n) {
    if (k + n > tok.size()) throw std::runtime_error(path + ": truncated setfl tables");
  };
  need(1);
  b.n_el = std::stoi(tok[k++]);
  if (b.n_el < 1) throw std::runtime_error(path + ": invalid element count");
  need(static_cast<size_t>(b.n_el) + 5);
  for (int e = 0; e < b.n_el; ++e) b.elements.push_back(tok[k++]);
  b.nrho = std::stoi(tok[k++]);
  b.drho = std::stod(tok[k++]);
  b.nr = std::stoi(tok[k++]);
  b.dr = std::stod(tok[k++]);
  b.eam_cutoff = std::stod(tok[k++]);
  if (b.nrho < 5 || b.nr < 5) throw std::runtime_error(path + ": tables need at least 5 nodes");
  const int npair = b.n_el * (b.n_el + 1) / 2;
  b.emb.assign(static_cast<size_t>(b.n_el) * b.nrho * 4, 0.0);
  b.dens.assign(static_cast<size_t>(b.n_el) * b.nr * 4, 0.0);
  b.pair.assign(static_cast<size_t>(npair) * b.nr * 4, 0.0);
  std::vector<double> v;
  auto values = [&](int n) {
    need(static_cast<size_t>(n));
    v.resize(static_cast<size_t>(n));
    for (int q = 0; q < n; ++q) v[q] = std::stod(tok[k++]);
  };
  for (int e = 0; e < b.n_el; ++e) {
    need(4);
    b.masses.push_back(std::stod(tok[k + 1]));
    k += 4;
    values(b.nrho);
    interpolate(v.data(), b.nrho, &b.emb[static_cast<size_t>(e) * b.nrho * 4]);
    values(b.nr);
    interpolate(v.data(), b.nr, &b.dens[static_cast<size_t>(e) * b.nr * 4]);
  }
  for (int p = 0; p < npair; ++p) {
    values(b.nr);
    interpolate(v.data(), b.nr, &b.pair[static_cast<size_t>(p) * b.nr * 4]);
  }
  if (k != tok.size())
    throw std::runtime_error(path + ": " + std::to_string(tok.size() - k) +
                             " unparsed trailing values");
}

void load_setfl(lk_bundle &b, const std::string &path)
{
  parse_setfl(b, read_text(path, "setfl file"), path);
}

std::string dir_of(const std::string &path)
{
  const size_t slash = path.find_last_of('/');
  return slash == std::string::npos ? std::string() : path.substr(0, slash + 1);
}

// The reference's contract checks in its order (cpp/lammps_jax_model.cpp:245-313), for the
// sparse-edge layout this library runs.
void parse(lk_bundle &b, const std::string &json, const std::string &path)
{
  b.format = str(json, "format");
  b.input_layout = str(json, "input_layout");
  if (b.input_layout != "sparse-edge" && b.input_layout != "neighbor-matrix")
    throw std::runtime_error("Unsupported LAMMPS-JAX input layout '" + b.input_layout +
                             "'; re-export the bundle with the current lammps_jax exporter");
  b.max_atoms = static_cast<int>(num(json, "max_atoms"));
  b.max_edges = int_or(json, "max_edges", 0);
  b.max_neighbors = int_or(json, "max_neighbors", 0);
  b.cutoff = num(json, "cutoff");
  b.unit_style = str(json, "unit_style");
  b.precision = str(json, "precision");
  if (b.precision != "float32" && b.precision != "float64")
    throw std::runtime_error("Unsupported LAMMPS-JAX precision '" + b.precision +
                             "'; expected float32 or float64");
  b.force_output = str(json, "force_output");
  if (b.force_output != "atom-force" && b.force_output != "edge-force")
    throw std::runtime_error("Unsupported LAMMPS-JAX force output layout '" + b.force_output + "'");
  b.newton = str(json, "newton");
  if (b.newton != "any" && b.newton != "on" && b.newton != "off")
    throw std::runtime_error("Unsupported LAMMPS-JAX newton mode '" + b.newton + "'");
  b.n_hops = int_or(json, "n_hops", 1);
  b.comm_widths = ints_or(json, "comm_widths");
  b.uses_box = boolean(json, "uses_box");
  b.pair_sum = bool_or(json, "pair_sum", false);
  b.n_species = int_or(json, "n_species", 0);
  if (b.n_species < 0) throw std::runtime_error("Invalid n_species in bundle");
  b.max_owned = int_or(json, "max_owned", 0);
  if (b.max_owned < 0 || b.max_owned > b.max_atoms) throw std::runtime_error("Invalid max_owned in bundle");

  if (b.format != "lammps-jax-json" && b.format != "lammps-jax-json-distributed" &&
      b.format != "lammps-jax-json-half-edge" && b.format != "lammps-jax-hip-json")
    throw std::runtime_error("Unsupported bundle format");
  const bool comm = !b.comm_widths.empty();
  // The half-edge tag requires edge_pairing; this library's tag defaults it to full pairing.
  // Other tags pair fully whatever the key says.
  b.edge_pairing = "full";
  if (b.format == "lammps-jax-json-half-edge" || b.format == "lammps-jax-hip-json") {
    if (b.format == "lammps-jax-json-half-edge" || has_key(json, "edge_pairing"))
      b.edge_pairing = str(json, "edge_pairing");
    if (b.edge_pairing == "half") {
      if (comm)
        throw std::runtime_error(
            "Communicating half-edge bundles now pack each boundary pair on one rank; re-export "
            "this bundle");
      b.half_edges = true;
    } else if (b.edge_pairing == "half-unique") {
      if (!comm)
        throw std::runtime_error(
            "Unique-boundary bundles need a communication schedule; the partner rank's density "
            "share arrives through reverse comm");
      b.half_edges = true;
    } else if (b.edge_pairing != "full") {
      throw std::runtime_error("Invalid edge_pairing in bundle");
    }
  }
  if (b.half_edges && b.n_hops == 1 && !comm)
    throw std::runtime_error(
        "Half-edge bundles require n_hops > 1 or a communication schedule; the single-hop packer "
        "does not deduplicate edge directions");
  const bool matrix = b.input_layout == "neighbor-matrix";
  if (b.max_atoms <= 0 || (matrix ? b.max_neighbors : b.max_edges) <= 0)
    throw std::runtime_error("Invalid fixed capacities in bundle");
  if (matrix && b.force_output == "edge-force")
    throw std::runtime_error(
        "Neighbor-matrix bundles return per-atom forces; edge-force output needs sparse edges");
  if (b.max_owned > 0 && !comm && !(matrix && b.n_hops == 1))
    throw std::runtime_error(
        "max_owned needs a communicating or single-hop neighbor-matrix bundle; other layouts hold "
        "ghost rows past the owned ones");
  if (matrix && b.half_edges && !comm)
    throw std::runtime_error(
        "Neighbor-matrix half pairing needs a communication schedule; the pair style hands the "
        "model the LAMMPS half list as is");
  if (b.n_hops < 1) throw std::runtime_error("Invalid n_hops in bundle");
  if (b.n_hops > 1 && (b.newton != "on" || b.force_output != "atom-force"))
    throw std::runtime_error(
        "Bundles with n_hops > 1 require newton on and atom-force output; ghost force rows must "
        "flow back through the LAMMPS reverse communication");
  for (const int w : b.comm_widths)
    if (w <= 0) throw std::runtime_error("Invalid communication width in bundle");
  if (comm && b.n_hops != 1)
    throw std::runtime_error("Communicating bundles require a one-cutoff ghost shell (n_hops = 1)");
  if (comm && b.newton != "on" && (b.half_edges || b.force_output != "atom-force"))
    throw std::runtime_error(
        "Communicating bundles require newton on unless they pair fully and return atom forces; "
        "ghost force rows flow back through the LAMMPS reverse communication");
  if (comm && b.force_output == "edge-force" && !b.half_edges)
    throw std::runtime_error(
        "Communicating edge-force bundles require half-edge packing; full pairing packs both "
        "directions and the newton scatter doubles forces");

  // model section of this library's bundles
  if (!has_key(json, "model_kind")) return;
  const std::string kind = str(json, "model_kind");
  if (has_key(json, "model_accumulation")) {
    const std::string acc = str(json, "model_accumulation");
    if (acc == "plain") b.accumulation = LK_ACCUM_PLAIN;
    else if (acc == "half") b.accumulation = LK_ACCUM_HALF;
    else if (acc == "onesided") b.accumulation = LK_ACCUM_ONESIDED;
    else throw std::runtime_error("Invalid model_accumulation in bundle: " + acc);
  }
  if (kind == "eam/alloy") {
    std::string setfl = str(json, "eam_setfl");
    if (!setfl.empty() && setfl[0] != '/') setfl = dir_of(path) + setfl;
    load_setfl(b, setfl);
    if (b.n_species > 0 && b.n_species != b.n_el)
      throw std::runtime_error("Bundle n_species does not match the setfl element count");
    b.kind = 1;
  } else if (kind == "lj/cut") {
    b.lj.epsilon = num(json, "lj_epsilon");
    b.lj.sigma = num(json, "lj_sigma");
    b.lj.cutoff = num(json, "lj_cutoff");
    b.lj.edge_energy_scale = has_key(json, "lj_edge_energy_scale")
                                 ? num(json, "lj_edge_energy_scale")
                                 : 0.5;
    b.kind = 2;
  } else {
    throw std::runtime_error("Unsupported model_kind in bundle: " + kind);
  }
}

void set_error(char *err, int errlen, const std::string &msg)
{
  if (!err || errlen <= 0) return;
  std::snprintf(err, static_cast<size_t>(errlen), "%s", msg.c_str());
}

}  // namespace

extern "C" {

int lk_bundle_load(const char *path, lk_bundle **out, char *err, int errlen)
{
  if (!out || !path) {
    set_error(err, errlen, "invalid bundle arguments");
    return LK_ERR_ARGUMENT;
  }
  *out = nullptr;
  auto *b = new lk_bundle();
  try {
    const std::string json = read_text(path, "model bundle");
    parse(*b, json, path);
  } catch (const std::exception &e) {
    set_error(err, errlen, e.what());
    delete b;
    return LK_ERR_ARGUMENT;
  }
  *out = b;
  return LK_OK;
}

void lk_bundle_free(lk_bundle *b) { delete b; }

int lk_bundle_contract(const lk_bundle *b, int newton_pair, lk_contract *out)
{
  if (!b || !out) return LK_ERR_ARGUMENT;
  lk_contract c{};
  c.max_atoms = b->max_atoms;
  c.max_edges = b->max_edges;
  c.n_species = b->n_species;
  c.precision = b->precision == "float64" ? LK_FLOAT64 : LK_FLOAT32;
  c.newton = b->newton == "on" ? LK_NEWTON_ON : (b->newton == "off" ? LK_NEWTON_OFF : LK_NEWTON_ANY);
  const bool comm = !b->comm_widths.empty();
  c.pairing = !b->half_edges ? LK_PAIRING_FULL
                             : (b->edge_pairing == "half-unique" ? LK_PAIRING_HALF_UNIQUE
                                                                 : LK_PAIRING_HALF);
  c.n_hops = b->n_hops;
  c.pair_sum = b->pair_sum ? 1 : 0;
  c.comm = comm ? 1 : 0;
  c.edge_force = b->force_output == "edge-force" ? 1 : 0;
  c.newton_pair = newton_pair ? 1 : 0;
  // PairJaxKokkos::half_list (cpp/pair_jax_kokkos.cpp:425-431): bundles that need one direction
  // per pair take the LAMMPS half list.
  const bool matrix = b->input_layout == "neighbor-matrix";
  if (!newton_pair) c.half_list = 0;
  else if (comm) c.half_list = b->half_edges ? 1 : 0;
  else if (matrix) c.half_list = 0;
  else c.half_list = b->n_hops == 1 && (c.edge_force || b->pair_sum) ? 1 : 0;
  c.cutoff = b->cutoff;
  c.input_layout = matrix ? LK_LAYOUT_NEIGHBOR_MATRIX : LK_LAYOUT_SPARSE_EDGE;
  c.max_neighbors = b->max_neighbors;
  c.max_owned = b->max_owned;
  *out = c;
  return LK_OK;
}

int lk_bundle_model(const lk_bundle *b, int *kind, lk_eam_tables *eam, lk_lj_params *lj,
                    int *accumulation)
{
  if (!b) return LK_ERR_ARGUMENT;
  if (kind) *kind = b->kind;
  if (accumulation) *accumulation = b->accumulation;
  if (b->kind == 0) return LK_ERR_UNSUPPORTED;  // a PJRT bundle: no model section to run here
  if (b->kind == 1 && eam) {
    eam->n_el = b->n_el;
    eam->nrho = b->nrho;
    eam->nr = b->nr;
    eam->drho = b->drho;
    eam->dr = b->dr;
    eam->cutoff = b->eam_cutoff;
    eam->embedding = b->emb.data();
    eam->density = b->dens.data();
    eam->pair = b->pair.data();
  }
  if (b->kind == 2 && lj) *lj = b->lj;
  return LK_OK;
}

const char *lk_bundle_unit_style(const lk_bundle *b) { return b ? b->unit_style.c_str() : ""; }

int lk_setfl_parse(const char *text, long len, const char *source, lk_bundle **out, char *err,
                   int errlen)
{
  if (!out || !text || len < 0) {
    set_error(err, errlen, "invalid setfl arguments");
    return LK_ERR_ARGUMENT;
  }
  *out = nullptr;
  auto *b = new lk_bundle();
  b->kind = 1;
  try {
    parse_setfl(*b, std::string(text, static_cast<size_t>(len)), source ? source : "setfl");
  } catch (const std::exception &e) {
    set_error(err, errlen, e.what());
    delete b;
    return LK_ERR_ARGUMENT;
  }
  *out = b;
  return LK_OK;
}

int lk_bundle_element(const lk_bundle *b, int index, char *name, int name_len, double *mass)
{
  if (!b || b->kind != 1 || index < 0 || index >= static_cast<int>(b->elements.size()))
    return LK_ERR_ARGUMENT;
  if (name && name_len > 0)
    std::snprintf(name, static_cast<size_t>(name_len), "%s", b->elements[index].c_str());
  if (mass) *mass = b->masses[static_cast<size_t>(index)];
  return LK_OK;
}

}  // extern "C"
