// SafetensorsCheckpoint: a single file or a sharded directory as one tensor
// table sorted by name.
//
// Opening a sharded checkpoint: the index is read with the pull parser into
// a name-ordered weight map (a repeated name keeps its last shard, as a JSON
// object does); shards are numbered in the order the map first names them;
// each shard's header is read and its tensors are merged, as a sorted list,
// against the sorted list of names the index assigns to it.  A name only in
// the shard is either unknown to the index or indexed elsewhere; a name only
// in the index is missing from its shard (reported once every shard has been
// read); both sides agreeing gives a table row.
//
// Loading many tensors: the requests are resolved first, sorted by (shard,
// file offset) so each mapped file is read front to back, every needed shard
// is opened once and its records re-checked, and the whole batch, whatever
// its shards, goes through one staged upload; results return in request
// order.
//
// The checks, their order, exception types and messages are the contract of
// the reference's src/io/safetensors_checkpoint.cpp (constructor :137-172,
// index :22-132 and :174-318, load :356-376, load_many :378-422).
#include "qwen3/io/safetensors_checkpoint.h"

#include "json_cursor.hpp"
#include "staged_upload.hpp"

#include <algorithm>
#include <fstream>
#include <iterator>
#include <limits>
#include <map>
#include <numeric>
#include <optional>
#include <sstream>
#include <stdexcept>

namespace qwen3
{
    namespace
    {
        namespace fs = std::filesystem;
        using io_detail::JsonCursor;

        [[noreturn]] void fail(const std::string &message) { throw std::runtime_error(message); }

        // What model.safetensors.index.json says.
        struct Index
        {
            std::optional<std::size_t> total_size;   // empty: metadata or total_size missing / not unsigned
            bool has_metadata_object = false;
            bool total_too_large = false;
            bool has_weight_map_object = false;
            // tensor name -> shard name; nullopt: an entry whose value is not a string
            std::map<std::string, std::optional<std::string>> weight_map;
        };

        Index read_index(const fs::path &path)
        {
            std::ifstream in{path, std::ios::binary};
            if (!in)
                fail("cannot open checkpoint index: " + path.string());
            std::ostringstream text;
            text << in.rdbuf();
            const std::string body = text.str();
            Index idx;
            bool root_is_object = true;
            try
            {
                JsonCursor cur(body);
                if (cur.peek_kind() != JsonCursor::Kind::Object)
                {
                    root_is_object = false;
                    cur.skip_value();
                }
                else
                {
                    cur.open_object();
                    std::string key;
                    while (cur.next_key(key))
                    {
                        if (key == "metadata" && cur.peek_kind() == JsonCursor::Kind::Object)
                        {
                            idx.has_metadata_object = true;
                            idx.total_size.reset();
                            idx.total_too_large = false;
                            cur.open_object();
                            std::string field;
                            while (cur.next_key(field))
                            {
                                if (field != "total_size")
                                {
                                    cur.skip_value();
                                    continue;
                                }
                                idx.total_size.reset();
                                idx.total_too_large = false;
                                if (cur.peek_kind() != JsonCursor::Kind::Number)
                                {
                                    cur.skip_value();
                                    continue;
                                }
                                const JsonCursor::Number n = cur.read_number();
                                if (!n.is_unsigned)
                                    continue;
                                if (n.value > static_cast<std::uint64_t>(std::numeric_limits<std::size_t>::max()))
                                    idx.total_too_large = true;
                                else
                                    idx.total_size = static_cast<std::size_t>(n.value);
                            }
                        }
                        else if (key == "metadata")
                        {
                            idx.has_metadata_object = false;
                            idx.total_size.reset();
                            cur.skip_value();
                        }
                        else if (key == "weight_map" && cur.peek_kind() == JsonCursor::Kind::Object)
                        {
                            idx.has_weight_map_object = true;
                            idx.weight_map.clear();
                            cur.open_object();
                            std::string name;
                            while (cur.next_key(name))
                            {
                                if (cur.peek_kind() == JsonCursor::Kind::String)
                                {
                                    idx.weight_map.insert_or_assign(name, cur.read_string());
                                }
                                else
                                {
                                    idx.weight_map.insert_or_assign(name, std::nullopt);
                                    cur.skip_value();
                                }
                            }
                        }
                        else
                        {
                            if (key == "weight_map")
                            {
                                idx.has_weight_map_object = false;
                                idx.weight_map.clear();
                            }
                            cur.skip_value();
                        }
                    }
                }
                // nothing after the root value is read: the reference reads the
                // index with nlohmann's stream operator, which stops at the end
                // of the first value (safetensors_checkpoint.cpp:36)
            }
            catch (const std::runtime_error &e)
            {
                fail("invalid checkpoint index '" + path.string() + "': " + e.what());
            }
            if (!root_is_object)
                fail("checkpoint index root must be an object");
            return idx;
        }

        // A shard named by the index: a plain file name ending in
        // .safetensors, present in the model directory.
        fs::path shard_path(const fs::path &dir, const std::string &name)
        {
            const bool plain = !name.empty() && name.find('/') == std::string::npos &&
                               name.find('\\') == std::string::npos;
            const fs::path rel{name};
            if (!plain || rel.is_absolute() || rel.has_parent_path() || rel.extension() != ".safetensors")
                fail("invalid checkpoint shard name: " + name);
            fs::path full = dir / rel;
            if (!fs::is_regular_file(full))
                fail("checkpoint shard does not exist: " + full.string());
            return full;
        }

        bool same_record(const SafetensorsTensorInfo &a, const SafetensorsTensorInfo &b)
        {
            return a.dtype == b.dtype && a.shape == b.shape && a.begin_offset == b.begin_offset &&
                   a.end_offset == b.end_offset;
        }

        // The records of one shard, sorted by name.
        std::vector<std::pair<std::string, SafetensorsTensorInfo>> sorted_records(const fs::path &file)
        {
            const SafetensorsFile f(file);
            const SafetensorsMetadata md(f);
            std::vector<std::pair<std::string, SafetensorsTensorInfo>> out(md.tensors().begin(), md.tensors().end());
            std::sort(out.begin(), out.end(), [](const auto &a, const auto &b) { return a.first < b.first; });
            return out;
        }
    } // namespace

    SafetensorsCheckpoint::SafetensorsCheckpoint(const std::filesystem::path &model_directory)
        : model_directory_{fs::absolute(model_directory)}
    {
        if (!fs::is_directory(model_directory_))
            throw std::invalid_argument("model directory does not exist: " + model_directory_.string());
        const fs::path single = model_directory_ / "model.safetensors";
        const fs::path index = model_directory_ / "model.safetensors.index.json";
        const bool has_single = fs::is_regular_file(single), has_index = fs::is_regular_file(index);
        if (has_single && has_index)
            fail("model directory contains both model.safetensors and model.safetensors.index.json");
        if (!has_single && !has_index)
            fail("model directory contains neither model.safetensors ans model.safetensor.index.json");

        if (has_single)
        {
            shard_files_.push_back(single);
            for (auto &[name, info] : sorted_records(single))
                table_.push_back(Entry{name, 0, info});
            if (table_.empty())
                fail("single-file checkpoint contains no tensors");
            return;
        }

        const Index idx = read_index(index);
        if (!idx.has_metadata_object)
            fail("checkpoint index must contain a metadata object");
        if (idx.total_too_large)
            fail("checkpoint total_size is too large");
        if (!idx.total_size)
            fail("checkpoint metadata.total_size must be an unsigned integer");
        if (!idx.has_weight_map_object || idx.weight_map.empty())
            fail("checkpoint index weight_map must be a non-empty object");

        // shard numbers in first-mention order; per shard, the names the index gives it (sorted)
        std::map<std::string, std::size_t> shard_of_name;
        std::vector<std::vector<const std::string *>> indexed;
        std::vector<std::size_t> shard_of_entry;  // parallel to weight_map order
        for (const auto &[tensor, shard] : idx.weight_map)
        {
            if (tensor.empty() || !shard)
                fail("checkpoint weight_map contains an valid entry");
            auto found = shard_of_name.find(*shard);
            if (found == shard_of_name.end())
            {
                shard_files_.push_back(shard_path(model_directory_, *shard));
                found = shard_of_name.emplace(*shard, shard_files_.size() - 1).first;
                indexed.emplace_back();
            }
            indexed[found->second].push_back(&tensor);
            shard_of_entry.push_back(found->second);
        }

        const auto indexed_shard = [&](const std::string &name) -> std::optional<std::size_t> {
            const auto it = idx.weight_map.find(name);
            if (it == idx.weight_map.end())
                return std::nullopt;
            return shard_of_entry[static_cast<std::size_t>(std::distance(idx.weight_map.begin(), it))];
        };

        std::size_t bytes = 0;
        std::vector<std::string> missing;
        for (std::size_t s = 0; s < shard_files_.size(); ++s)
        {
            const auto records = sorted_records(shard_files_[s]);
            const auto &want = indexed[s];   // sorted: weight_map iterates in name order
            std::size_t a = 0, b = 0;
            while (a < records.size() || b < want.size())
            {
                if (b == want.size() || (a < records.size() && records[a].first < *want[b]))
                {
                    // in the shard, not indexed here
                    const std::string &name = records[a].first;
                    if (records[a].second.size_bytes() > std::numeric_limits<std::size_t>::max() - bytes)
                        throw std::overflow_error("checkpoint tensor byte count overflow");
                    bytes += records[a].second.size_bytes();
                    if (!indexed_shard(name))
                        fail("tensor '" + name + "' exists in a shard but not in the checkpoint index");
                    fail("tensor '" + name + "' is stored in the wrong shard");
                }
                if (a == records.size() || *want[b] < records[a].first)
                {
                    missing.push_back(*want[b++]);   // indexed here, not in the shard
                    continue;
                }
                const SafetensorsTensorInfo &info = records[a].second;
                if (info.size_bytes() > std::numeric_limits<std::size_t>::max() - bytes)
                    throw std::overflow_error("checkpoint tensor byte count overflow");
                bytes += info.size_bytes();
                table_.push_back(Entry{records[a].first, s, info});
                ++a;
                ++b;
            }
        }
        if (!missing.empty())
            fail("indexed tensor is missing from its shard: " + *std::min_element(missing.begin(), missing.end()));
        if (bytes != *idx.total_size)
            fail("checkpoint total_size mismatch: expected" + std::to_string(*idx.total_size) + ", got" +
                 std::to_string(bytes));
        std::sort(table_.begin(), table_.end(), [](const Entry &x, const Entry &y) { return x.name < y.name; });
        for (std::size_t i = 1; i < table_.size(); ++i)
            if (table_[i].name == table_[i - 1].name)
                fail("tensor appears in multiple shards: " + table_[i].name);
        sharded_ = true;
    }

    const SafetensorsCheckpoint::Entry *SafetensorsCheckpoint::find(std::string_view name) const
    {
        const auto it = std::lower_bound(table_.begin(), table_.end(), name,
                                         [](const Entry &e, std::string_view n) { return e.name < n; });
        return it != table_.end() && it->name == name ? &*it : nullptr;
    }

    const SafetensorsCheckpoint::Entry &SafetensorsCheckpoint::find_or_throw(std::string_view name) const
    {
        const Entry *e = find(name);
        if (e == nullptr)
            throw std::out_of_range("checkpoint tensor not found: " + std::string(name));
        return *e;
    }

    bool SafetensorsCheckpoint::contains(std::string_view name) const { return find(name) != nullptr; }

    const SafetensorsTensorInfo &SafetensorsCheckpoint::tensor_info(std::string_view name) const
    {
        return find_or_throw(name).info;
    }

    Tensor SafetensorsCheckpoint::load(std::string_view name, Device target_device) const
    {
        const Entry &e = find_or_throw(name);
        const SafetensorsFile file(shard_files_.at(e.shard));
        const SafetensorsMetadata now(file);
        if (!now.contains(name) || !same_record(now.tensor(name), e.info))
            fail("checkpoint changed while loading tensor: " + std::string(name));
        return io_detail::copy_out(file, e.info, target_device, name);
    }

    std::vector<Tensor> SafetensorsCheckpoint::load_many(const std::vector<std::string> &names,
                                                         Device target_device) const
    {
        std::vector<const Entry *> want;
        want.reserve(names.size());
        for (const std::string &n : names)
            want.push_back(&find_or_throw(n));
        // read order: by shard, then by position in the file
        std::vector<std::size_t> order(names.size());
        std::iota(order.begin(), order.end(), std::size_t{0});
        std::stable_sort(order.begin(), order.end(), [&](std::size_t x, std::size_t y) {
            if (want[x]->shard != want[y]->shard)
                return want[x]->shard < want[y]->shard;
            return want[x]->info.begin_offset < want[y]->info.begin_offset;
        });
        // each needed shard opened once, its records checked against the table
        std::map<std::size_t, SafetensorsFile> files;
        for (const std::size_t i : order)
        {
            const Entry &e = *want[i];
            auto it = files.find(e.shard);
            if (it == files.end())
                it = files.emplace(e.shard, SafetensorsFile(shard_files_.at(e.shard))).first;
        }
        for (auto &[shard, file] : files)
        {
            const SafetensorsMetadata now(file);
            for (const Entry *e : want)
                if (e->shard == shard && (!now.contains(e->name) || !same_record(now.tensor(e->name), e->info)))
                    fail("checkpoint changed while loading tensor: " + e->name);
        }

        std::vector<std::optional<Tensor>> slots(names.size());
        if (target_device.is_cpu())
        {
            for (const std::size_t i : order)
                slots[i].emplace(io_detail::copy_out(files.at(want[i]->shard), want[i]->info, target_device, names[i]));
        }
        else
        {
            std::size_t total = 0;
            for (const Entry *e : want)
                total += e->info.size_bytes();
            io_detail::StagedUpload upload(target_device.index());
            upload.run(order.size(), total, [&](std::size_t k) {
                const std::size_t i = order[k];
                const SafetensorsTensorInfo &info = want[i]->info;
                Tensor &t = slots[i].emplace(Tensor::empty(info.shape, info.dtype, target_device));
                if (t.nbytes() != info.size_bytes())
                    throw std::logic_error("Tensor size does not match metadata for '" + names[i] + "'");
                const std::byte *src = files.at(want[i]->shard).data_bytes().data() + info.begin_offset;
                return io_detail::UploadPiece{src, t.data(), info.size_bytes()};
            });
        }
        std::vector<Tensor> out;
        out.reserve(slots.size());
        for (auto &s : slots)
            out.push_back(std::move(*s));
        return out;
    }
} // namespace qwen3
