# affine_lsq(loss, w, x, b, t, r, i_m, i_n)
#
# Least-squares loss of an affine map: loss += 0.5 * sum((w * x + b - t) .^ 2).
#
# One iteration per row; the row sum is a value carried over the column loop
# (rule 1), so the column loop stays sequential inside the row.
#
# loss: length-1 output array, accumulated in place
# w: matrix of shape (i_m, i_n), column-major
# x: input vector of length i_n
# b: bias vector of length i_m
# t: target vector of length i_m
# r: residual vector of length i_m, overwritten
# i_m: number of rows of w
# i_n: number of columns of w
function affine_lsq(loss, w, x, b, t, r, i_m, i_n)
    # residual of each row
    for i_i = 1:i_m
        s = b[i_i] - t[i_i]
        for i_j = 1:i_n
            s = s + w[i_i, i_j] * x[i_j]
        end
        r[i_i] = s
    end
    # half the squared norm of the residual
    for i_i2 = 1:i_m
        loss[1] = loss[1] + 0.5 * r[i_i2] ^ 2
    end
    return nothing
end
